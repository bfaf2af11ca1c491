"""W4A4 INT4 GEMM ops for MI355X (gfx950) as torch custom ops (torch.compile friendly).

Mirrors the reference op surface of ``pi05_fast/w4a4/extension.py`` (lines 15-178):
the ``torch.ops.pi05_w4a4.{int4_gemm, int4_gemm_tiled, int4_gemm2, int4_gemm2_tiled,
int4_gemm3}`` custom ops with shape-only fake implementations, the Python wrappers of
the same names, ``load_int4_gemm()`` and ``preload()``.  The op bodies call the
hipcc-built C-ABI library ``_lib/libpi05_w4a4.so`` (``include/pi05_w4a4.h``) through
ctypes, on the current torch stream, with torch-allocated outputs and temporaries.

Validation and error messages follow the reference's TORCH_CHECKs
(``pi05_fast/w4a4/csrc/int4_gemm.cu:487-501, 570-577``); they surface as RuntimeError.

Weight layouts accepted (the reference's marker-stride convention):
  * row-major ``[N, K/8+1]`` (L1) or row-padded ``[N, K/8+P]`` (L2) -- repacked into an
    MFMA-layout copy on the first call with that tensor, which later calls reuse (kept
    for drop-in use; the copy doubles the weight's device memory);
  * WMMA-tiled ``[N, K/8+9]`` (L3) -- ``*_tiled`` ops, repacked once likewise;
  * MFMA-fragment-major ``[N, K/8+16]`` -- produced once by ``repack_weight`` (and by
    ``apply.replace_linears_from_packed`` at load), consumed directly (fast path);
  * E3M2 column pairs ``[N, 3K/16+16]`` -- the same codes as FP6 E3M2 values for the
    FP6 MFMA (``repack_weight_e3m2``; the gate/up weights at load): the ops quantize the
    activations into the matching E3M2 fragments.  All weights of one call must share it.

There is no CPU fallback: without the library (or without a GPU) the ops raise.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import weakref
from pathlib import Path

import torch

MFMA_MARKER_WORDS = 16
WMMA_MARKER_WORDS = 9
E3M2_MARKER_WORDS = 16  # [N, 3K/16 + 16]: E3M2 codes are 3K/16 words per column

_LAYOUT_ROW_MAJOR = 0
_LAYOUT_WMMA_TILED = 1

_LIB_NAME = "libpi05_w4a4.so"
_lib = None
_op_registered = False


def library_path() -> Path:
    override = os.environ.get("PI05_W4A4_LIB")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / "_lib" / _LIB_NAME


def _build_library(path: Path) -> None:
    """Compile the library to ``path`` with hipcc (``build_lib.py`` beside the package:
    offload target from PYTORCH_ROCM_ARCH / GPU_ARCHS, commands shown with
    PI05_W4A4_VERBOSE=1), as the reference's loader JIT-builds on first use."""
    import importlib.util

    script = Path(__file__).resolve().parents[2] / "build_lib.py"
    if not script.is_file():
        raise RuntimeError(f"W4A4 HIP library not found at {path}, and no build script at {script}")
    spec = importlib.util.spec_from_file_location("_pi05_w4a4_build_lib", script)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if mod.verbose_from_env():
        print(f"w4a4: building {path} for {','.join(mod.target_archs())}", flush=True)
    mod.build(out=path)


def load_int4_gemm():
    """Load the gfx950 C-ABI library, building it first when it is absent (the reference
    JIT-builds its pybind module here, extension.py:15-75).  ``PI05_W4A4_NO_BUILD=1``
    turns the build off: a missing library then raises."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.is_file():
        if os.environ.get("PI05_W4A4_NO_BUILD", "0") == "1":
            raise RuntimeError(
                f"W4A4 HIP library not found at {path} (PI05_W4A4_NO_BUILD=1); build it first "
                "(python pi05-pytorch-fast_amd/build_lib.py, or __graft_entry__.build())"
            )
        try:
            _build_library(path)
        except Exception as e:  # noqa: BLE001 - surfaced with the path
            raise RuntimeError(f"W4A4 HIP library not found at {path}, and building it failed: {e}") from e
    lib = ctypes.CDLL(str(path))
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    sig = {
        "pi05w4a4_version": (ctypes.c_int, []),
        "pi05w4a4_last_error": (ctypes.c_char_p, []),
        "pi05w4a4_quantize": (ctypes.c_int, [vp, i64, i32, vp, vp, vp]),
        "pi05w4a4_quantize_warm": (ctypes.c_int, [vp, i64, i32, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(sz),
                                                  i32, vp]),
        "pi05w4a4_q_words": (sz, [i64, i32]),
        "pi05w4a4_mfma_words": (sz, [i32, i32]),
        "pi05w4a4_repack_weight": (ctypes.c_int, [vp, i32, i32, i32, i64, vp, vp]),
        "pi05w4a4_gemm_workspace_bytes": (sz, [i64, i32, i32, vp, i32]),
        "pi05w4a4_gemm": (ctypes.c_int, [vp, vp, i64, i32, vp, i32, vp, vp, sz, vp]),
        "pi05w4a4_gemm_multi": (ctypes.c_int, [vp, vp, i64, i32, i32, vp, vp, vp, vp, sz, vp]),
        "pi05w4a4_gemm_gelu_up": (ctypes.c_int, [vp, vp, i64, i32, vp, vp, i32, vp, vp, sz, vp]),
        "pi05w4a4_gemm_acc": (ctypes.c_int, [vp, i64, i32, vp, i32, vp, vp]),
        "pi05w4a4_int4_gemm": (ctypes.c_int, [vp, i64, i32, vp, i32, vp, vp, vp, vp, sz, vp]),
        "pi05w4a4_int4_gemm_noalloc": (ctypes.c_int, [vp, i64, i32, vp, i32, vp, vp]),
        "pi05w4a4_rmsnorm": (ctypes.c_int, [vp, vp, ctypes.c_float, i32, i64, i32, vp, vp]),
        "pi05w4a4_gelu_tanh_mul": (ctypes.c_int, [vp, vp, i64, vp, vp]),
        "pi05w4a4_gemm_residual": (ctypes.c_int, [vp, vp, i64, i32, vp, i32, vp, vp, vp, sz, vp]),
        "pi05w4a4_quant_gemm_small": (ctypes.c_int, [vp, vp, ctypes.c_float, i32, i64, i32, i32, vp, vp, vp, vp, vp]),
        "pi05w4a4_rmsnorm_quantize": (ctypes.c_int, [vp, vp, ctypes.c_float, i32, i64, i32, vp, vp, vp]),
        "pi05w4a4_rmsnorm_quantize_warm": (
            ctypes.c_int, [vp, vp, ctypes.c_float, i32, i64, i32, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(sz), i32,
                           vp]),
        "pi05w4a4_attn_kv_mfma_elems": (sz, [i64, i32, i32, i32]),
        "pi05w4a4_attn_kv_prep": (ctypes.c_int, [vp, vp, i64, vp, vp, i64, i32, i32, i32, vp, vp, vp]),
        "pi05w4a4_prefix_attention": (
            ctypes.c_int,
            [vp, i64, vp, vp, vp, vp, i64, i64, i32, ctypes.c_float, i64, i32, i32, i32, i32, vp, i64, vp, vp, vp],
        ),
        "pi05w4a4_prefix_attention_warm": (
            ctypes.c_int,
            [vp, i64, vp, vp, vp, vp, i64, i64, i32, ctypes.c_float, i64, i32, i32, i32, i32, vp, i64, vp, vp,
             ctypes.POINTER(vp), ctypes.POINTER(sz), i32, vp],
        ),
        "pi05w4a4_gemm_qkv_rope": (
            ctypes.c_int, [vp, vp, i64, i32, vp, i32, vp, vp, vp, vp, i64, i32, vp, vp, vp, vp, vp]),
        "pi05w4a4_permute_rope_pairs": (ctypes.c_int, [vp, i32, vp, vp]),
        "pi05w4a4_gemm_gelu_up_quant": (
            ctypes.c_int, [vp, vp, i64, i32, vp, vp, i32, vp, vp, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(sz),
                           i32, i32, i32, vp]),
        "pi05w4a4_mlp_ctl_words": (sz, [i64]),
        "pi05w4a4_mlp_status": (i64, [i32]),
        "pi05w4a4_q_e3m2_bytes": (sz, [i64, i32]),
        "pi05w4a4_e3m2_words": (sz, [i32, i32]),
        "pi05w4a4_repack_weight_e3m2": (ctypes.c_int, [vp, i32, i32, vp, vp]),
        "pi05w4a4_quantize_e3m2": (ctypes.c_int, [vp, i64, i32, vp, vp, vp]),
        "pi05w4a4_rmsnorm_quantize_e3m2": (ctypes.c_int, [vp, vp, ctypes.c_float, i32, i64, i32, vp, vp, vp]),
        "pi05w4a4_rmsnorm_quantize_e3m2_warm": (
            ctypes.c_int, [vp, vp, ctypes.c_float, i32, i64, i32, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(sz), i32,
                           vp]),
        "pi05w4a4_gemm_e3m2": (ctypes.c_int, [vp, vp, i64, i32, i32, vp, vp, vp, i32, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_int4_gemm().pi05w4a4_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


# The current stream of a device as a raw pointer value (torch.cuda.current_stream(d)
# .cuda_stream without building Stream objects), and tensor pointers as plain ints (the
# ctypes argtypes convert them): the ops' host path runs once per projection in eager use.
_raw_stream = torch._C._cuda_getCurrentRawStream


def _stream(device: torch.device) -> int:
    idx = device.index
    return _raw_stream(torch._C._cuda_getDevice() if idx is None else idx)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_NO_SWITCH = contextlib.nullcontext()


def _on_device(device: torch.device):
    """torch.cuda.device(device), or nothing when it is already the current device (the
    library launches on the current HIP device)."""
    idx = device.index
    if idx is None or idx == torch._C._cuda_getDevice():
        return _NO_SWITCH
    return torch.cuda.device(device)


def _q_words(m: int, k: int) -> int:
    """pi05w4a4_q_words: activation code words of M rows (16-row blocks x 128-deep k
    blocks of 256 words) followed by one row correction per row of those blocks."""
    if m <= 0 or k <= 0:
        return 0
    mb = (m + 15) // 16
    return mb * 16 * ((k + 127) // 128) * 16 + mb * 16


_WS_CACHE: dict[tuple, int] = {}
_KV_ELEMS: dict[tuple, int] = {}
_N_ARRAYS: dict[tuple, ctypes.Array] = {}


def _n_array(ns: tuple) -> ctypes.Array:
    arr = _N_ARRAYS.get(ns)
    if arr is None:
        arr = _N_ARRAYS[ns] = (ctypes.c_int32 * len(ns))(*ns)
    return arr


def _workspace_bytes(lib, device: torch.device, m: int, k: int, ns: tuple, gelu: bool) -> int:
    """pi05w4a4_gemm_workspace_bytes, cached per shape and device (the split-K plan
    depends on the device's CU count)."""
    key = (device.index, m, k, ns, gelu)
    nbytes = _WS_CACHE.get(key)
    if nbytes is None:
        with _on_device(device):
            nbytes = _WS_CACHE[key] = int(lib.pi05w4a4_gemm_workspace_bytes(m, k, len(ns), _n_array(ns),
                                                                             1 if gelu else 0))
    return nbytes


def _kv_mfma_elems(lib, b: int, s: int, kvh: int, d: int) -> int:
    key = (b, s, kvh, d)
    n = _KV_ELEMS.get(key)
    if n is None:
        n = _KV_ELEMS[key] = int(lib.pi05w4a4_attn_kv_mfma_elems(b, s, kvh, d))
    return n


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Split-K workspace for one call.  Every call overwrites it completely (no zeroing),
    so a fresh block from the caching allocator is enough, also under graph capture."""
    if nbytes <= 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


# ----------------------------------------------------------------------------- checks
def _check_x(x: torch.Tensor) -> int:
    """quantize_x preconditions (int4_gemm.cu:497-501)."""
    if not x.is_cuda:
        raise RuntimeError("int4_gemm expects CUDA/HIP tensors")
    if x.dtype != torch.float16:
        raise RuntimeError("int4_gemm activations must be float16")
    if x.dim() == 0 or x.size(-1) <= 0:
        raise RuntimeError("Expected x.size(-1) > 0 to be true, but got false.")
    k = int(x.size(-1))
    if k % 64 != 0:
        raise RuntimeError(f"K must be a multiple of 64, got {k}")
    return k


def _check_packed(w: torch.Tensor, k: int, name: str = "packed W") -> None:
    """check_packed (int4_gemm.cu:487-494)."""
    if not w.is_cuda:
        raise RuntimeError(f"{name} must be on CUDA/HIP")
    _check_packed_shape(w, k, name)


def _check_packed_shape(w: torch.Tensor, k: int, name: str = "packed W") -> None:
    if w.dtype != torch.int32 or w.dim() != 2:
        raise RuntimeError(f"{name} must be int32 [N, K/8+1]")
    if w.size(1) < k // 8 + 1:
        raise RuntimeError(f"{name} second dim must contain K/8 packed words plus a scale")


def _check_tiled(w: torch.Tensor, k: int) -> None:
    """Tiled-layout checks of gemm_from_q<true> (int4_gemm.cu:570-577)."""
    n = int(w.size(0))
    if w.size(1) == k // 8 + MFMA_MARKER_WORDS and n % 16 == 0:
        return  # already MFMA-fragment-major: accepted by the tiled ops as well
    if not (k == 2048 and n == 16384):
        raise RuntimeError("WMMA-fragment-major weights currently support only K=2048, N=16384")
    if w.size(1) != k // 8 + WMMA_MARKER_WORDS:
        raise RuntimeError("WMMA-fragment-major weights must use the K/8+9 marker stride")


def is_mfma_layout(w: torch.Tensor, k: int) -> bool:
    return w.dim() == 2 and w.size(1) == k // 8 + MFMA_MARKER_WORDS and w.size(0) % 16 == 0


def is_e3m2_layout(w: torch.Tensor, k: int) -> bool:
    """An E3M2 column-pair weight [N, 3K/16 + 16] (K % 128 == 0, N % 32 == 0)."""
    return (w.dim() == 2 and k % 128 == 0 and w.size(1) == 3 * k // 16 + E3M2_MARKER_WORDS
            and w.size(0) % 32 == 0)


def _q6_bytes(m: int, k: int) -> int:
    """pi05w4a4_q_e3m2_bytes: 1536 bytes per 16-row block and 128-deep k block."""
    if m <= 0 or k <= 0:
        return 0
    return (m + 15) // 16 * ((k + 127) // 128) * 1536


# ----------------------------------------------------------------------------- pieces
# ctypes argument arrays of warm lists, by their (pointer, bytes) pairs: building ctypes
# arrays costs several microseconds per call, a large share of an eager op call.
_WARM_ARGS: dict[tuple, tuple] = {}


def _warm_args(warm, who: str):
    """(pointer array, byte-size array, count) of the non-empty warm tensors, or None."""
    ws = [t for t in (warm or []) if t is not None and t.numel() > 0]
    if not ws:
        return None
    if len(ws) > 4 or any((not t.is_cuda) or (not t.is_contiguous()) for t in ws):
        raise RuntimeError(f"{who}: warm takes up to 4 contiguous CUDA/HIP tensors")
    key = tuple((t.data_ptr(), (t.numel() * t.element_size()) // 16 * 16) for t in ws)
    hit = _WARM_ARGS.get(key)
    if hit is None:
        if len(_WARM_ARGS) > 1024:
            _WARM_ARGS.clear()
        wp = (ctypes.c_void_p * len(key))(*[p for p, _ in key])
        wb = (ctypes.c_size_t * len(key))(*[b for _, b in key])
        hit = _WARM_ARGS[key] = (wp, wb, len(key))
    return hit


def quantize(x: torch.Tensor, warm: list[torch.Tensor] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused FWHT + per-token INT4 quant + nibble pack (the reference's quantize_x,
    int4_gemm.cu:496-531): x fp16 [..., K] -> (q, sa fp32 [M]).

    ``q`` is int32 ``[pi05w4a4_q_words(M, K)]`` holding the codes in the
    MFMA-fragment-major layout the GEMM reads (``pack.codes_from_fragment_major`` converts
    it back to the reference's row-major ``[M, K/8]`` words); M is padded to 16 rows and K
    to 128 codes.
    """
    k = _check_x(x)
    x2 = x if x.is_contiguous() else x.contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    m = x2.numel() // k
    lib = _lib if _lib is not None else load_int4_gemm()
    dev = x2.device
    q = torch.empty((_q_words(m, k),), dtype=torch.int32, device=dev)
    sa = torch.empty((m,), dtype=torch.float32, device=dev)
    with _on_device(dev):
        wa = _warm_args(warm, "quantize") if warm else None
        if wa is None:
            _check(lib.pi05w4a4_quantize(x2.data_ptr(), m, k, q.data_ptr(), sa.data_ptr(), _stream(dev)),
                   "pi05w4a4_quantize")
        else:
            _check(lib.pi05w4a4_quantize_warm(x2.data_ptr(), m, k, q.data_ptr(), sa.data_ptr(), *wa, _stream(dev)),
                   "pi05w4a4_quantize_warm")
    return q, sa


def repack_weight(w: torch.Tensor, k: int | None = None, tiled: bool | None = None) -> torch.Tensor:
    """Repack an L1/L2 (row-major) or L3 (WMMA-tiled, [N, K/8+9]) packed weight into the
    MFMA-fragment-major tensor int32 [N, K/8+16].  N must be a multiple of 16.

    ``k`` defaults to (size(1)-1)*8 for row-major input and (size(1)-9)*8 for tiled input.
    ``tiled`` defaults to the K/8+9 marker-stride convention (pack.py:45-50).
    """
    if not w.is_cuda:
        raise RuntimeError("packed W must be on CUDA/HIP")
    if w.dtype != torch.int32 or w.dim() != 2:
        raise RuntimeError("packed W must be int32 [N, K/8+1]")
    n = int(w.size(0))
    if tiled is None:
        tiled = k is not None and w.size(1) == k // 8 + WMMA_MARKER_WORDS
    if k is None:
        k = (int(w.size(1)) - (WMMA_MARKER_WORDS if tiled else 1)) * 8
    if k % 64 != 0:
        raise RuntimeError(f"K must be a multiple of 64, got {k}")
    if n % 16 != 0:
        raise RuntimeError(f"MFMA layout needs N % 16 == 0, got N={n}")
    src = w.contiguous()
    if not tiled and src.size(1) < k // 8 + 1:
        raise RuntimeError("packed W second dim must contain K/8 packed words plus a scale")
    out = torch.zeros((n, k // 8 + MFMA_MARKER_WORDS), dtype=torch.int32, device=w.device)
    lib = load_int4_gemm()
    layout = _LAYOUT_WMMA_TILED if tiled else _LAYOUT_ROW_MAJOR
    with torch.cuda.device(w.device):
        _check(lib.pi05w4a4_repack_weight(_ptr(src), layout, n, k, int(src.size(1)), _ptr(out),
                                          _stream(w.device)), "pi05w4a4_repack_weight")
    return out


def repack_weight_e3m2(w: torch.Tensor, k: int | None = None, tiled: bool | None = None) -> torch.Tensor:
    """The E3M2 column-pair form ``[N, 3K/16 + 16]`` of a packed weight (any layout
    ``repack_weight`` reads, or the MFMA layout): the same INT4 codes as FP6 E3M2 values,
    for the FP6-MFMA GEMM.  N % 32 == 0 and K % 128 == 0."""
    if not w.is_cuda:
        raise RuntimeError("packed W must be on CUDA/HIP")
    if w.dtype != torch.int32 or w.dim() != 2:
        raise RuntimeError("packed W must be int32 [N, K/8+1]")
    n = int(w.size(0))
    if k is None:
        if tiled is None:
            tiled = False
        k = (int(w.size(1)) - (WMMA_MARKER_WORDS if tiled else 1)) * 8
    if k % 128 != 0 or n % 32 != 0:
        raise RuntimeError(f"the E3M2 layout needs K % 128 == 0 and N % 32 == 0, got N={n} K={k}")
    if is_e3m2_layout(w, k):
        return w
    src = w if is_mfma_layout(w, k) else repack_weight(w, k, tiled=tiled)
    out = torch.zeros((n, 3 * k // 16 + E3M2_MARKER_WORDS), dtype=torch.int32, device=w.device)
    lib = load_int4_gemm()
    with torch.cuda.device(w.device):
        _check(lib.pi05w4a4_repack_weight_e3m2(_ptr(src.contiguous()), n, k, _ptr(out), _stream(w.device)),
               "pi05w4a4_repack_weight_e3m2")
    return out


def quantize_e3m2(x: torch.Tensor, norm=None, warm: list[torch.Tensor] | None = None
                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """``quantize`` (or, with ``norm`` = (weight, eps, unit_offset), ``rms_norm_quantize``)
    with the codes written as E3M2 fragments (uint8 [pi05w4a4_q_e3m2_bytes(M, K)]): the
    activation form of the FP6-MFMA GEMM.  K = 2048.  ``warm`` (with ``norm``): buffers the
    launch's idle CUs read into the Infinity Cache, as in ``rms_norm_quantize``."""
    k = _check_x(x)
    if k != 2048:
        raise RuntimeError(f"the E3M2 quantizer takes K = 2048, got {k}")
    x2 = x if x.is_contiguous() else x.contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    m = x2.numel() // k
    lib = _lib if _lib is not None else load_int4_gemm()
    dev = x2.device
    q6 = torch.empty((_q6_bytes(m, k),), dtype=torch.uint8, device=dev)
    sa = torch.empty((m,), dtype=torch.float32, device=dev)
    with _on_device(dev):
        if norm is None:
            _check(lib.pi05w4a4_quantize_e3m2(x2.data_ptr(), m, k, q6.data_ptr(), sa.data_ptr(), _stream(dev)),
                   "pi05w4a4_quantize_e3m2")
        else:
            weight, eps, unit_offset = norm
            if not weight.is_cuda or weight.dtype != torch.float16 or weight.dim() != 1 or weight.numel() != k:
                raise RuntimeError(f"RMSNorm weight must be a float16 CUDA/HIP tensor [{k}]")
            wn = weight if weight.is_contiguous() else weight.contiguous()
            wa = _warm_args(warm, "quantize_e3m2") if warm else None
            if wa is None:
                _check(lib.pi05w4a4_rmsnorm_quantize_e3m2(x2.data_ptr(), wn.data_ptr(), float(eps),
                                                          1 if unit_offset else 0, m, k, q6.data_ptr(),
                                                          sa.data_ptr(), _stream(dev)),
                       "pi05w4a4_rmsnorm_quantize_e3m2")
            else:
                _check(lib.pi05w4a4_rmsnorm_quantize_e3m2_warm(x2.data_ptr(), wn.data_ptr(), float(eps),
                                                               1 if unit_offset else 0, m, k, q6.data_ptr(),
                                                               sa.data_ptr(), *wa, _stream(dev)),
                       "pi05w4a4_rmsnorm_quantize_e3m2_warm")
    return q6, sa


def _gemm_e3m2_from_q(q6, sa, k, weights, out_shape_prefix, device, gelu=False):
    """GEMMs of 1..3 E3M2-layout weights (or the GELU pair) from E3M2 activation codes."""
    lib = _lib if _lib is not None else load_int4_gemm()
    m = int(sa.size(0))
    ns = tuple(int(w.size(0)) for w in weights)
    outs = [torch.empty((m, ns[0]), dtype=torch.float16, device=device)] if gelu else \
        [torch.empty((m, nn), dtype=torch.float16, device=device) for nn in ns]
    g = len(ns)
    w_arr = (ctypes.c_void_p * g)(*[w.data_ptr() for w in weights])
    y_arr = (ctypes.c_void_p * g)(*([outs[0].data_ptr(), None] if gelu else [o.data_ptr() for o in outs]))
    _check(lib.pi05w4a4_gemm_e3m2(q6.data_ptr(), sa.data_ptr(), m, k, g, w_arr, _n_array(ns), y_arr,
                                  1 if gelu else 0, _stream(device)), "pi05w4a4_gemm_e3m2")
    return [o.view(*out_shape_prefix, o.size(1)) for o in outs]


# Repacked copies of weights that arrive in a reference layout (L1/L2/L3), one per source
# tensor object: the repack runs on the first call only.  An entry is dropped when its
# source tensor is freed, and it is rebuilt when the tensor is modified in place through
# itself (its version counter moves), when its storage is replaced (``w.data = new``: the
# data pointer moves) or when it is used with another K.  An in-place write through
# ``w.data`` (``w.data.copy_(new)``) moves neither: after one, call
# ``clear_weight_caches()``.
_MFMA_CACHE: dict[int, tuple] = {}
# Other per-weight caches (the fused layer's RoPE-pair K copies) register a function that
# drops them; clear_weight_caches() runs every one.
_CACHE_CLEARERS: list = []


# INT4 MFMA-layout twins of E3M2-layout weights, registered by the loader, which converts
# the MLP's gate/up weights to E3M2 and keeps both forms (apply.load_time_weight): calls
# of at most E3M2_MAX_INT4_ROWS rows run the INT4 kernels on the twins, since the E3M2
# GEMM has no small-M tiles (gate/up + GELU at 1-128 rows: 17-18 us on E3M2 weights
# against 6-12 us on INT4 ones; from 160 rows on E3M2 is faster).  An entry lives as long
# as its E3M2 weight and is ignored once that weight is modified in place (version or data
# pointer moved): the call then runs on the E3M2 weight.  A write through ``w.data`` moves
# neither: clear_weight_caches() then drops every twin (and the calls run on the E3M2
# weights, correct and slower at few rows).
E3M2_MAX_INT4_ROWS = 128
_INT4_TWINS: dict[int, tuple] = {}


def register_int4_twin(w_e3m2: torch.Tensor, w_int4: torch.Tensor, k: int) -> None:
    """Record w_int4 (MFMA layout) as the INT4 form of the E3M2-layout weight w_e3m2."""
    if not (is_e3m2_layout(w_e3m2, k) and is_mfma_layout(w_int4, k)):
        raise RuntimeError("register_int4_twin takes an E3M2-layout weight and its MFMA-layout INT4 form")
    if int(w_e3m2.size(0)) != int(w_int4.size(0)):
        raise RuntimeError("the two forms of a weight must have the same N")
    key = id(w_e3m2)
    _INT4_TWINS[key] = (weakref.ref(w_e3m2, lambda _r, key=key: _INT4_TWINS.pop(key, None)), w_e3m2._version,
                        w_e3m2.data_ptr(), k, w_int4)


def int4_twin(w: torch.Tensor, k: int) -> torch.Tensor | None:
    """The registered INT4 form of the E3M2-layout weight w, or None."""
    hit = _INT4_TWINS.get(id(w))
    if hit is None:
        return None
    ref, version, ptr, hk, twin = hit
    if ref() is not w or version != w._version or ptr != w.data_ptr() or hk != k:
        return None
    return twin


def gemm_weights_for_rows(ws: list[torch.Tensor], k: int, m: int) -> list[torch.Tensor]:
    """The tensors a call of m rows on the weights ws reads: the INT4 twins of E3M2-layout
    weights at m <= E3M2_MAX_INT4_ROWS when every weight has one, else ws (for cache
    warming lists)."""
    if m <= E3M2_MAX_INT4_ROWS and ws and all(is_e3m2_layout(w, k) for w in ws):
        twins = [int4_twin(w, k) for w in ws]
        if all(t is not None for t in twins):
            return twins
    return list(ws)


def clear_weight_caches() -> None:
    """Drop every derived copy of a weight that the ops keep (the repacked L1/L2/L3
    weights, the RoPE-pair K weights of fused decoder layers and the INT4 twins of E3M2
    weights), so that the next call rebuilds them from the current weights (a twin is not
    rebuilt: calls on its E3M2 weight run the E3M2 kernels).  Needed after writing a
    weight in place through ``.data`` (which bypasses the version counter the caches
    check)."""
    _MFMA_CACHE.clear()
    _INT4_TWINS.clear()
    for fn in _CACHE_CLEARERS:
        fn()


def register_cache_clearer(fn) -> None:
    """Add ``fn`` (no arguments) to what clear_weight_caches() runs."""
    _CACHE_CLEARERS.append(fn)


def _as_mfma(w: torch.Tensor, k: int, tiled: bool) -> tuple[torch.Tensor, int]:
    """Weight in MFMA layout (repacked once per source tensor when needed) and its true N."""
    n = int(w.size(0))
    if is_mfma_layout(w, k):
        return w, n
    key = id(w)
    hit = _MFMA_CACHE.get(key)
    if hit is not None:
        ref, version, ptr, hk, htiled, out = hit
        if ref() is w and version == w._version and ptr == w.data_ptr() and hk == k and htiled == tiled:
            return out, n
    if tiled:
        out = repack_weight(w, k, tiled=True)
    else:
        src = w
        if n % 16 != 0:
            src = torch.nn.functional.pad(w.contiguous(), (0, 0, 0, 16 - n % 16))
        out = repack_weight(src, k, tiled=False)
    _MFMA_CACHE[key] = (weakref.ref(w, lambda _r, key=key: _MFMA_CACHE.pop(key, None)), w._version, w.data_ptr(),
                        k, tiled, out)
    return out, n


def _check_gelu_weights(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> None:
    """Gate and up weights of the fused GELU epilogue: one shape, row-major (L1/L2) or
    MFMA layout.  WMMA-tiled weights (the K/8+9 marker stride of pack.py:45-50) would be
    misread as row-major, so they are refused."""
    if w_gate.shape != w_up.shape:
        raise RuntimeError("gate and up weights must have the same shape")
    k = int(x.size(-1)) if x.dim() else 0
    if w_gate.dim() == 2 and w_gate.size(1) == k // 8 + WMMA_MARKER_WORDS:
        raise RuntimeError("int4_gemm2_gelu takes row-major or MFMA-layout weights; WMMA-tiled "
                           "(K/8+9) gate/up weights go through int4_gemm2_tiled")


def _check_residual(residual: torch.Tensor, device: torch.device, shape: tuple) -> None:
    """The residual of a fused residual-add GEMM: a float16 tensor of the output's shape on
    the activations' device (the kernel reads it as fp16 through a device pointer)."""
    if not isinstance(residual, torch.Tensor):
        raise RuntimeError("residual must be a tensor")
    if residual.device != device:
        raise RuntimeError(f"residual must be on {device}, got {residual.device}")
    if residual.dtype != torch.float16:
        raise RuntimeError(f"residual must be float16, got {residual.dtype}")
    if tuple(residual.shape) != tuple(shape):
        raise RuntimeError(f"residual must be [{', '.join(map(str, shape))}] "
                           f"with N a multiple of 16, got {tuple(residual.shape)}")


def _gemm_from_q(q, sa, k, weights, out_shape_prefix, device, kind, gelu=False, residual=None):
    """Shared-activation GEMMs of 1..3 MFMA-layout weights (one launch); with ``residual``
    (one weight) the epilogue adds it: fp16(fp16(y) + residual)."""
    lib = _lib if _lib is not None else load_int4_gemm()
    m = int(sa.size(0))
    ns = tuple(int(w.size(0)) for (w, _) in weights)
    if residual is not None:
        (w0, n_true), = weights
        if n_true != ns[0]:
            raise RuntimeError(f"residual must be [{', '.join(map(str, out_shape_prefix))}, {n_true}] "
                               f"with N a multiple of 16, got {tuple(residual.shape)}")
        _check_residual(residual, device, (*out_shape_prefix, n_true))
        res = residual if residual.is_contiguous() and residual.data_ptr() % 16 == 0 else residual.contiguous().clone()
        out = torch.empty((m, n_true), dtype=torch.float16, device=device)
        ws_bytes = _workspace_bytes(lib, device, m, k, ns, False)
        ws = _workspace(device, ws_bytes)
        _check(lib.pi05w4a4_gemm_residual(q.data_ptr(), sa.data_ptr(), m, k, w0.data_ptr(), n_true, res.data_ptr(),
                                          out.data_ptr(), _ptr(ws), ws_bytes, _stream(device)),
               "pi05w4a4_gemm_residual")
        return [out.view(*out_shape_prefix, n_true)]
    ws_bytes = _workspace_bytes(lib, device, m, k, ns, gelu)
    ws = _workspace(device, ws_bytes)
    stream = _stream(device)
    if gelu:
        outs = [torch.empty((m, ns[0]), dtype=torch.float16, device=device)]
        rc = lib.pi05w4a4_gemm_gelu_up(q.data_ptr(), sa.data_ptr(), m, k, weights[0][0].data_ptr(),
                                       weights[1][0].data_ptr(), ns[0], outs[0].data_ptr(), _ptr(ws), ws_bytes,
                                       stream)
    else:
        outs = [torch.empty((m, nn), dtype=torch.float16, device=device) for nn in ns]
        g = len(ns)
        w_arr = (ctypes.c_void_p * g)(*[w.data_ptr() for (w, _) in weights])
        y_arr = (ctypes.c_void_p * g)(*[o.data_ptr() for o in outs])
        rc = lib.pi05w4a4_gemm_multi(q.data_ptr(), sa.data_ptr(), m, k, g, w_arr, _n_array(ns), y_arr, _ptr(ws),
                                     ws_bytes, stream)
    _check(rc, "pi05w4a4_gemm")
    results = []
    for o, (w, n_true) in zip(outs, weights):
        if o.size(1) != n_true:
            o = o[:, :n_true].contiguous()
        results.append(o.view(*out_shape_prefix, n_true))
    return results


def rms_norm_quantize(x: torch.Tensor, weight: torch.Tensor, eps: float,
                      unit_offset: bool = True, warm: list[torch.Tensor] | None = None
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """``quantize`` of ``rms_norm(x, weight, eps, unit_offset)`` in one kernel (K = 2048):
    the norm's fp16 output is rotated and quantized without being stored.  ``warm``: up to 4
    device tensors that the CUs left idle by the rows read into the Infinity Cache (the
    GEMM's weights); the results are the same."""
    k = _check_x(x)
    if k != 2048:
        raise RuntimeError(f"the fused RMSNorm quantizer takes K = 2048, got {k}")
    if not weight.is_cuda or weight.dtype != torch.float16 or weight.dim() != 1 or weight.numel() != k:
        raise RuntimeError(f"RMSNorm weight must be a float16 CUDA/HIP tensor [{k}]")
    x2 = x if x.is_contiguous() else x.contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    w = weight if weight.is_contiguous() else weight.contiguous()
    m = x2.numel() // k
    lib = _lib if _lib is not None else load_int4_gemm()
    dev = x2.device
    q = torch.empty((_q_words(m, k),), dtype=torch.int32, device=dev)
    sa = torch.empty((m,), dtype=torch.float32, device=dev)
    with _on_device(dev):
        wa = _warm_args(warm, "rms_norm_quantize") if warm else None
        if wa is None:
            _check(lib.pi05w4a4_rmsnorm_quantize(x2.data_ptr(), w.data_ptr(), float(eps), 1 if unit_offset else 0, m,
                                                 k, q.data_ptr(), sa.data_ptr(), _stream(dev)),
                   "pi05w4a4_rmsnorm_quantize")
        else:
            _check(lib.pi05w4a4_rmsnorm_quantize_warm(x2.data_ptr(), w.data_ptr(), float(eps), 1 if unit_offset else 0,
                                                      m, k, q.data_ptr(), sa.data_ptr(), *wa, _stream(dev)),
                   "pi05w4a4_rmsnorm_quantize_warm")
    return q, sa


# Weights up to this many bytes per call are read into the Infinity Cache by the norm +
# quant launch ahead of their GEMM (the QKV projections: 2.6 MB at PaliGemma-2B sizes),
# from this many rows on.  With fewer rows the launch is too short to hide the reads: at
# M = 1 the norm + quant + QKV pair took 8.76 us with warming against 8.41 without, at
# M = 640 13.58 against 14.14 (weights from HBM).
_NORM_WARM_MAX_BYTES = 16 << 20
_NORM_WARM_MIN_ROWS = 256


# The tail of the up weight that the gate/up op's own norm + quant launch warms (from
# _NORM_WARM_MIN_ROWS rows on); the fused decoder layer's attention launch warms the rest
# (gate_up_warm_split).  At 776 tokens, E3M2 weights (forward A/B in one process, three
# rounds): 3-6 MB 15-25 us faster than none, 8 MB less, 12 MB and all 26 MB slower.
_GATE_UP_SELF_WARM_BYTES = 4 << 20


_UP_SPLITS: dict[int, tuple] = {}


def gate_up_warm_split(w_up: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor | None]:
    """(head, tail) byte ranges of the up weight as flat views: the gate/up op's norm +
    quant launch warms the tail (at most _GATE_UP_SELF_WARM_BYTES, a multiple of 16 bytes),
    the caller may warm the head earlier.  Cached per tensor (same storage, version and
    split size)."""
    key = id(w_up)
    hit = _UP_SPLITS.get(key)
    if hit is not None:
        ref, ptr, version, nbytes, split = hit
        if ref() is w_up and ptr == w_up.data_ptr() and version == w_up._version and nbytes == _GATE_UP_SELF_WARM_BYTES:
            return split
    split = _gate_up_split(w_up)
    _UP_SPLITS[key] = (weakref.ref(w_up, lambda _r, key=key: _UP_SPLITS.pop(key, None)), w_up.data_ptr(),
                       w_up._version, _GATE_UP_SELF_WARM_BYTES, split)
    return split


def _gate_up_split(w_up: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor | None]:
    flat = w_up.reshape(-1)
    per16 = max(1, 16 // flat.element_size())
    tail = min(flat.numel(), _GATE_UP_SELF_WARM_BYTES // flat.element_size()) // per16 * per16
    if tail <= 0:
        return flat, None
    return flat[: flat.numel() - tail], flat[flat.numel() - tail:]


def _gate_up_warm(w_up: torch.Tensor, x: torch.Tensor) -> list[torch.Tensor] | None:
    """The up weight's tail for the gate/up op's norm + quant launch to warm."""
    if os.environ.get("PI05_W4A4_CACHE_WARM", "1") == "0" or not (w_up.is_cuda and w_up.is_contiguous()):
        return None
    if x.numel() // int(x.size(-1)) < _NORM_WARM_MIN_ROWS:
        return None
    return [t for t in gate_up_warm_split(w_up)[1:] if t is not None and t.numel() > 0] or None


def _norm_warm(ws: list[torch.Tensor], x: torch.Tensor) -> list[torch.Tensor] | None:
    """The weights for the norm + quant launch of x to warm (PI05_W4A4_CACHE_WARM=0: none):
    MFMA-layout weights only (what the GEMM reads), at most _NORM_WARM_MAX_BYTES in total,
    for at least _NORM_WARM_MIN_ROWS rows."""
    if os.environ.get("PI05_W4A4_CACHE_WARM", "1") == "0":
        return None
    k = int(x.size(-1))
    if x.numel() // k < _NORM_WARM_MIN_ROWS:
        return None
    if not all(w.is_cuda and w.is_contiguous() and is_mfma_layout(w, k) for w in ws):
        return None
    if sum(w.numel() * w.element_size() for w in ws) > _NORM_WARM_MAX_BYTES:
        return None
    return list(ws)


# Control blocks of pi05w4a4_gemm_gelu_up_quant, one per (device, stream): zeroed when
# allocated and left zeroed by every call that completes.  Calls on one stream are ordered,
# so they can share one; calls on different streams get their own.
_MLP_CTL: dict[tuple[int, int], torch.Tensor] = {}


def _mlp_ctl(lib, device: torch.device, m: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch._C._cuda_getDevice(), _stream(device))
    ctl = _MLP_CTL.get(key)
    words = int(lib.pi05w4a4_mlp_ctl_words(m))
    if ctl is None or ctl.numel() < words:
        ctl = _MLP_CTL[key] = torch.zeros(max(words, 64), dtype=torch.int32, device=device)
    return ctl


def _check_mlp_status(lib) -> None:
    """Raise when a bounded wait of an earlier fused gate/up + down-quant call ran out (the
    kernels set a pinned host word; reading it does not synchronize).  The control blocks
    are zeroed again so that later calls start clean."""
    if lib.pi05w4a4_mlp_status(0) > 0:
        lib.pi05w4a4_mlp_status(1)
        for ctl in _MLP_CTL.values():
            ctl.zero_()
        raise RuntimeError("pi05w4a4_gemm_gelu_up_quant: a bounded wait for a row block ran out in an "
                           "earlier call; that call's outputs are invalid")


def _gemm_gelu_quant_from_q(q, sa, k, w_gate, w_up, n, device, warm=None, spin_limit=0, wait_extra=0):
    """h = fp16(gelu_tanh(gate) * up) and the down projection's quant of h (codes, scales),
    from quantized activations (one launch at N = 16384, M > 64)."""
    lib = _lib if _lib is not None else load_int4_gemm()
    m = int(sa.size(0))
    h = torch.empty((m, n), dtype=torch.float16, device=device)
    dq = torch.empty((_q_words(m, n),), dtype=torch.int32, device=device)
    dsa = torch.empty((m,), dtype=torch.float32, device=device)
    wa = _warm_args(warm, "rms_norm_int4_mlp") if warm else None
    wp, wb, wn = wa if wa is not None else (None, None, 0)
    ctl = _mlp_ctl(lib, device, m)
    _check(lib.pi05w4a4_gemm_gelu_up_quant(q.data_ptr(), sa.data_ptr(), m, k, w_gate.data_ptr(), w_up.data_ptr(), n,
                                           h.data_ptr(), dq.data_ptr(), dsa.data_ptr(), ctl.data_ptr(), wp, wb, wn,
                                           int(spin_limit), int(wait_extra), _stream(device)),
           "pi05w4a4_gemm_gelu_up_quant")
    _check_mlp_status(lib)
    return h, dq, dsa


def _rms_norm_mlp_impl(x, norm_weight, eps, unit_offset, w_gate, w_up, w_down, residual, warm):
    """The Gemma MLP block of a decoder layer on W4A4 ops: post-attention RMSNorm fused into
    the gate/up activation quant, gate/up with the GELU-tanh*up epilogue and the down
    projection's activation quant in one launch, then down with the residual add in its
    epilogue.  Returns (residual + down(h), h)."""
    k = _check_x(x)
    _check_gelu_weights(x, w_gate, w_up)
    n = int(w_gate.size(0))
    for w, kw, name in ((w_gate, k, "gate weight"), (w_up, k, "up weight"), (w_down, n, "down weight")):
        _check_packed(w, kw, name)
        if not is_mfma_layout(w, kw):
            raise RuntimeError(f"rms_norm_int4_mlp takes MFMA-layout weights ({name}: [N, {kw // 8 + 16}] "
                               f"with N % 16 == 0, got {tuple(w.shape)})")
    _check_residual(residual, x.device, (*x.shape[:-1], int(w_down.size(0))))
    q, sa = rms_norm_quantize(x, norm_weight, eps, unit_offset)
    dev = x.device
    with _on_device(dev):
        h, dq, dsa = _gemm_gelu_quant_from_q(q, sa, k, w_gate, w_up, n, dev, warm=warm)
        (y,) = _gemm_from_q(dq, dsa, n, [(w_down, int(w_down.size(0)))], tuple(x.shape[:-1]), dev, "int4_gemm",
                            residual=residual)
    return y, h.view(*x.shape[:-1], n)


def _run(x: torch.Tensor, ws: list[torch.Tensor], tiled: bool, kind: str, gelu: bool = False,
         norm=None, residual=None, warm=None):
    k = _check_x(x)
    n_e3m2 = sum(1 for w in ws if is_e3m2_layout(w, k))
    if n_e3m2 == len(ws) and x.numel() // k <= E3M2_MAX_INT4_ROWS:
        twins = gemm_weights_for_rows(ws, k, x.numel() // k)
        if twins[0] is not ws[0]:  # small M on INT4 twins
            ws, n_e3m2 = twins, 0
    if n_e3m2:
        return _run_e3m2(x, ws, k, n_e3m2, kind, gelu, norm, residual, warm=warm)
    if residual is not None:  # before any launch: the kernel reads it through a raw pointer
        _check_residual(residual, x.device, (*x.shape[:-1], int(ws[0].size(0))))
    m = x.numel() // k
    if not gelu and k == 2048 and 1 <= m <= SMALL_M_MAX_ROWS and x.is_cuda:
        return _run_small(x, ws, k, m, tiled, kind, norm, residual)
    # the reference quantizes before checking the weights
    q, sa = quantize(x, warm) if norm is None else rms_norm_quantize(x, *norm, warm=warm)
    conv = []
    for w in ws:
        _check_packed(w, k)
        if tiled:
            _check_tiled(w, k)
        conv.append(_as_mfma(w, k, tiled))
    dev = x.device
    with _on_device(dev):
        return _gemm_from_q(q, sa, k, conv, tuple(x.shape[:-1]), dev, kind, gelu=gelu, residual=residual)


# Up to this many rows (K = 2048) a call quantizes inside its GEMM launch
# (pi05w4a4_quant_gemm_small): no activation codes in memory, one launch instead of two.
SMALL_M_MAX_ROWS = 4


def _run_small(x, ws, k, m, tiled, kind, norm, residual):
    """_run for 1..SMALL_M_MAX_ROWS rows at K = 2048 (INT4 weights, fp16 outputs): the norm
    (if any) and the activation quant run in the GEMM launch's prologue; outputs are the
    two-launch path's bit for bit."""
    conv = []
    for w in ws:
        _check_packed(w, k)
        if tiled:
            _check_tiled(w, k)
        conv.append(_as_mfma(w, k, tiled))
    x2 = x if x.is_contiguous() else x.contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    nw, eps, unit_offset = None, 0.0, False
    if norm is not None:
        weight, eps, unit_offset = norm
        if not weight.is_cuda or weight.dtype != torch.float16 or weight.dim() != 1 or weight.numel() != k:
            raise RuntimeError(f"RMSNorm weight must be a float16 CUDA/HIP tensor [{k}]")
        nw = weight if weight.is_contiguous() else weight.contiguous()
    dev = x2.device
    lib = _lib if _lib is not None else load_int4_gemm()
    outs = [torch.empty((m, int(w.size(0))), dtype=torch.float16, device=dev) for (w, _) in conv]
    res = None
    if residual is not None:
        (w0, n_true), = conv
        if n_true != int(w0.size(0)):
            raise RuntimeError(f"residual must be [{', '.join(map(str, x.shape[:-1]))}, {n_true}] "
                               f"with N a multiple of 16, got {tuple(residual.shape)}")
        res = residual if residual.is_contiguous() and residual.data_ptr() % 16 == 0 else residual.contiguous().clone()
    g = len(conv)
    w_arr = (ctypes.c_void_p * g)(*[w.data_ptr() for (w, _) in conv])
    y_arr = (ctypes.c_void_p * g)(*[o.data_ptr() for o in outs])
    with _on_device(dev):
        _check(lib.pi05w4a4_quant_gemm_small(x2.data_ptr(), _ptr(nw), float(eps), 1 if unit_offset else 0, m, k, g,
                                             w_arr, _n_array(tuple(int(w.size(0)) for (w, _) in conv)), y_arr,
                                             _ptr(res), _stream(dev)), f"pi05w4a4_quant_gemm_small ({kind})")
    results = []
    for o, (w, n_true) in zip(outs, conv):
        if o.size(1) != n_true:
            o = o[:, :n_true].contiguous()
        results.append(o.view(*x.shape[:-1], n_true))
    return results


def _run_e3m2(x, ws, k, n_e3m2, kind, gelu, norm, residual, warm=None):
    """_run for E3M2-layout weights: E3M2 activation quant, then the FP6-MFMA GEMM."""
    if n_e3m2 != len(ws):
        raise RuntimeError(f"{kind}: the weights of one call must all be E3M2-layout ([N, 3K/16+16]) or none")
    if residual is not None:
        raise RuntimeError(f"{kind}: the residual epilogue takes INT4-layout weights, not E3M2")
    for w in ws:
        _check_packed(w, k)
    q6, sa = quantize_e3m2(x, norm, warm=warm if norm is not None else None)
    dev = x.device
    with _on_device(dev):
        return _gemm_e3m2_from_q(q6, sa, k, ws, tuple(x.shape[:-1]), dev, gelu=gelu)


def _rms_norm_impl(x: torch.Tensor, weight: torch.Tensor, eps: float, unit_offset: bool) -> torch.Tensor:
    if not x.is_cuda or not weight.is_cuda:
        raise RuntimeError("rms_norm expects CUDA/HIP tensors")
    if x.dtype != torch.float16 or weight.dtype != torch.float16:
        raise RuntimeError("rms_norm expects float16 activations and weight")
    k = int(x.size(-1))
    if weight.dim() != 1 or int(weight.numel()) != k:
        raise RuntimeError(f"rms_norm weight must be [{k}], got {tuple(weight.shape)}")
    xc = x if x.is_contiguous() else x.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    y = torch.empty_like(xc)
    m = xc.numel() // k if k else 0
    lib = _lib if _lib is not None else load_int4_gemm()
    dev = x.device
    with _on_device(dev):
        _check(lib.pi05w4a4_rmsnorm(xc.data_ptr(), w.data_ptr(), float(eps), 1 if unit_offset else 0, m, k,
                                    y.data_ptr(), _stream(dev)), "pi05w4a4_rmsnorm")
    return y


def gelu_tanh_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """fp16(gelu(gate, approximate="tanh") * up) elementwise with the fused gate/up GEMM
    epilogue's arithmetic; equal bit for bit to the two eager fp16 ops (apply.py:135-138)."""
    if not gate.is_cuda or not up.is_cuda:
        raise RuntimeError("gelu_tanh_mul expects CUDA/HIP tensors")
    if gate.dtype != torch.float16 or up.dtype != torch.float16:
        raise RuntimeError("gelu_tanh_mul expects float16 tensors")
    if gate.shape != up.shape:
        raise RuntimeError(f"gelu_tanh_mul shapes differ: {tuple(gate.shape)} vs {tuple(up.shape)}")
    g = gate if gate.is_contiguous() else gate.contiguous()
    u = up if up.is_contiguous() else up.contiguous()
    y = torch.empty_like(g)
    lib = _lib if _lib is not None else load_int4_gemm()
    dev = gate.device
    with _on_device(dev):
        _check(lib.pi05w4a4_gelu_tanh_mul(g.data_ptr(), u.data_ptr(), g.numel(), y.data_ptr(), _stream(dev)),
               "pi05w4a4_gelu_tanh_mul")
    return y


ATTN_HEAD_DIM = 256
ATTN_MAX_KEYS = 1024


def _attention_mask_arg(mask: torch.Tensor | None, b: int, s: int, device: torch.device):
    """(tensor, batch stride, row stride, row length) of an additive fp16 mask [B|1, 1, S, >=S]
    on the queries' device, in the form the kernel reads (row length a multiple of 4 >= S,
    strides multiples of 4, 8-byte aligned); a padded copy is made only when the given tensor
    does not fit."""
    if mask is None:
        return None, 0, 0, 0
    if mask.device != device:
        raise RuntimeError(f"prefix_attention mask must be on {device}, got {mask.device}")
    if mask.dtype != torch.float16 or mask.dim() != 4 or mask.size(1) != 1:
        raise RuntimeError("prefix_attention mask must be an additive float16 [B, 1, S, Sk] tensor")
    if mask.size(0) not in (1, b) or mask.size(2) != s or mask.size(3) < s:
        raise RuntimeError(f"prefix_attention mask shape {tuple(mask.shape)} does not fit B={b}, S={s}")
    m = mask[:, 0, :, :]
    s4 = (s + 3) // 4 * 4
    fits = (
        m.size(2) >= s4
        and m.stride(2) == 1
        and m.stride(1) % 4 == 0
        and (m.size(0) == 1 or m.stride(0) % 4 == 0)
        and m.data_ptr() % 8 == 0
    )
    if not fits:
        m = torch.nn.functional.pad(m[:, :, :s], (0, s4 - s)).contiguous()
    bs = 0 if m.size(0) == 1 else m.stride(0)
    return m, bs, m.stride(1), s4


def _prefix_attention_impl(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
    mask: torch.Tensor | None, scaling: float, num_heads: int, num_kv_heads: int,
    quantize_out: bool = False, warm: list[torch.Tensor] | None = None, need_out: bool = True,
    kv_mfma: torch.Tensor | None = None,
):
    """(out, key states) or, with ``quantize_out`` (one KV head, 8 query heads), (out, key
    states, q codes, scales) of the output rows' K = 2048 activation quant.  ``warm``: up to
    four contiguous device tensors that the attention launch's idle workgroups read into
    the Infinity Cache (``pi05w4a4_prefix_attention_warm``).  ``need_out=False`` (with
    ``quantize_out``): the fp16 output is not written and an empty tensor is returned.
    ``kv_mfma``: K with RoPE and V^T already in the fragment-major layout (from
    ``rms_norm_int4_gemm3_rope``); k and v are then only checked for shape, the K/V prep
    launch is skipped and the key states are returned as None."""
    d = ATTN_HEAD_DIM
    for name, t in (("q", q), ("k", k), ("v", v), ("cos", cos), ("sin", sin)):
        if not t.is_cuda:
            raise RuntimeError(f"prefix_attention: {name} must be on CUDA/HIP")
        if t.dtype != torch.float16:
            raise RuntimeError(f"prefix_attention: {name} must be float16")
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise RuntimeError("prefix_attention expects q [B, S, H*256], k and v [B, S, KVH*256]")
    b, s = int(q.size(0)), int(q.size(1))
    h, kvh = int(num_heads), int(num_kv_heads)
    if q.size(2) != h * d or k.size(2) != kvh * d or tuple(k.shape[:2]) != (b, s):
        raise RuntimeError(f"prefix_attention: q {tuple(q.shape)} / k {tuple(k.shape)} do not match "
                           f"{h} query and {kvh} KV heads of {d}")
    qc, kc, vc = (t if t.is_contiguous() else t.contiguous() for t in (q, k, v))
    cs = _rope_tables(cos, sin, b, s)
    m, mbs, mrs, mlen = _attention_mask_arg(mask, b, s, q.device)
    lib = _lib if _lib is not None else load_int4_gemm()
    dev = q.device
    prepped = kv_mfma is not None
    if prepped:
        if kv_mfma.device != dev or kv_mfma.dtype != torch.float16 or kv_mfma.numel() != _kv_mfma_elems(lib, b, s, kvh, d):
            raise RuntimeError("prefix_attention: kv_mfma must be the fp16 fragment-major K/V^T of this call")
        k_rope = None
    else:
        k_rope = torch.empty((b, kvh, s, d), dtype=torch.float16, device=dev)
        kv_mfma = torch.empty(_kv_mfma_elems(lib, b, s, kvh, d), dtype=torch.float16, device=dev)
    if not (need_out or quantize_out):
        raise RuntimeError("prefix_attention: the output can only be dropped when it is quantized")
    out = torch.empty((b, s, h * d) if need_out else (0,), dtype=torch.float16, device=dev)
    out_ptr = _ptr(out) if need_out else None
    codes = scales = None
    if quantize_out:
        codes = torch.empty((_q_words(b * s, h * d),), dtype=torch.int32, device=dev)
        scales = torch.empty((b * s,), dtype=torch.float32, device=dev)
    with _on_device(dev):
        st = _stream(dev)
        if not prepped:
            _check(lib.pi05w4a4_attn_kv_prep(_ptr(kc), _ptr(vc), kvh * d, _ptr(cs[0]), _ptr(cs[1]), b, s, kvh, d,
                                             _ptr(k_rope), _ptr(kv_mfma), st), "pi05w4a4_attn_kv_prep")
        wa = _warm_args(warm, "prefix_attention") if warm else None
        if wa is not None:
            _check(lib.pi05w4a4_prefix_attention_warm(_ptr(qc), h * d, _ptr(kv_mfma), _ptr(cs[0]), _ptr(cs[1]),
                                                      _ptr(m), mbs, mrs, mlen, float(scaling), b, s, h, kvh, d,
                                                      out_ptr, h * d, _ptr(codes), _ptr(scales), *wa,
                                                      st), "pi05w4a4_prefix_attention_warm")
        else:
            _check(lib.pi05w4a4_prefix_attention(_ptr(qc), h * d, _ptr(kv_mfma), _ptr(cs[0]), _ptr(cs[1]),
                                                 _ptr(m), mbs, mrs, mlen, float(scaling), b, s, h, kvh, d,
                                                 out_ptr, h * d, _ptr(codes), _ptr(scales), st),
                   "pi05w4a4_prefix_attention")
    if quantize_out:
        return out, k_rope, codes, scales
    return out, k_rope


def _rope_tables(cos: torch.Tensor, sin: torch.Tensor, b: int, s: int) -> list[torch.Tensor]:
    return [t.expand(b, s, ATTN_HEAD_DIM).contiguous() if t.dim() == 3 else t.reshape(b, s, ATTN_HEAD_DIM).contiguous()
            for t in (cos, sin)]


def rope_pair_weight(w: torch.Tensor) -> torch.Tensor:
    """The K weight of ``rms_norm_int4_gemm3_rope``: an MFMA-layout K projection (N = 256
    output channels = one head of 256) with its 16-channel blocks in RoPE-pair order, so
    that one wave of the QKV GEMM holds the dimensions d and d + 128 that RoPE mixes
    (``pi05w4a4_permute_rope_pairs``)."""
    if w.dim() != 2 or int(w.size(0)) != ATTN_HEAD_DIM or w.dtype != torch.int32 or not w.is_cuda:
        raise RuntimeError("rope_pair_weight takes an int32 MFMA-layout K weight [256, K/8+16] on the GPU")
    k = (int(w.size(1)) - MFMA_MARKER_WORDS) * 8
    if not is_mfma_layout(w, k):
        raise RuntimeError("rope_pair_weight takes an MFMA-layout weight ([N, K/8+16])")
    src = w.contiguous()
    out = torch.zeros_like(src)
    lib = _lib if _lib is not None else load_int4_gemm()
    with _on_device(w.device):
        _check(lib.pi05w4a4_permute_rope_pairs(src.data_ptr(), k, out.data_ptr(), _stream(w.device)),
               "pi05w4a4_permute_rope_pairs")
    return out


def _rms_norm_qkv_rope_impl(x, norm_weight, eps, unit_offset, w_q, w_k_rope, w_v, cos, sin):
    """(q [B, S, Nq], key states with RoPE [B, 1, S, 256], v [B, S, 256], fragment-major K/V^T)
    of ``rms_norm_int4_gemm3`` plus the attention prep, from one norm + quant and one GEMM
    launch (``pi05w4a4_gemm_qkv_rope``)."""
    if x.dim() != 3:
        raise RuntimeError("rms_norm_int4_gemm3_rope expects x [B, S, 2048]")
    k = _check_x(x)
    for name, w in (("q", w_q), ("k", w_k_rope), ("v", w_v)):
        _check_packed(w, k, f"{name} weight")
        if not is_mfma_layout(w, k):
            raise RuntimeError(f"rms_norm_int4_gemm3_rope takes MFMA-layout weights ({name})")
    if int(w_k_rope.size(0)) != ATTN_HEAD_DIM or int(w_v.size(0)) != ATTN_HEAD_DIM:
        raise RuntimeError("rms_norm_int4_gemm3_rope needs one KV head of 256")
    b, s = int(x.size(0)), int(x.size(1))
    for name, t in (("cos", cos), ("sin", sin)):
        if not t.is_cuda or t.dtype != torch.float16 or t.device != x.device:
            raise RuntimeError(f"rms_norm_int4_gemm3_rope: {name} must be float16 on {x.device}")
    q, sa = rms_norm_quantize(x, norm_weight, eps, unit_offset, warm=_norm_warm([w_q, w_k_rope, w_v], x))
    return _gemm_qkv_rope(q, sa, k, w_q, w_k_rope, w_v, _rope_tables(cos, sin, b, s), b, s, x.device)


def _gemm_qkv_rope(q, sa, k, w_q, w_k_rope, w_v, cs, b, s, dev):
    """The GEMM launch of rms_norm_int4_gemm3_rope on quantized activations."""
    lib = _lib if _lib is not None else load_int4_gemm()
    m = b * s
    nq = int(w_q.size(0))
    yq = torch.empty((b, s, nq), dtype=torch.float16, device=dev)
    k_rope = torch.empty((b, 1, s, ATTN_HEAD_DIM), dtype=torch.float16, device=dev)
    yv = torch.empty((b, s, ATTN_HEAD_DIM), dtype=torch.float16, device=dev)
    kv = torch.empty(_kv_mfma_elems(lib, b, s, 1, ATTN_HEAD_DIM), dtype=torch.float16, device=dev)
    with _on_device(dev):
        _check(lib.pi05w4a4_gemm_qkv_rope(q.data_ptr(), sa.data_ptr(), m, k, w_q.data_ptr(), nq, w_k_rope.data_ptr(),
                                          w_v.data_ptr(), cs[0].data_ptr(), cs[1].data_ptr(), b, s, yq.data_ptr(),
                                          k_rope.data_ptr(), yv.data_ptr(), kv.data_ptr(), _stream(dev)),
               "pi05w4a4_gemm_qkv_rope")
    return yq, k_rope, yv, kv


def _prefix_attention_o_proj_impl(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads, w_o, residual,
                                  warm=None, return_out=True, kv_mfma=None):
    """RoPE + attention + o_proj + residual add: with one KV head and 8 query heads of 256
    the attention kernel quantizes its own output rows for the o GEMM; otherwise the output
    goes through the separate quantizer.  Returns (residual + o_proj(out), key states, out);
    with ``return_out=False`` and the in-kernel quant, out is not written (an empty
    tensor)."""
    k_in = ATTN_HEAD_DIM * int(num_heads)
    _check_packed(w_o, k_in, "o_proj weight")
    lead = tuple(q.shape[:-1])
    _check_residual(residual, q.device, (*lead, int(w_o.size(0))))  # before any launch
    w, n_true = _as_mfma(w_o, k_in, tiled=False)
    if int(num_kv_heads) == 1 and k_in == 2048:
        out, k_rope, codes, scales = _prefix_attention_impl(q, k, v, cos, sin, mask, scaling, num_heads,
                                                            num_kv_heads, quantize_out=True, warm=warm,
                                                            need_out=return_out, kv_mfma=kv_mfma)
        with _on_device(q.device):
            y = _gemm_from_q(codes, scales, k_in, [(w, n_true)], lead, q.device, "int4_gemm", residual=residual)[0]
        return y, k_rope, out
    out, k_rope = _prefix_attention_impl(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads, warm=warm,
                                         kv_mfma=kv_mfma)
    return _run(out, [w_o], tiled=False, kind="int4_gemm", residual=residual)[0], k_rope, out


# ----------------------------------------------------------------------------- custom ops
def _register_custom_op() -> None:
    global _op_registered
    if _op_registered:
        return
    try:
        torch.ops.pi05_w4a4.prefix_attention_o_proj_kv
        _op_registered = True
        return
    except (AttributeError, RuntimeError):
        pass

    def _fake_out(x: torch.Tensor, packed: torch.Tensor) -> torch.Tensor:
        return torch.empty(*x.shape[:-1], packed.shape[0], device=x.device, dtype=torch.float16)

    @torch.library.custom_op("pi05_w4a4::int4_gemm", mutates_args=())
    def _int4_gemm(x: torch.Tensor, packed: torch.Tensor) -> torch.Tensor:
        return _run(x, [packed], tiled=False, kind="gemm")[0]

    @_int4_gemm.register_fake
    def _int4_gemm_fake(x: torch.Tensor, packed: torch.Tensor) -> torch.Tensor:
        return _fake_out(x, packed)

    @torch.library.custom_op("pi05_w4a4::int4_gemm_tiled", mutates_args=())
    def _int4_gemm_tiled(x: torch.Tensor, packed: torch.Tensor) -> torch.Tensor:
        return _run(x, [packed], tiled=True, kind="gemm")[0]

    @_int4_gemm_tiled.register_fake
    def _int4_gemm_tiled_fake(x: torch.Tensor, packed: torch.Tensor) -> torch.Tensor:
        return _fake_out(x, packed)

    @torch.library.custom_op("pi05_w4a4::int4_gemm2", mutates_args=())
    def _int4_gemm2(
        x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        a, b = _run(x, [w0, w1], tiled=False, kind="gemm2")
        return a, b

    @_int4_gemm2.register_fake
    def _int4_gemm2_fake(x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor):
        return _fake_out(x, w0), _fake_out(x, w1)

    @torch.library.custom_op("pi05_w4a4::int4_gemm2_tiled", mutates_args=())
    def _int4_gemm2_tiled(
        x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        a, b = _run(x, [w0, w1], tiled=True, kind="gemm2")
        return a, b

    @_int4_gemm2_tiled.register_fake
    def _int4_gemm2_tiled_fake(x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor):
        return _fake_out(x, w0), _fake_out(x, w1)

    @torch.library.custom_op("pi05_w4a4::int4_gemm3", mutates_args=())
    def _int4_gemm3(
        x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        a, b, c = _run(x, [w0, w1, w2], tiled=False, kind="gemm3")
        return a, b, c

    @_int4_gemm3.register_fake
    def _int4_gemm3_fake(x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor):
        return _fake_out(x, w0), _fake_out(x, w1), _fake_out(x, w2)

    # Not in the reference: gate/up GEMMs with the GELU-tanh(gate) * up epilogue fused.
    @torch.library.custom_op("pi05_w4a4::int4_gemm2_gelu", mutates_args=())
    def _int4_gemm2_gelu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
        _check_gelu_weights(x, w_gate, w_up)
        return _run(x, [w_gate, w_up], tiled=False, kind="gemm2_gelu", gelu=True)[0]

    @_int4_gemm2_gelu.register_fake
    def _int4_gemm2_gelu_fake(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor):
        return _fake_out(x, w_gate)

    # Not in the reference: the decoder's RMSNorm (transformers GemmaRMSNorm) in one kernel.
    @torch.library.custom_op("pi05_w4a4::rms_norm", mutates_args=())
    def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, unit_offset: bool) -> torch.Tensor:
        return _rms_norm_impl(x, weight, eps, unit_offset)

    @_rms_norm.register_fake
    def _rms_norm_fake(x: torch.Tensor, weight: torch.Tensor, eps: float, unit_offset: bool):
        return torch.empty_like(x)

    # Not in the reference: the decoder's RMSNorm fused into the QKV / gate-up activation
    # quant, and the residual add fused into the o / down GEMM epilogue.
    @torch.library.custom_op("pi05_w4a4::rms_norm_int4_gemm3", mutates_args=())
    def _rms_norm_int4_gemm3(
        x: torch.Tensor, norm_weight: torch.Tensor, eps: float, unit_offset: bool,
        w0: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        a, b, c = _run(x, [w0, w1, w2], tiled=False, kind="int4_gemm3", norm=(norm_weight, eps, unit_offset),
                       warm=_norm_warm([w0, w1, w2], x))
        return a, b, c

    @_rms_norm_int4_gemm3.register_fake
    def _rms_norm_int4_gemm3_fake(x, norm_weight, eps, unit_offset, w0, w1, w2):
        return _fake_out(x, w0), _fake_out(x, w1), _fake_out(x, w2)

    @torch.library.custom_op("pi05_w4a4::rms_norm_int4_gemm2_gelu", mutates_args=())
    def _rms_norm_int4_gemm2_gelu(
        x: torch.Tensor, norm_weight: torch.Tensor, eps: float, unit_offset: bool,
        w_gate: torch.Tensor, w_up: torch.Tensor,
    ) -> torch.Tensor:
        _check_gelu_weights(x, w_gate, w_up)
        return _run(x, [w_gate, w_up], tiled=False, kind="int4_gemm2_gelu", gelu=True,
                    norm=(norm_weight, eps, unit_offset), warm=_gate_up_warm(w_up, x))[0]

    @_rms_norm_int4_gemm2_gelu.register_fake
    def _rms_norm_int4_gemm2_gelu_fake(x, norm_weight, eps, unit_offset, w_gate, w_up):
        return _fake_out(x, w_gate)

    @torch.library.custom_op("pi05_w4a4::int4_gemm_residual", mutates_args=())
    def _int4_gemm_residual(x: torch.Tensor, packed_w: torch.Tensor, residual: torch.Tensor,
                            warm: list[torch.Tensor]) -> torch.Tensor:
        return _run(x, [packed_w], tiled=False, kind="int4_gemm", residual=residual, warm=warm)[0]

    @_int4_gemm_residual.register_fake
    def _int4_gemm_residual_fake(x, packed_w, residual, warm):
        return _fake_out(x, packed_w)

    # Not in the reference: the Gemma MLP block (post norm, gate/up + GELU*up with the down
    # projection's activation quant in the same launch, down + residual); returns (y, h).
    @torch.library.custom_op("pi05_w4a4::rms_norm_int4_mlp", mutates_args=())
    def _rms_norm_int4_mlp(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, unit_offset: bool,
                           w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor, residual: torch.Tensor,
                           warm: list[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor]:
        return _rms_norm_mlp_impl(x, norm_weight, eps, unit_offset, w_gate, w_up, w_down, residual, warm)

    @_rms_norm_int4_mlp.register_fake
    def _rms_norm_int4_mlp_fake(x, norm_weight, eps, unit_offset, w_gate, w_up, w_down, residual, warm):
        return _fake_out(x, w_down), _fake_out(x, w_gate)

    # Not in the reference: RoPE + attention between int4_gemm3 and o_proj in two kernels.
    @torch.library.custom_op("pi05_w4a4::prefix_attention", mutates_args=())
    def _prefix_attention(
        q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
        mask: torch.Tensor | None, scaling: float, num_heads: int, num_kv_heads: int,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        return _prefix_attention_impl(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads)

    @_prefix_attention.register_fake
    def _prefix_attention_fake(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads):
        b, s = q.shape[0], q.shape[1]
        out = q.new_empty((b, s, num_heads * ATTN_HEAD_DIM))
        return out, q.new_empty((b, num_kv_heads, s, ATTN_HEAD_DIM))

    @torch.library.custom_op("pi05_w4a4::prefix_attention_o_proj", mutates_args=())
    def _prefix_attention_o_proj(
        q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
        mask: torch.Tensor | None, scaling: float, num_heads: int, num_kv_heads: int,
        w_o: torch.Tensor, residual: torch.Tensor, warm: list[torch.Tensor], return_out: bool,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return _prefix_attention_o_proj_impl(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads, w_o,
                                             residual, warm, return_out)

    @_prefix_attention_o_proj.register_fake
    def _prefix_attention_o_proj_fake(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads, w_o, residual, warm,
                                      return_out):
        b, s = q.shape[0], q.shape[1]
        dropped = not return_out and num_kv_heads == 1 and num_heads * ATTN_HEAD_DIM == 2048
        return (q.new_empty((b, s, w_o.shape[0])), q.new_empty((b, num_kv_heads, s, ATTN_HEAD_DIM)),
                q.new_empty((0,) if dropped else (b, s, num_heads * ATTN_HEAD_DIM)))

    # Not in the reference: the QKV GEMMs with RoPE and the attention's K/V layout in the
    # epilogue, and the attention + o_proj that reads them (no K/V prep launch).
    @torch.library.custom_op("pi05_w4a4::rms_norm_int4_gemm3_rope", mutates_args=())
    def _rms_norm_int4_gemm3_rope(
        x: torch.Tensor, norm_weight: torch.Tensor, eps: float, unit_offset: bool,
        w_q: torch.Tensor, w_k_rope: torch.Tensor, w_v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        return _rms_norm_qkv_rope_impl(x, norm_weight, eps, unit_offset, w_q, w_k_rope, w_v, cos, sin)

    @_rms_norm_int4_gemm3_rope.register_fake
    def _rms_norm_int4_gemm3_rope_fake(x, norm_weight, eps, unit_offset, w_q, w_k_rope, w_v, cos, sin):
        b, s = x.shape[0], x.shape[1]
        s_pad = (s + 63) // 64 * 64
        return (x.new_empty((b, s, w_q.shape[0])), x.new_empty((b, 1, s, ATTN_HEAD_DIM)),
                x.new_empty((b, s, ATTN_HEAD_DIM)), x.new_empty((b * 2 * s_pad * ATTN_HEAD_DIM,)))

    @torch.library.custom_op("pi05_w4a4::prefix_attention_o_proj_kv", mutates_args=())
    def _prefix_attention_o_proj_kv(
        q: torch.Tensor, v: torch.Tensor, kv_mfma: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
        mask: torch.Tensor | None, scaling: float, num_heads: int, w_o: torch.Tensor, residual: torch.Tensor,
        warm: list[torch.Tensor], return_out: bool,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        y, _, out = _prefix_attention_o_proj_impl(q, v, v, cos, sin, mask, scaling, num_heads, 1, w_o, residual,
                                                  warm, return_out, kv_mfma=kv_mfma)
        return y, out

    @_prefix_attention_o_proj_kv.register_fake
    def _prefix_attention_o_proj_kv_fake(q, v, kv_mfma, cos, sin, mask, scaling, num_heads, w_o, residual, warm,
                                         return_out):
        b, s = q.shape[0], q.shape[1]
        dropped = not return_out and num_heads * ATTN_HEAD_DIM == 2048
        return (q.new_empty((b, s, w_o.shape[0])),
                q.new_empty((0,) if dropped else (b, s, num_heads * ATTN_HEAD_DIM)))

    _op_registered = True


_register_custom_op()


# Eager calls skip the torch.ops dispatcher (tens of microseconds of host time per call,
# several per decoder layer) when nothing needs it: plain tensors, no autograd graph to
# record, no Dynamo trace, no torch.jit.trace (whose graph only sees dispatched ops), no
# dispatch or function mode.  The direct and the dispatched route run the same
# implementation.
_is_compiling = torch.compiler.is_compiling
_jit_tracing = torch._C._get_tracing_state
_dispatch_modes = torch._C._len_torch_dispatch_stack
_function_modes = torch._C._is_torch_function_mode_enabled
_PLAIN = (torch.Tensor, torch.nn.Parameter)


def _direct(*ts) -> bool:
    if _is_compiling() or _jit_tracing() is not None or _dispatch_modes() or _function_modes():
        return False
    grad = torch.is_grad_enabled()
    for t in ts:
        if t is not None and (type(t) not in _PLAIN or (grad and t.requires_grad)):
            return False
    return True


def int4_gemm(x: torch.Tensor, packed_w: torch.Tensor) -> torch.Tensor:
    """Compiled-graph-friendly INT4 GEMM. x: fp16 [..., K], packed: int32 [N, K/8+1|+P|+16]."""
    if _direct(x, packed_w):
        return _run(x, [packed_w], tiled=False, kind="gemm")[0]
    return torch.ops.pi05_w4a4.int4_gemm(x, packed_w)


def int4_gemm_tiled(x: torch.Tensor, packed_w: torch.Tensor) -> torch.Tensor:
    """INT4 GEMM with fragment-major weights (WMMA-tiled K/8+9 or MFMA K/8+16)."""
    if _direct(x, packed_w):
        return _run(x, [packed_w], tiled=True, kind="gemm")[0]
    return torch.ops.pi05_w4a4.int4_gemm_tiled(x, packed_w)


def int4_gemm2(x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Shared activation quant plus two INT4 GEMMs (one launch)."""
    if _direct(x, w0, w1):
        return tuple(_run(x, [w0, w1], tiled=False, kind="gemm2"))
    return torch.ops.pi05_w4a4.int4_gemm2(x, w0, w1)


def int4_gemm2_tiled(x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Shared activation quant plus two fragment-major INT4 GEMMs."""
    if _direct(x, w0, w1):
        return tuple(_run(x, [w0, w1], tiled=True, kind="gemm2"))
    return torch.ops.pi05_w4a4.int4_gemm2_tiled(x, w0, w1)


def int4_gemm3(
    x: torch.Tensor, w0: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Shared activation quant plus three INT4 GEMMs (QKV, one launch)."""
    if _direct(x, w0, w1, w2):
        return tuple(_run(x, [w0, w1, w2], tiled=False, kind="gemm3"))
    return torch.ops.pi05_w4a4.int4_gemm3(x, w0, w1, w2)


def int4_gemm2_gelu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """h = gelu_tanh(x @ W_gate^T) * (x @ W_up^T) with one shared activation quant."""
    if _direct(x, w_gate, w_up):
        _check_gelu_weights(x, w_gate, w_up)
        return _run(x, [w_gate, w_up], tiled=False, kind="gemm2_gelu", gelu=True)[0]
    return torch.ops.pi05_w4a4.int4_gemm2_gelu(x, w_gate, w_up)


def int4_gemm_acc(x: torch.Tensor, packed_w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Debug: (int32 accumulators [M, N], codes q (fragment-major, see ``quantize``),
    scales sa [M]) for bit-exact checks."""
    k = _check_x(x)
    _check_packed(packed_w, k)
    q, sa = quantize(x)
    w, n_true = _as_mfma(packed_w, k, tiled=packed_w.size(1) == k // 8 + WMMA_MARKER_WORDS)
    m = int(sa.size(0))
    acc = torch.empty((m, int(w.size(0))), dtype=torch.int32, device=x.device)
    lib = load_int4_gemm()
    with torch.cuda.device(x.device):
        _check(lib.pi05w4a4_gemm_acc(_ptr(q), m, k, _ptr(w), int(w.size(0)), _ptr(acc),
                                     _stream(x.device)), "pi05w4a4_gemm_acc")
    return acc[:, :n_true], q, sa


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, unit_offset: bool = True) -> torch.Tensor:
    """RMSNorm over the last dim in one kernel: fp16((x * rsqrt(mean(x^2) + eps)) *
    (unit_offset + weight)), fp32 inside (transformers GemmaRMSNorm semantics when
    ``unit_offset``)."""
    if _direct(x, weight):
        return _rms_norm_impl(x, weight, float(eps), bool(unit_offset))
    return torch.ops.pi05_w4a4.rms_norm(x, weight, float(eps), bool(unit_offset))


def rms_norm_int4_gemm3(x, norm_weight, eps, w0, w1, w2, unit_offset=True):
    """int4_gemm3 of rms_norm(x): the decoder's input norm fused into the QKV activation
    quant (K = 2048)."""
    if _direct(x, norm_weight, w0, w1, w2):
        return tuple(_run(x, [w0, w1, w2], tiled=False, kind="int4_gemm3",
                          norm=(norm_weight, float(eps), bool(unit_offset)),
                          warm=_norm_warm([w0, w1, w2], x)))
    return torch.ops.pi05_w4a4.rms_norm_int4_gemm3(x, norm_weight, float(eps), bool(unit_offset), w0, w1, w2)


def rms_norm_int4_gemm2_gelu(x, norm_weight, eps, w_gate, w_up, unit_offset=True):
    """int4_gemm2_gelu of rms_norm(x): the post-attention norm fused into the gate/up
    activation quant (K = 2048)."""
    if _direct(x, norm_weight, w_gate, w_up):
        _check_gelu_weights(x, w_gate, w_up)
        return _run(x, [w_gate, w_up], tiled=False, kind="int4_gemm2_gelu", gelu=True,
                    norm=(norm_weight, float(eps), bool(unit_offset)), warm=_gate_up_warm(w_up, x))[0]
    return torch.ops.pi05_w4a4.rms_norm_int4_gemm2_gelu(x, norm_weight, float(eps), bool(unit_offset),
                                                        w_gate, w_up)


def rms_norm_int4_mlp(x, norm_weight, eps, w_gate, w_up, w_down, residual, warm=None, unit_offset=True):
    """The decoder's MLP block, residual + down(gelu_tanh(gate(n)) * up(n)) with
    n = rms_norm(x), on W4A4 ops: the norm fused into the gate/up activation quant, the
    GELU-tanh*up epilogue, the down projection's activation quant in the gate/up launch
    (``pi05w4a4_gemm_gelu_up_quant``) and the residual add in the down epilogue.  MFMA-layout
    weights; ``warm``: buffers read into the Infinity Cache by the quant workgroups that
    find no row left (the down weights, say).  Returns (y, h) with h = the fp16 GELU*up
    output that the down projection quantized."""
    if _direct(x, norm_weight, w_gate, w_up, w_down, residual):
        return _rms_norm_mlp_impl(x, norm_weight, float(eps), bool(unit_offset), w_gate, w_up, w_down, residual,
                                  warm)
    return torch.ops.pi05_w4a4.rms_norm_int4_mlp(x, norm_weight, float(eps), bool(unit_offset), w_gate, w_up,
                                                 w_down, residual, list(warm or []))


def int4_gemm_residual(x: torch.Tensor, packed_w: torch.Tensor, residual: torch.Tensor,
                       warm: list[torch.Tensor] | None = None) -> torch.Tensor:
    """residual + int4_gemm(x, packed_w), the add done in the GEMM epilogue with the
    rounding of the eager fp16 add (MFMA-layout or row-major weights, N % 16 == 0).
    ``warm``: up to four device tensors that the K = 16384 activation quant's idle
    workgroup slots read into the Infinity Cache (``pi05w4a4_quantize_warm``; results
    unchanged)."""
    if _direct(x, packed_w, residual):
        return _run(x, [packed_w], tiled=False, kind="int4_gemm", residual=residual, warm=warm)[0]
    return torch.ops.pi05_w4a4.int4_gemm_residual(x, packed_w, residual, list(warm or []))


def prefix_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
    mask: torch.Tensor | None, scaling: float, num_heads: int, num_kv_heads: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE + attention of the prefix LM (head_dim 256, fp16, at most 1024 tokens).

    q [B, S, H*256], k and v [B, S, KVH*256] as int4_gemm3 returns them (before RoPE),
    cos/sin [B, S, 256] (the decoder's position embeddings), mask None or additive fp16
    [B|1, 1, S, >=S].  Returns (attention output [B, S, H*256], key states with RoPE
    [B, KVH, S, 256]): transformers' apply_rotary_pos_emb + eager_attention_forward, the
    key states bit-identical to the eager ones."""
    if _direct(q, k, v, cos, sin, mask):
        return _prefix_attention_impl(q, k, v, cos, sin, mask, float(scaling), int(num_heads), int(num_kv_heads))
    return torch.ops.pi05_w4a4.prefix_attention(q, k, v, cos, sin, mask, float(scaling), int(num_heads),
                                                int(num_kv_heads))


def prefix_attention_o_proj(q, k, v, cos, sin, mask, scaling, num_heads, num_kv_heads, w_o, residual, warm=None,
                            return_out=True):
    """residual + o_proj(attention(q, k, v)) of a prefix forward, plus the RoPE'd key
    states and the attention output: ``prefix_attention`` followed by
    ``int4_gemm_residual``, with the o-proj activation quant done inside the attention
    kernel when the layer has one KV head and 8 query heads of 256 (PaliGemma).  ``warm``:
    up to four weight tensors of the following ops that the attention launch's idle CUs
    read into the Infinity Cache (results unchanged).  ``return_out=False``: a caller that
    does not use the attention output gets an empty tensor in its place, and the kernel
    skips writing it when it quantizes the output itself."""
    if _direct(q, k, v, cos, sin, mask, w_o, residual):
        return _prefix_attention_o_proj_impl(q, k, v, cos, sin, mask, float(scaling), int(num_heads),
                                             int(num_kv_heads), w_o, residual, warm, bool(return_out))
    return torch.ops.pi05_w4a4.prefix_attention_o_proj(q, k, v, cos, sin, mask, float(scaling), int(num_heads),
                                                       int(num_kv_heads), w_o, residual, list(warm or []),
                                                       bool(return_out))


def rms_norm_int4_gemm3_rope(x, norm_weight, eps, w_q, w_k_rope, w_v, cos, sin, unit_offset=True):
    """``rms_norm_int4_gemm3`` for one KV head of 256 with the attention prep in the GEMM
    epilogue: (q [B, S, Nq], key states with RoPE [B, 1, S, 256], v [B, S, 256], K/V^T in
    the attention kernel's fragment-major layout).  ``w_k_rope`` is ``rope_pair_weight`` of
    the K weight; S must be a multiple of 8 (at most 1024).  The key states are the eager
    ``apply_rotary_pos_emb`` keys bit for bit, as ``prefix_attention`` returns them."""
    if _direct(x, norm_weight, w_q, w_k_rope, w_v, cos, sin):
        return _rms_norm_qkv_rope_impl(x, norm_weight, float(eps), bool(unit_offset), w_q, w_k_rope, w_v, cos, sin)
    return torch.ops.pi05_w4a4.rms_norm_int4_gemm3_rope(x, norm_weight, float(eps), bool(unit_offset), w_q, w_k_rope,
                                                        w_v, cos, sin)


def prefix_attention_o_proj_kv(q, v, kv_mfma, cos, sin, mask, scaling, num_heads, w_o, residual, warm=None,
                               return_out=True):
    """``prefix_attention_o_proj`` for one KV head with K and V^T already laid out by
    ``rms_norm_int4_gemm3_rope`` (no K/V prep launch): (residual + o_proj(attention), out)."""
    if _direct(q, v, kv_mfma, cos, sin, mask, w_o, residual):
        y, _, out = _prefix_attention_o_proj_impl(q, v, v, cos, sin, mask, float(scaling), int(num_heads), 1, w_o,
                                                  residual, warm, bool(return_out), kv_mfma=kv_mfma)
        return y, out
    return torch.ops.pi05_w4a4.prefix_attention_o_proj_kv(q, v, kv_mfma, cos, sin, mask, float(scaling),
                                                          int(num_heads), w_o, residual, list(warm or []),
                                                          bool(return_out))


def preload() -> None:
    """Load the HIP library before torch.compile traces the graph."""
    load_int4_gemm()
    _register_custom_op()
