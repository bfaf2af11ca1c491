"""CPU oracle for the W4A4 prefix-LM GEMM path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference's CPU semantics of the W4A4 path
(``pi05_fast/w4a4/pack.py``) plus the fused-op call sequences and dequant epilogue of
``pi05_fast/w4a4/csrc/int4_gemm.cu``.  It is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it.  The product path (``pi05_fast.w4a4`` ops) never imports, calls or links
anything under ``oracle/`` and raises when its HIP library is missing.

Pinning (each function is checked by ``tests/test_oracle.py``):
  * ``fwht_unnormalized``   golden vectors from the reference + closed form
                            H[i,j] = (-1)^popcount(i&j) (float64 brute force), H.H = K.I,
                            exactness on small-integer inputs.
  * ``pack_nibbles`` / ``unpack_nibbles``  golden vectors + hand-built known answers
                            (codes 0..7 -> 0x76543210, -8..-1 -> 0xFEDCBA98).
  * ``quant_activation``    golden vectors (codes and scale bits, K in {64..16384})
                            + hand-built half-even ties, zero rows, one-hot rows.
  * ``pack_linear_weight``  golden vectors (payload and scale bits).
  * ``preshuffle_wmma_weight`` golden vector + inverse round trip.
  * ``int4_gemm_ref`` / ``gemm_acc_int32``  golden vectors + int64 brute force.
  * ``dequant_fp16``        golden vectors through ``int4_gemm_ref``.
  * ``gelu_tanh``           torch.nn.functional.gelu(approximate="tanh") in float64 on the CPU
                            (transformers' GELUTanh, the reference MLP's act_fn), to 1e-15
                            relative plus the float64 cancellation of 1 + tanh near -1;
                            a wrong constant or the erf form fails it.
  * ``rms_norm_lanes``      transformers' GemmaRMSNorm (torch fp32 on the CPU) to one fp16
                            ulp; constant rows (closed form); the wave-order sum against
                            float64 (it is a restatement of an fp32 summation order, so
                            only its order, not its arithmetic, is ours).
"""

from __future__ import annotations

import math

import numpy as np

ROTATE_K = frozenset({1024, 2048, 16384})  # pi05_fast/w4a4/pack.py:14
WMMA_PRESHUFFLE_PAD_WORDS = 9               # pi05_fast/w4a4/pack.py:15


def should_rotate(k: int, rotate: bool | None = None) -> bool:
    """pi05_fast/w4a4/pack.py:79-82 (the GPU decides by K alone, int4_gemm.cu:520-527)."""
    if rotate is not None:
        return bool(rotate)
    return k in ROTATE_K


def inv_sqrt_k(k: int) -> np.float32:
    """fp32(1/sqrt(K)) as torch forms it from the Python double (pack.py:96,124)."""
    return np.float32(1.0 / math.sqrt(k))


def fwht_unnormalized(x: np.ndarray) -> np.ndarray:
    """Unnormalised Sylvester FWHT along the last axis in fp32 (pack.py:18-31).

    Stage h = 1, 2, 4, ... pairs element i (bit h clear) with i + h and writes
    (a + b, a - b); every add/sub is one fp32 rounding.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    if n <= 0 or (n & (n - 1)) != 0:
        raise ValueError(f"FWHT length must be a power of 2, got {n}")
    lead = x.shape[:-1]
    out = x.copy()
    h = 1
    while h < n:
        v = out.reshape(*lead, n // (2 * h), 2, h)
        a = v[..., 0, :]
        b = v[..., 1, :]
        out = np.stack((a + b, a - b), axis=-2).reshape(*lead, n)
        h *= 2
    return out


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """codes [..., K] -> int32 words [..., K/8]; element 8p+j at bits 4j..4j+3 (pack.py:34-42)."""
    q = np.asarray(q)
    if q.shape[-1] % 8 != 0:
        raise ValueError(f"K must be a multiple of 8, got {q.shape[-1]}")
    q = q.astype(np.int64).reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    word = np.zeros(q.shape[:-1], dtype=np.int64)
    for j in range(8):
        word |= (q[..., j] & 0xF) << (4 * j)
    return word.astype(np.uint32).view(np.int32)


def unpack_nibbles(packed: np.ndarray, k: int) -> np.ndarray:
    """int32 words [..., K/8] -> int32 codes [..., K]; nibble >= 8 means value - 16 (pack.py:71-76)."""
    p = np.asarray(packed).astype(np.int32).view(np.uint32).astype(np.int64)
    out = np.empty(p.shape + (8,), dtype=np.int32)
    for j in range(8):
        nib = (p >> (4 * j)) & 0xF
        out[..., j] = np.where(nib >= 8, nib - 16, nib)
    return out.reshape(*p.shape[:-1], k)


def pack_linear_weight(weight: np.ndarray, rotate: bool | None = None) -> np.ndarray:
    """Linear.weight [N, K] fp32 -> int32 [N, K/8+1], scale bits in word K/8 (pack.py:85-101)."""
    w = np.asarray(weight, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError(f"expected 2D weight, got {w.shape}")
    n, k = w.shape
    if k % 64 != 0:
        raise ValueError(f"K must be a multiple of 64 for gemm_iu4, got {k}")
    if should_rotate(k, rotate):
        w = fwht_unnormalized(w) * inv_sqrt_k(k)
    amax = np.maximum(np.abs(w).max(axis=-1), np.float32(1e-12))
    scale = (amax / np.float32(7.0)).astype(np.float32)
    q = np.clip(np.rint(w / scale[:, None]), -7, 7).astype(np.int32)
    packed = pack_nibbles(q)
    return np.concatenate([packed, scale.view(np.int32)[:, None]], axis=1)


def unpack_linear_weight(packed: np.ndarray) -> tuple[np.ndarray, np.ndarray, int]:
    """int32 [N, K/8+1] -> (codes [N, K], scale fp32 [N], K) (pack.py:104-110)."""
    packed = np.asarray(packed, dtype=np.int32)
    k = (packed.shape[1] - 1) * 8
    q = unpack_nibbles(packed[:, :-1], k)
    scale = np.ascontiguousarray(packed[:, -1]).view(np.float32)
    return q, scale, k


def quant_activation(x: np.ndarray, rotate: bool | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Per-token symmetric INT4 activation quant (pack.py:113-131; int4_gemm.cu:396-477).

    x fp16 [M, K] -> (codes int8 [M, K] in [-7, 7], scale fp32 [M]).
    sdiv = amax/7 + 1e-12 (fp32); codes = clamp(rint_half_even(x'/sdiv), -7, 7);
    scale = sdiv * fp32(1/sqrt(K)) when rotating, else sdiv.
    """
    xf = np.asarray(x).astype(np.float32)
    if xf.ndim != 2:
        raise ValueError("quant_activation expects [M, K]")
    k = xf.shape[1]
    rot = should_rotate(k, rotate)
    if rot:
        xf = fwht_unnormalized(xf)
    amax = np.abs(xf).max(axis=-1) if k else np.zeros(xf.shape[0], np.float32)
    sdiv = (amax / np.float32(7.0) + np.float32(1e-12)).astype(np.float32)
    scale = (sdiv * inv_sqrt_k(k)).astype(np.float32) if rot else sdiv
    q = np.clip(np.rint(xf / sdiv[:, None]), -7, 7).astype(np.int8)
    return q, scale


def gemm_acc_int32(q_a: np.ndarray, q_w: np.ndarray) -> np.ndarray:
    """acc[m, n] = sum_k q_a[m, k] * q_w[n, k], exact.

    The reference forms it as an fp32 matmul of the codes (pack.py:143), which is exact
    because |acc| <= 64*K < 2^24 for K <= 16384 * 2; here the fp32 BLAS product is
    converted back to int32 (every partial sum is an integer below 2^24, so no rounding
    can occur in any order).
    """
    a = np.asarray(q_a, dtype=np.float32)
    b = np.asarray(q_w, dtype=np.float32)
    if a.shape[1] * 64 >= (1 << 24):
        raise ValueError("K too large for an exact fp32 accumulation")
    return (a @ b.T).astype(np.int32)


def dequant_fp16(acc: np.ndarray, s_a: np.ndarray, s_w: np.ndarray) -> np.ndarray:
    """y = fp16_rne((fp32(acc) * s_a[m]) * s_w[n]) (int4_gemm.cu:199-200; pack.py:144-145)."""
    y = acc.astype(np.float32) * np.asarray(s_a, np.float32)[:, None]
    y = y * np.asarray(s_w, np.float32)[None, :]
    return y.astype(np.float16)


def int4_gemm_ref(x: np.ndarray, packed_w: np.ndarray, rotate: bool | None = None) -> np.ndarray:
    """CPU reference for one W4A4 linear (pack.py:134-145): x fp16 [..., K] -> y fp16 [..., N]."""
    x = np.asarray(x)
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    q_a, s_a = quant_activation(x2, rotate=rotate)
    q_w, s_w, k_w = unpack_linear_weight(packed_w)
    if k_w != k:
        raise ValueError(f"K mismatch act={k} weight={k_w}")
    y = dequant_fp16(gemm_acc_int32(q_a, q_w), s_a, s_w)
    return y.reshape(*x.shape[:-1], packed_w.shape[0])


def preshuffle_wmma_weight(packed: np.ndarray, k: int) -> np.ndarray:
    """Layout L3: flat[(t*N + n)*2 + h] = L1[n, 2t + h], scales at flat[N*K/8 + n] (pack.py:45-68)."""
    packed = np.asarray(packed, dtype=np.int32)
    n = packed.shape[0]
    words = k // 8
    if k % 16 != 0 or packed.shape[1] < words + 1:
        raise ValueError(f"invalid packed weight shape {packed.shape} for K={k}")
    out = np.zeros((n, words + WMMA_PRESHUFFLE_PAD_WORDS), dtype=np.int32)
    flat = out.reshape(-1)
    payload = packed[:, :words].reshape(n, words // 2, 2).transpose(1, 0, 2)
    flat[: n * words] = payload.reshape(-1)
    flat[n * words : n * words + n] = packed[:, words]
    return out


def unshuffle_wmma_weight(tiled: np.ndarray, k: int) -> np.ndarray:
    """Inverse of ``preshuffle_wmma_weight`` back to L1 [N, K/8+1] (tests/test_w4a4.py:24-42)."""
    n = tiled.shape[0]
    words = k // 8
    flat = np.asarray(tiled, dtype=np.int32).reshape(-1)
    payload = flat[: n * words].reshape(words // 2, n, 2).transpose(1, 0, 2).reshape(n, words)
    return np.concatenate([payload, flat[n * words : n * words + n, None]], axis=1)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """GELU, tanh approximation, in float64: the reference MLP's act_fn (apply.py:135-138,
    transformers' GELUTanh = F.gelu(approximate='tanh')).  The GPU's fused GELU*up is
    checked bit for bit against torch's eager fp16 ops on the same GPU instead (every fp16
    gate); this float64 form serves tolerance checks."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x**3)))


def rms_norm_lanes(x: np.ndarray, weight: np.ndarray, eps: float, unit_offset: bool = True,
                   lanes: int = 64) -> np.ndarray:
    """GemmaRMSNorm (transformers modeling_gemma.py:64-78: fp32 inside, (1 + w), fp16
    out) in the fp32 summation order of the RMSNorm kernels (the standalone one and the
    one fused into the K = 2048 activation quant), so that the fp16 rows it returns are
    the ones those kernels write or rotate and quantize, bit for bit:
    lane l sums x^2 over its R = 8 * ceil(K / (8 * lanes)) consecutive elements
    l*R .. min((l+1)*R, K) - 1 in order, the lanes are combined by the butterfly
    p[l] += p[l ^ o] for o = lanes/2, .., 1, and h = fp16((x * r) * g) with
    r = 1 / sqrt(ss * fp32(1/K) + eps) (each op one fp32 rounding) and g = 1 + w
    (unit_offset) or w.  x fp16 [M, K], weight fp16 [K], K a multiple of 8."""
    v = np.asarray(x, dtype=np.float16).astype(np.float32)
    m, k = v.shape
    if k % 8:
        raise ValueError(f"K must be a multiple of 8, got {k}")
    r_len = 8 * (-(-(k // 8) // lanes))
    sq = np.zeros((m, lanes * r_len), dtype=np.float32)
    sq[:, :k] = v * v  # elements past K add +0.0, which leaves every fp32 partial sum unchanged
    part = np.zeros((m, lanes), dtype=np.float32)
    per_lane = sq.reshape(m, lanes, r_len)
    for j in range(r_len):
        part = part + per_lane[:, :, j]
    idx = np.arange(lanes)
    o = lanes // 2
    while o >= 1:
        part = part + part[:, idx ^ o]
        o //= 2
    ss = part[:, 0]
    r = np.float32(1.0) / np.sqrt(ss * np.float32(1.0 / k) + np.float32(eps))
    w = np.asarray(weight, dtype=np.float16).astype(np.float32)
    g = (np.float32(1.0) + w) if unit_offset else w
    return ((v * r[:, None]) * g[None, :]).astype(np.float16)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
