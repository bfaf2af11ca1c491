"""Host-side logic of the W4A4 package and the C ABI boundary -- CPU only (no GPU calls).

* The package's packer / CPU reference API (pi05_fast.w4a4.pack) against the golden
  vectors and the oracle.
* Layout transforms: WMMA preshuffle round trip (the reference's CPU test,
  tests/test_w4a4.py:24-42) and the MFMA-fragment-major permutation.
* The C-ABI library loads and exports every symbol include/pi05_w4a4.h declares; its
  argument validation rejects bad calls before touching the GPU.
* The custom ops are registered under the reference's names with shape-only fakes;
  host-side checks raise the reference's messages.
"""

from __future__ import annotations

import ctypes
import json
import os
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc
from tests import w4a4_inputs as inp
from tests.conftest import ROOT

PKG_ROOT = ROOT / "pi05-pytorch-fast_amd"


@pytest.fixture(scope="module")
def pack():
    from pi05_fast.w4a4 import pack as p

    return p


# ----------------------------------------------------------------------------- packer API
@pytest.mark.parametrize("shape", [(8, 64), (8, 192), (8, 1024), (16, 2048), (2, 16384)])
def test_pack_linear_weight_matches_golden(golden, pack, shape):
    n, k = shape
    got = pack.pack_linear_weight(torch.from_numpy(golden[f"w_in_{n}x{k}"]))
    assert np.array_equal(got.numpy(), golden[f"w_packed_{n}x{k}"])


@pytest.mark.parametrize("k", [64, 192, 512, 1024, 2048, 16384])
def test_quant_activation_cpu_matches_golden(golden, pack, k):
    q, s = pack.quant_activation_cpu(torch.from_numpy(golden[f"act_x_{k}"]))
    assert np.array_equal(q.numpy(), golden[f"act_q_{k}"])
    assert np.array_equal(s.numpy().view(np.int32), golden[f"act_s_{k}"].view(np.int32))


@pytest.mark.parametrize("m,n,k", [(6, 8, 64), (8, 16, 2048), (4, 2, 16384), (6, 8, 1024)])
def test_int4_gemm_ref_matches_golden(golden, pack, m, n, k):
    y = pack.int4_gemm_ref(torch.from_numpy(golden[f"act_x_{k}"][:m]),
                           torch.from_numpy(golden[f"w_packed_{n}x{k}"]))
    assert np.array_equal(y.numpy().view(np.int16), golden[f"gemm_y_{m}x{n}x{k}"].view(np.int16))


def test_nibbles_match_golden(golden, pack):
    assert np.array_equal(pack.pack_nibbles(torch.from_numpy(golden["nib_codes"])).numpy(),
                          golden["nib_packed"])
    assert np.array_equal(pack.unpack_nibbles(torch.from_numpy(golden["nib_words"]), 40).numpy(),
                          golden["nib_unpacked"])


def test_fwht_matches_golden(golden, pack):
    for n in (8, 64, 2048):
        got = pack.fwht_unnormalized(torch.from_numpy(golden[f"fwht_in_{n}"])).numpy()
        assert np.array_equal(got.view(np.int32), golden[f"fwht_out_{n}"].view(np.int32))


# ----------------------------------------------------------------------------- layouts
def test_payload_and_scales_round_trip(pack):
    """The reference's PreshuffleLayoutTest (tests/test_w4a4.py:24-42)."""
    n, k = 7, 64
    packed = inp.random_packed(inp.generator(1), n, k)
    tiled = pack.preshuffle_wmma_weight(packed, k)
    words = k // 8
    flat = tiled.view(-1)
    restored_payload = flat[: n * words].view(words // 2, n, 2).permute(1, 0, 2).reshape(n, words)
    restored_scales = flat[n * words : n * words + n]
    assert tuple(tiled.shape) == (n, words + 9)
    assert torch.equal(restored_payload, packed[:, :words])
    assert torch.equal(restored_scales, packed[:, words])
    assert np.array_equal(tiled.numpy(), orc.preshuffle_wmma_weight(packed.numpy(), k))


@pytest.mark.parametrize("n,k", [(16, 64), (32, 192), (48, 2048)])
def test_mfma_layout_definition(pack, n, k):
    """Fragment (column block nb, 128-deep block t) is 1 KB at word (nb*KB + t)*256 made of
    64 16-byte slots; slot L holds codes 128*t + 32*(L//16) .. +31 of column 16*nb + L%16
    (zero words past K), so lane L's two MFMA operands are codes 0-15 and 16-31 of it and
    the 4 lane groups cover the block's 128 codes once.  Byte j of a word holds the code of
    k = 2j in its high nibble (two's complement) and that of k = 2j + 1 in its low nibble
    (offset binary).  The scales follow the payload, then wcorr = -128 * even-k code sums."""
    packed = inp.random_packed(inp.generator(n + k), n, k)
    mf = pack.pack_mfma_weight(packed, k)
    assert tuple(mf.shape) == (n, k // 8 + pack.MFMA_MARKER_WORDS)
    flat = mf.view(-1).numpy()
    codes = orc.unpack_nibbles(packed.numpy()[:, : k // 8], k)
    kb = (k + 127) // 128
    for nb in range(n // 16):
        for t in range(kb):
            seen = np.zeros((16, 128), np.int32)
            for lane in range(64):
                w = (nb * kb + t) * 256 + 4 * lane
                byts = flat[w : w + 4].astype(np.uint32).view(np.uint8).astype(np.int32)
                hi = byts >> 4
                got = np.empty(32, np.int32)
                got[0::2] = np.where(hi >= 8, hi - 16, hi)  # k even: two's complement
                got[1::2] = (byts & 15) - 8                 # k odd: offset binary
                k0 = 128 * t + 32 * (lane // 16)
                seg = codes[16 * nb + lane % 16, k0 : k0 + 32]
                assert np.array_equal(got[: seg.size], seg), (nb, t, lane)
                # pad words past K are all-zero bits (not encoded zero codes)
                assert np.all(flat[w + seg.size // 8 : w + 4] == 0), (nb, t, lane)
                seen[lane % 16, 32 * (lane // 16) : 32 * (lane // 16) + 32] += 1
            assert np.all(seen == 1)
    pw = n * kb * 16
    assert np.array_equal(flat[pw : pw + n], packed.numpy()[:, k // 8])
    assert np.array_equal(flat[pw + n : pw + 2 * n], -128 * codes[:, 0::2].sum(axis=1))
    assert np.all(flat[pw + 2 * n :] == 0)
    assert torch.equal(pack.unpack_mfma_weight(mf, k), packed)


def _unpack_bytes(words: np.ndarray, mask: int) -> np.ndarray:
    """int8 bytes of (word & mask) for every word: the GPU's one-AND unpack."""
    return (words.astype(np.uint32) & np.uint32(mask)).view(np.uint8).view(np.int8).astype(np.int64)


@pytest.mark.parametrize("m,n,k", [(3, 5, 64), (16, 16, 2048), (7, 9, 16384)])
def test_nibble_encoding_identity(pack, m, n, k):
    """The MFMA-side algebra: unpacking encoded activation and weight words with one AND
    each (activation: & 0x0F0F0F0F paired with the weight's & 0xF0F0F0F0, and vice versa)
    and summing the int8 byte products gives S = 16 * acc + 128 * (odd-k activation code
    sum) + 128 * (even-k weight code sum), so S + qcorr + wcorr = 16 * acc.  Checked with
    extreme codes too (-8/7 weights, +-7 activations)."""
    gen = np.random.default_rng(m * n + k)
    a = gen.integers(-7, 8, (m, k)).astype(np.int64)
    b = gen.integers(-8, 8, (n, k)).astype(np.int64)
    a[0, :] = 7 if m > 1 else a[0, :]
    b[0, :] = -8
    if n > 1:
        b[1, :] = 7
    wa = pack.flip_activation_words(torch.from_numpy(orc.pack_nibbles(a.astype(np.int32)))).numpy()
    wb = pack.encode_weight_words(torch.from_numpy(orc.pack_nibbles(b.astype(np.int32)))).numpy()
    a_lo, a_hi = _unpack_bytes(wa, 0x0F0F0F0F), _unpack_bytes(wa, 0xF0F0F0F0)
    b_lo, b_hi = _unpack_bytes(wb, 0x0F0F0F0F), _unpack_bytes(wb, 0xF0F0F0F0)
    s = a_lo.reshape(m, -1) @ b_hi.reshape(n, -1).T + a_hi.reshape(m, -1) @ b_lo.reshape(n, -1).T
    acc = a @ b.T
    qcorr = -128 * a[:, 1::2].sum(axis=1)
    wcorr = -128 * b[:, 0::2].sum(axis=1)
    assert np.array_equal(s + qcorr[:, None] + wcorr[None, :], 16 * acc)
    assert np.abs(s).max() <= 2048 * k
    mf = pack.pack_mfma_weight(torch.from_numpy(np.concatenate(
        [orc.pack_nibbles(b.astype(np.int32)), np.ones((n, 1), np.int32)], axis=1)), k) if n % 16 == 0 else None
    if mf is not None:
        assert np.array_equal(pack.mfma_weight_corrections(mf, k).numpy(), wcorr)


@pytest.mark.parametrize("m,k", [(1, 64), (17, 128), (40, 2048)])
def test_activation_fragment_layout(pack, m, k):
    """Quantized activations use the weight fragment layout on 16-row blocks: the index map
    is injective into the first ceil(M/16)*16 * ceil(K/128)*16 words and places word
    (row, kw) in slot row%16 + 16*((kw%16)//4) of fragment (row//16, kw//16)."""
    idx = pack.fragment_word_index(m, k).numpy()
    m16 = (m + 15) // 16 * 16
    total = m16 * ((k + 127) // 128) * 16
    full = pack.fragment_word_index(m16, k).numpy().reshape(-1)
    assert len(np.unique(full)) == full.size and full.max() < total
    assert np.array_equal(idx, full.reshape(m16, k // 8)[:m])
    kb = (k + 127) // 128
    for row, kw in [(0, 0), (m - 1, k // 8 - 1), (m // 2, k // 16)]:
        slot = row % 16 + 16 * ((kw % 16) // 4)
        assert idx[row, kw] == ((row // 16) * kb + kw // 16) * 256 + 4 * slot + kw % 4
    words = torch.randint(-(2**31), 2**31 - 1, (m, k // 8), dtype=torch.int32)
    buf = torch.zeros(total + m16, dtype=torch.int32)
    buf[torch.from_numpy(idx.reshape(-1))] = pack.flip_activation_words(words).reshape(-1)
    buf[total : total + m] = torch.arange(m, dtype=torch.int32)
    assert torch.equal(pack.codes_from_fragment_major(buf, m, k), words)
    assert torch.equal(pack.qcorr_from_fragment_major(buf, m, k), torch.arange(m, dtype=torch.int32))
    # activation encoding: low nibble of each byte offset binary, high nibble two's complement
    w0 = int(orc.pack_nibbles(np.array([[-8, -1, 0, 7, 3, -3, 1, -7]], np.int32))[0, 0]) & 0xFFFFFFFF
    e0 = int(pack.flip_activation_words(torch.tensor([w0 - (1 << 32) if w0 >= 1 << 31 else w0], dtype=torch.int32))[0]) & 0xFFFFFFFF
    assert [(e0 >> (8 * j)) & 15 for j in range(4)] == [-8 + 8, 0 + 8, 3 + 8, 1 + 8]
    assert [(e0 >> (8 * j + 4)) & 15 for j in range(4)] == [15, 7, 13, 9]


def test_mfma_layout_rejects_bad_shapes(pack):
    with pytest.raises(ValueError):
        pack.mfma_word_permutation(8, 64)
    with pytest.raises(ValueError):
        pack.mfma_word_permutation(16, 96)


# ----------------------------------------------------------------------------- C ABI
HEADER = ROOT / "include" / "pi05_w4a4.h"


def _declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(pi05w4a4_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from pi05_fast.w4a4 import extension

    path = extension.library_path()
    if not path.is_file():
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    return extension.load_int4_gemm()


def test_library_exports_every_declared_symbol(lib):
    syms = _declared_symbols()
    assert len(syms) >= 10
    raw = ctypes.CDLL(str(lib._name))
    missing = [s for s in syms if not hasattr(raw, s)]
    assert not missing, f"missing exports: {missing}"


def test_library_version_and_sizes(lib):
    assert lib.pi05w4a4_version() >= 100
    assert lib.pi05w4a4_q_words(776, 2048) == 784 * 256 + 784  # codes, then qcorr per row
    assert lib.pi05w4a4_q_words(16, 64) == 16 * 16 + 16  # K padded to 128
    assert lib.pi05w4a4_q_words(0, 64) == 0
    assert lib.pi05w4a4_mfma_words(2048, 2048) == 2048 * (2048 // 8 + 2)  # + scale, wcorr
    assert lib.pi05w4a4_mfma_words(32, 192) == 32 * (256 // 8 + 2)
    assert lib.pi05w4a4_mfma_words(0, 64) == 0


def test_host_q_words_matches_library(lib):
    from pi05_fast.w4a4 import extension as ext

    for m in (0, 1, 15, 16, 17, 776, 1552, 6208):
        for k in (0, 64, 128, 192, 2048, 16384):
            assert ext._q_words(m, k) == lib.pi05w4a4_q_words(m, k), (m, k)


def test_direct_route_only_for_plain_untraced_calls():
    """The eager bypass of torch.ops is taken only when the dispatcher has nothing to do."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.overrides import TorchFunctionMode

    from pi05_fast.w4a4 import extension as ext

    x = torch.zeros(4, 64, dtype=torch.float16)
    w = torch.nn.Parameter(torch.zeros(16, 9, dtype=torch.int32), requires_grad=False)
    assert ext._direct(x, w, None)
    xg = torch.zeros(4, 64, requires_grad=True)
    assert not ext._direct(xg, w)
    with torch.no_grad():
        assert ext._direct(xg, w)
    with torch.inference_mode():
        assert ext._direct(torch.zeros(4, 64), w)
    with FakeTensorMode() as mode:
        assert not ext._direct(torch.empty(4, 64))
    assert not ext._direct(mode.from_tensor(x))

    class _Mode(TorchFunctionMode):
        def __torch_function__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    with _Mode():
        assert not ext._direct(x)

    # torch.jit.trace records only dispatched ops: inside a trace the call must take
    # torch.ops, or the traced graph would replay uninitialised outputs.
    seen = []

    def probe(t):
        seen.append(ext._direct(t, w))
        return t * 2

    torch.jit.trace(probe, (x,), check_trace=False)
    assert seen == [False]
    assert ext._direct(x, w)


def test_weight_caches_follow_data_rebinding_and_clear():
    """The per-tensor repack cache (and the RoPE-pair K copies) key on the tensor, its
    version counter and its data pointer: ``w.data = new`` (same object, same version,
    new storage) is seen; ``w.data.copy_`` is not, and clear_weight_caches() drops every
    entry.  CPU-side bookkeeping only: the entries here are planted, nothing is launched."""
    from pi05_fast.w4a4 import apply, extension as ext

    w = torch.zeros(16, 9, dtype=torch.int32)
    key = id(w)
    sentinel = torch.ones(1)
    ext._MFMA_CACHE[key] = (ext.weakref.ref(w), w._version, w.data_ptr(), 64, False, sentinel)
    try:
        hit = ext._MFMA_CACHE[key]
        assert hit[0]() is w and hit[1] == w._version and hit[2] == w.data_ptr()
        w.data = torch.ones(16, 9, dtype=torch.int32)  # new storage, same object and version
        assert ext._MFMA_CACHE[key][2] != w.data_ptr()  # the lookup in _as_mfma misses
        w.data.copy_(torch.full((16, 9), 3, dtype=torch.int32))  # bypasses the version counter
        assert ext._MFMA_CACHE[key][1] == w._version
        ext.clear_weight_caches()
        assert key not in ext._MFMA_CACHE
    finally:
        ext._MFMA_CACHE.pop(key, None)

    class _Attn(torch.nn.Module):
        pass

    attn = _Attn()
    attn._w4a4_k_rope = (w, w._version, sentinel, w.data_ptr())
    apply._K_ROPE_HOLDERS.add(attn)
    ext.clear_weight_caches()
    assert not hasattr(attn, "_w4a4_k_rope")


def test_workspace_sizing(lib):
    n1 = (ctypes.c_int32 * 1)(2048)
    ws_down = lib.pi05w4a4_gemm_workspace_bytes(776, 16384, 1, n1, 0)
    assert ws_down % (776 * 2048 * 4) == 0
    n2 = (ctypes.c_int32 * 2)(16384, 16384)
    assert lib.pi05w4a4_gemm_workspace_bytes(776, 2048, 2, n2, 0) == 0  # enough tiles: no split
    assert lib.pi05w4a4_gemm_workspace_bytes(0, 2048, 1, n1, 0) == 0


def _err(lib) -> str:
    return lib.pi05w4a4_last_error().decode()


def test_abi_validation_without_gpu(lib):
    vp = ctypes.c_void_p
    # K not a multiple of 64
    assert lib.pi05w4a4_quantize(vp(16), 4, 100, vp(16), vp(16), vp(0)) == 1
    assert "multiple of 64" in _err(lib)
    # null pointers
    assert lib.pi05w4a4_quantize(vp(0), 4, 128, vp(16), vp(16), vp(0)) == 1
    # misaligned activations
    assert lib.pi05w4a4_quantize(vp(18), 4, 128, vp(16), vp(16), vp(0)) == 1
    assert "aligned" in _err(lib)
    # M == 0 is a no-op success
    assert lib.pi05w4a4_quantize(vp(0), 0, 128, vp(0), vp(0), vp(0)) == 0
    # repack: N not a multiple of 16, short row stride, bad layout
    assert lib.pi05w4a4_repack_weight(vp(16), 0, 7, 64, 9, vp(16), vp(0)) == 1
    assert lib.pi05w4a4_repack_weight(vp(16), 0, 16, 64, 8, vp(16), vp(0)) == 1
    assert "scale" in _err(lib)
    assert lib.pi05w4a4_repack_weight(vp(16), 5, 16, 64, 9, vp(16), vp(0)) == 1
    # gemm: bad ngroups, misaligned codes, bad N
    n1 = (ctypes.c_int32 * 1)(16)
    w1 = (ctypes.c_void_p * 1)(16)
    y1 = (ctypes.c_void_p * 1)(16)
    assert lib.pi05w4a4_gemm_multi(vp(16), vp(16), 4, 64, 4, w1, n1, y1, vp(0), 0, vp(0)) == 1
    assert lib.pi05w4a4_gemm_multi(vp(20), vp(16), 4, 64, 1, w1, n1, y1, vp(0), 0, vp(0)) == 1
    assert lib.pi05w4a4_gemm(vp(16), vp(16), 4, 64, vp(16), 24, vp(16), vp(0), 0, vp(0)) == 1
    assert "multiple of 16" in _err(lib)
    # K is bounded so that the int32 MFMA sum (at most 2048 K in magnitude) cannot overflow
    assert lib.pi05w4a4_gemm_acc(vp(16), 4, 1 << 20, vp(16), 16, vp(16), vp(0)) == 1
    assert "at most 524288" in _err(lib)
    assert lib.pi05w4a4_gemm(vp(16), vp(16), 4, 1 << 20, vp(16), 16, vp(16), vp(0), 0, vp(0)) == 1
    # M == 0 GEMM is a no-op success
    assert lib.pi05w4a4_gemm(vp(16), vp(16), 0, 64, vp(16), 16, vp(0), vp(0), 0, vp(0)) == 0


def test_attention_abi_validation_without_gpu(lib):
    vp = ctypes.c_void_p
    p = vp(256)  # aligned, never dereferenced: every call below fails validation first

    def prep(b=1, s=776, kvh=1, d=256, ld=256, k=p):
        return lib.pi05w4a4_attn_kv_prep(k, p, ld, p, p, b, s, kvh, d, p, p, vp(0))

    def attn(b=1, s=776, h=8, kvh=1, d=256, mask=vp(0), mlen=0, mbs=0, mrs=0, ld_q=2048, out=p, qc=vp(0)):
        return lib.pi05w4a4_prefix_attention(p, ld_q, p, p, p, mask, mbs, mrs, mlen, 0.0625,
                                             b, s, h, kvh, d, out, 2048, qc, vp(0), vp(0))

    assert lib.pi05w4a4_attn_kv_mfma_elems(1, 776, 1, 256) == 2 * 256 * 832  # K, V^T; keys padded to 64
    assert lib.pi05w4a4_attn_kv_mfma_elems(2, 64, 2, 256) == 2 * 2 * 2 * 256 * 64
    assert prep(d=128) == 1 and "head_dim must be 256" in _err(lib)
    assert prep(s=1025) == 1 and "sequence length" in _err(lib)
    assert prep(s=0) == 1
    assert prep(ld=200) == 1 and "token stride" in _err(lib)
    assert prep(k=vp(258)) == 1 and "aligned" in _err(lib)
    assert attn(h=6, kvh=4) == 1 and "multiple of KV heads" in _err(lib)
    assert attn(ld_q=1024) == 1 and "token stride" in _err(lib)
    assert attn(out=vp(0)) == 1 and "null" in _err(lib)
    # mask rows: a multiple of 4 keys, at least S, strides multiples of 4
    assert attn(mask=p, mlen=775, mrs=776) == 1 and "mask rows" in _err(lib)
    assert attn(mask=p, mlen=776, mrs=776, mbs=2) == 1 and "mask strides" in _err(lib)
    assert attn(mask=vp(260), mlen=776, mrs=776) == 1 and "8-byte" in _err(lib)
    # the fused output quant needs one KV head and 8 query heads of 256, and its scales
    assert attn(h=16, kvh=2, qc=p) == 1 and "one KV head" in _err(lib)
    assert attn(qc=p) == 1 and "q_scales" in _err(lib)

    # the QKV GEMMs with the attention prep: M = B * S with S a multiple of 8 in [8, 1024],
    # one KV head of 256 (the weights' N is fixed), everything 16-byte aligned
    def qkv_rope(m=776, b=1, s=776, n_q=2048, out=p, cos=p):
        return lib.pi05w4a4_gemm_qkv_rope(p, p, m, 2048, p, n_q, p, p, cos, p, b, s, p, out, p, p, vp(0))

    assert qkv_rope(m=20, s=20) == 1 and "multiple of 8" in _err(lib)
    assert qkv_rope(m=776, b=2) == 1 and "M = B * S" in _err(lib)
    assert qkv_rope(m=2056, s=1028, b=2) == 1
    assert qkv_rope(n_q=2040) == 1 and "multiple of 16" in _err(lib)
    assert qkv_rope(out=vp(0)) == 1 and "null" in _err(lib)
    assert qkv_rope(cos=vp(264)) == 1 and "16-byte aligned" in _err(lib)
    assert lib.pi05w4a4_permute_rope_pairs(p, 2048, p, vp(0)) == 1 and "not in place" in _err(lib)
    assert lib.pi05w4a4_permute_rope_pairs(p, 100, vp(512), vp(0)) == 1 and "multiple of 64" in _err(lib)

    # the cache-warming variant: up to 4 buffers, 16-byte aligned, sizes multiples of 16;
    # the attention arguments are validated the same way
    def warm(ptrs, sizes, n=None, ld_q=2048):
        arr = (vp * max(len(ptrs), 1))(*ptrs)
        sz = (ctypes.c_size_t * max(len(sizes), 1))(*sizes)
        return lib.pi05w4a4_prefix_attention_warm(p, ld_q, p, p, p, vp(0), 0, 0, 0, 0.0625, 1, 776, 8, 1, 256, p,
                                                  2048, vp(0), vp(0), arr, sz, len(ptrs) if n is None else n, vp(0))

    assert warm([p] * 5, [16] * 5) == 1 and "0..4 buffers" in _err(lib)
    assert warm([vp(264)], [1024]) == 1 and "16-byte aligned" in _err(lib)
    assert warm([p], [1000]) == 1 and "multiple of 16" in _err(lib)
    assert warm([p], [1024], ld_q=1024) == 1 and "token stride" in _err(lib)

    # the quantizer's cache-warming variant: the same buffer rules, then the quantize ones
    def qwarm(ptrs, sizes, k=16384, x=p):
        arr = (vp * max(len(ptrs), 1))(*ptrs)
        sz = (ctypes.c_size_t * max(len(sizes), 1))(*sizes)
        return lib.pi05w4a4_quantize_warm(x, 776, k, p, p, arr, sz, len(ptrs), vp(0))

    assert qwarm([p] * 5, [16] * 5) == 1 and "0..4 buffers" in _err(lib)
    assert qwarm([vp(264)], [1024]) == 1 and "16-byte aligned" in _err(lib)
    assert qwarm([p], [1000]) == 1 and "multiple of 16" in _err(lib)
    assert qwarm([p], [1024], k=100) == 1 and "multiple of 64" in _err(lib)
    assert qwarm([p], [1024], x=vp(0)) == 1 and "null" in _err(lib)


# ----------------------------------------------------------------------------- op surface
def test_custom_ops_registered_with_fakes():
    from pi05_fast.w4a4 import extension  # noqa: F401

    for name in ("int4_gemm", "int4_gemm_tiled", "int4_gemm2", "int4_gemm2_tiled", "int4_gemm3",
                 "int4_gemm2_gelu"):
        assert hasattr(torch.ops.pi05_w4a4, name)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(2, 776, 2048, dtype=torch.float16)
        w = torch.empty(2560, 2048 // 8 + 16, dtype=torch.int32)
        y = torch.ops.pi05_w4a4.int4_gemm(x, w)
        assert tuple(y.shape) == (2, 776, 2560) and y.dtype == torch.float16
        a, b, c = torch.ops.pi05_w4a4.int4_gemm3(x, w, w[:256], w[:256])
        assert tuple(b.shape) == (2, 776, 256)
        g, u = torch.ops.pi05_w4a4.int4_gemm2_tiled(x, w, w)
        assert tuple(u.shape) == (2, 776, 2560)
        # QKV with the attention prep: q, key states [B, 1, S, 256], v, K/V^T (keys padded to 64)
        nw = torch.empty(2048, dtype=torch.float16)
        cos = torch.empty(2, 776, 256, dtype=torch.float16)
        q, kr, v, kv = torch.ops.pi05_w4a4.rms_norm_int4_gemm3_rope(x, nw, 1e-6, True, w[:2048], w[:256], w[:256],
                                                                  cos, cos)
        assert (tuple(q.shape), tuple(kr.shape), tuple(v.shape)) == ((2, 776, 2048), (2, 1, 776, 256), (2, 776, 256))
        assert kv.numel() == 2 * 2 * 832 * 256
        y, out = torch.ops.pi05_w4a4.prefix_attention_o_proj_kv(q, v, kv, cos, cos, None, 0.0625, 8, w[:2048], q, [],
                                                                False)
        assert tuple(y.shape) == (2, 776, 2048) and out.numel() == 0


def test_ops_reject_cpu_tensors_with_reference_message():
    from pi05_fast.w4a4 import extension

    x = torch.zeros(3, 2048, dtype=torch.float16)
    w = torch.zeros(16, 2048 // 8 + 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="int4_gemm expects CUDA/HIP tensors"):
        extension.int4_gemm(x, w)
    with pytest.raises(RuntimeError, match="int4_gemm expects CUDA/HIP tensors"):
        extension.int4_gemm3(x, w, w, w)


def test_host_checks_messages():
    from pi05_fast.w4a4 import extension as ext

    meta = lambda *s, dt: torch.empty(*s, dtype=dt, device="meta")  # noqa: E731
    # packed weight checks (check_packed, int4_gemm.cu:487-494) on shape/dtype only
    with pytest.raises(RuntimeError, match="packed W must be int32 \\[N, K/8\\+1\\]"):
        ext._check_packed_shape(meta(16, 257, dt=torch.float32), 2048)
    with pytest.raises(RuntimeError, match="must be int32"):
        ext._check_packed_shape(meta(16, 257, 1, dt=torch.int32), 2048)
    with pytest.raises(RuntimeError, match="second dim must contain K/8 packed words plus a scale"):
        ext._check_packed_shape(meta(16, 256, dt=torch.int32), 2048)
    ext._check_packed_shape(meta(16, 257, dt=torch.int32), 2048)
    with pytest.raises(RuntimeError, match="must be on CUDA/HIP"):
        ext._check_packed(meta(16, 257, dt=torch.int32), 2048)
    w_row = meta(16384, 2048 // 8 + 1, dt=torch.int32)
    with pytest.raises(RuntimeError, match="K/8\\+9 marker stride"):
        ext._check_tiled(w_row, 2048)
    with pytest.raises(RuntimeError, match="only K=2048, N=16384"):
        ext._check_tiled(meta(128, 2048 // 8 + 9, dt=torch.int32), 2048)
    ext._check_tiled(meta(16384, 2048 // 8 + 9, dt=torch.int32), 2048)
    ext._check_tiled(meta(256, 2048 // 8 + 16, dt=torch.int32), 2048)  # MFMA accepted
    assert ext.is_mfma_layout(meta(256, 2048 // 8 + 16, dt=torch.int32), 2048)
    assert not ext.is_mfma_layout(meta(256, 2048 // 8 + 8, dt=torch.int32), 2048)


def test_library_missing_fails_loudly(monkeypatch, tmp_path):
    from pi05_fast.w4a4 import extension

    monkeypatch.setenv("PI05_W4A4_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setenv("PI05_W4A4_NO_BUILD", "1")
    monkeypatch.setattr(extension, "_lib", None)
    with pytest.raises(RuntimeError, match="HIP library not found"):
        extension.load_int4_gemm()
    # a build that cannot run (no hipcc) surfaces as the same error, never as a fallback
    monkeypatch.setenv("PI05_W4A4_NO_BUILD", "0")
    monkeypatch.setenv("ROCM_PATH", str(tmp_path / "no_rocm"))
    with pytest.raises(RuntimeError, match="building it failed"):
        extension.load_int4_gemm()
    assert extension._lib is None


def _build_lib_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("_build_lib_under_test", PKG_ROOT / "build_lib.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_build_knobs_reach_hipcc(monkeypatch, tmp_path):
    """GPU_ARCHS / PYTORCH_ROCM_ARCH pick the offload targets (PYTORCH_ROCM_ARCH first, as
    the reference's setdefault does), PI05_W4A4_EXTRA_CFLAGS is appended to every unit and
    PI05_W4A4_VERBOSE=1 turns the command echo on."""
    bl = _build_lib_module()
    monkeypatch.delenv("PYTORCH_ROCM_ARCH", raising=False)
    monkeypatch.delenv("GPU_ARCHS", raising=False)
    assert bl.target_archs() == ["gfx950"]
    monkeypatch.setenv("GPU_ARCHS", "gfx950;gfx942")
    assert bl.target_archs() == ["gfx950", "gfx942"]
    monkeypatch.setenv("PYTORCH_ROCM_ARCH", "gfx950")
    assert bl.target_archs() == ["gfx950"]
    assert bl.target_archs("gfx942") == ["gfx942"]
    monkeypatch.setenv("PI05_W4A4_EXTRA_CFLAGS", "-DPI05_PROBE=1 -g0")
    cmds, objs = bl.compile_commands(bl.target_archs("gfx950,gfx942"), tmp_path)
    assert len(cmds) == len(bl.SOURCES) == len(objs)
    for c in cmds:
        assert "--offload-arch=gfx950" in c and "--offload-arch=gfx942" in c
        assert c[-6:-4] == ["-DPI05_PROBE=1", "-g0"] or ("-DPI05_PROBE=1" in c and "-g0" in c)
    monkeypatch.setenv("PI05_W4A4_VERBOSE", "1")
    assert bl.verbose_from_env()
    monkeypatch.setenv("PI05_W4A4_VERBOSE", "0")
    assert not bl.verbose_from_env()


def test_missing_library_is_built_on_first_load(monkeypatch, tmp_path, capsys):
    """load_int4_gemm() with no library at its path builds one there with hipcc (for the
    GPU_ARCHS target, echoing the commands under PI05_W4A4_VERBOSE=1) and loads it; the
    result exports every symbol the header declares.  (No GPU needed: only the loader runs.)"""
    import shutil

    from pi05_fast.w4a4 import extension

    if shutil.which(str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc")) is None:
        pytest.skip("no hipcc here")
    out = tmp_path / "built" / "libpi05_w4a4.so"
    monkeypatch.setenv("PI05_W4A4_LIB", str(out))
    monkeypatch.delenv("PI05_W4A4_NO_BUILD", raising=False)
    monkeypatch.delenv("PYTORCH_ROCM_ARCH", raising=False)
    monkeypatch.setenv("GPU_ARCHS", "gfx950")
    monkeypatch.setenv("PI05_W4A4_VERBOSE", "1")
    monkeypatch.setattr(extension, "_lib", None)
    lib = extension.load_int4_gemm()
    printed = capsys.readouterr().out
    assert out.is_file()
    assert "--offload-arch=gfx950" in printed and "capi.hip" in printed
    for sym in _declared_symbols():
        assert hasattr(lib, sym), sym
    monkeypatch.setattr(extension, "_lib", None)  # the next user reloads the in-tree library


# ----------------------------------------------------------------------------- module / apply
def test_w4a4_linear_surface():
    from pi05_fast.w4a4 import W4A4Linear

    w = inp.random_packed(inp.generator(5), 32, 2048)
    lin = W4A4Linear(w, in_features=2048)
    assert lin.in_features == 2048 and lin.out_features == 32 and lin.rotate
    assert lin.weight.dtype == torch.float16 and lin.weight.numel() == 0
    assert "packed" in lin.state_dict() and "weight" not in lin.state_dict()
    with pytest.raises(ValueError, match="K/8\\+9 marker stride"):
        W4A4Linear(w, in_features=2048, preshuffled=True)
    with pytest.raises(ValueError, match="too short"):
        W4A4Linear(w[:, :100], in_features=2048)
    assert not lin.mfma
    from pi05_fast.w4a4.pack import pack_mfma_weight

    assert W4A4Linear(pack_mfma_weight(w), in_features=2048).mfma


def test_apply_reference_layouts_on_cpu(monkeypatch):
    from pi05_fast.w4a4.apply import load_time_weight

    w = inp.random_packed(inp.generator(6), 16384, 2048)
    pre, is_pre = load_time_weight(w, "x.layers.0.mlp.gate_proj", 2048, 16384, None)
    assert is_pre and tuple(pre.shape) == (16384, 2048 // 8 + 9)
    pad, is_pre = load_time_weight(w[:256], "x.layers.0.self_attn.k_proj", 2048, 256, None)
    assert not is_pre and tuple(pad.shape) == (256, 2048 // 8 + 8)
    monkeypatch.setenv("PI05_W4A4_ROW_PAD_WORDS", "16")
    with pytest.raises(ValueError, match="collides"):
        load_time_weight(w[:256], "x.layers.0.self_attn.k_proj", 2048, 256, None)


def test_pack_checkpoint_format(tmp_path):
    from safetensors.torch import save_file

    from pi05_fast.w4a4.pack_w4a4_prefix import FORMAT, pack_checkpoint, weight_to_module_name

    prefix = "model.paligemma_with_expert.paligemma.model.language_model.layers.0."
    tensors = {
        prefix + "self_attn.k_proj.weight": torch.randn(256, 2048) * 0.02,
        prefix + "mlp.down_proj.weight": torch.randn(64, 16384) * 0.02,
        prefix + "input_layernorm.weight": torch.zeros(2048),
        "model.other.weight": torch.zeros(4, 4),
    }
    save_file(tensors, str(tmp_path / "model.safetensors"))
    meta = pack_checkpoint(tmp_path / "model.safetensors", tmp_path / "out")
    assert meta["format"] == FORMAT == "embedl-int4-gemm-v1"
    on_disk = json.loads((tmp_path / "out" / "meta.json").read_text())
    name = "paligemma_with_expert.paligemma.model.language_model.layers.0.self_attn.k_proj"
    assert on_disk["layers"][name] == {"in_features": 2048, "out_features": 256, "rotate": True,
                                       "has_bias": False}
    from safetensors.torch import load_file

    packed = load_file(str(tmp_path / "out" / "packed.safetensors"))
    want = orc.pack_linear_weight(tensors[prefix + "self_attn.k_proj.weight"].numpy())
    assert np.array_equal(packed[name + ".packed"].numpy(), want)
    assert weight_to_module_name(prefix + "input_layernorm.weight") is None


def test_prefix_lm_builds_and_fails_loudly_on_cpu():
    from pi05_fast.w4a4 import W4A4Linear
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm, prefix_inputs, prefix_ops

    model, weights = build_prefix_lm("cpu", num_layers=1)
    layer = model.layers[0]
    for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
        assert isinstance(getattr(layer.self_attn, proj), W4A4Linear)
    for proj in ("gate_proj", "up_proj", "down_proj"):
        assert isinstance(getattr(layer.mlp, proj), W4A4Linear)
    assert len(weights) == 7
    assert layer.mlp.gate_proj.preshuffled  # reference layouts off the GPU
    with pytest.raises(RuntimeError, match="CUDA/HIP"):
        model(prefix_inputs(1, 8, "cpu"))
    ops = prefix_ops(776)
    assert abs(sum(ops.values()) / 1e9 - 3075.8) < 0.1


def test_fused_forwards_trace_with_fullgraph(monkeypatch):
    """The fused decoder layer, the fused MLP and a W4A4Linear trace with
    ``torch.compile(fullgraph=True)`` (rocm_pi05_optim.py:254-262): Dynamo captures each as
    one graph over the W4A4 custom ops, run here on meta tensors through the ops' fake
    implementations (the GPU test compiles them with Inductor and runs them)."""
    import types

    import torch
    from transformers.models.gemma.modeling_gemma import GemmaDecoderLayer

    from pi05_fast.w4a4 import apply
    from pi05_fast.w4a4.linear import W4A4Linear
    from pi05_fast.w4a4.norm import FusedRMSNorm
    from pi05_fast.w4a4.prefix_lm import gemma_config

    cfg = gemma_config(1)
    with torch.device("meta"):
        layer = GemmaDecoderLayer(cfg, 0)
    for parent in (layer.self_attn, layer.mlp):
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            lin = getattr(parent, name, None)
            if lin is not None:
                w = torch.empty(lin.out_features, lin.in_features // 8 + 16, dtype=torch.int32, device="meta")
                setattr(parent, name, W4A4Linear(w, in_features=lin.in_features))
    for name in ("input_layernorm", "post_attention_layernorm"):
        weight = torch.nn.Parameter(torch.empty(2048, dtype=torch.float16, device="meta"), requires_grad=False)
        setattr(layer, name, FusedRMSNorm(weight, 1e-6))
    apply.fuse_shared_activation_quant(layer)
    assert layer.mlp._w4a4_fuse_gelu
    assert apply.fuse_decoder_layers(layer) == 1
    # meta tensors are not on a GPU: let the call-time fit checks pass
    monkeypatch.setattr(apply, "_attention_call_fits", lambda *a, **k: True)
    monkeypatch.setattr(apply, "_norms_fit", lambda *a, **k: True)
    x = torch.empty(1, 776, 2048, dtype=torch.float16, device="meta")
    cos = torch.empty(1, 776, 256, dtype=torch.float16, device="meta")
    mask = torch.empty(1, 1, 776, 776, dtype=torch.float16, device="meta")
    torch._dynamo.reset()
    y = torch.compile(layer, fullgraph=True, backend="eager")(x, attention_mask=mask, position_embeddings=(cos, cos))
    assert (y[0] if isinstance(y, tuple) else y).shape == (1, 776, 2048)
    torch._dynamo.reset()
    assert torch.compile(layer.mlp, fullgraph=True, backend="eager")(x).shape == (1, 776, 2048)
    torch._dynamo.reset()
    assert torch.compile(layer.self_attn.o_proj, fullgraph=True, backend="eager")(x).shape == (1, 776, 2048)


def test_residual_and_mask_checks_precede_any_launch():
    """A residual or attention mask on the wrong device or of the wrong dtype is rejected by
    the host checks (the kernels read them through raw device pointers)."""
    import torch

    from pi05_fast.w4a4 import extension as ext

    dev = torch.device("cuda:0")
    ok = torch.empty(4, 256, dtype=torch.float16, device="meta")
    with pytest.raises(RuntimeError, match="residual must be on cuda:0"):
        ext._check_residual(torch.zeros(4, 256, dtype=torch.float16), dev, (4, 256))
    with pytest.raises(RuntimeError, match="residual must be on cuda:0"):
        ext._check_residual(ok, dev, (4, 256))
    meta = torch.device("meta")
    with pytest.raises(RuntimeError, match="residual must be float16"):
        ext._check_residual(torch.empty(4, 256, dtype=torch.bfloat16, device="meta"), meta, (4, 256))
    with pytest.raises(RuntimeError, match="residual must be \\[4, 256\\]"):
        ext._check_residual(torch.empty(4, 128, dtype=torch.float16, device="meta"), meta, (4, 256))
    ext._check_residual(ok, meta, (4, 256))
    with pytest.raises(RuntimeError, match="mask must be on cuda:0"):
        ext._attention_mask_arg(torch.zeros(1, 1, 8, 8, dtype=torch.float16), 1, 8, dev)


def test_gelu_op_rejects_wmma_tiled_weights():
    """int4_gemm2_gelu reads row-major or MFMA-layout weights only: WMMA-tiled gate/up
    weights (the K/8+9 marker stride) are refused instead of being misread."""
    import torch

    from pi05_fast.w4a4 import extension as ext

    x = torch.empty(4, 2048, dtype=torch.float16, device="meta")
    tiled = torch.empty(16384, 2048 // 8 + 9, dtype=torch.int32, device="meta")
    with pytest.raises(RuntimeError, match="int4_gemm2_tiled"):
        ext._check_gelu_weights(x, tiled, tiled)
    with pytest.raises(RuntimeError, match="same shape"):
        ext._check_gelu_weights(x, tiled, tiled[:16])
    row = torch.empty(16384, 2048 // 8 + 1, dtype=torch.int32, device="meta")
    ext._check_gelu_weights(x, row, row)


# ----------------------------------------------------------------------------- E3M2 form
def _e3m2_encode_closed_form(c: int) -> int:
    """The 6-bit E3M2 pattern of integer c from the format's definition alone (search over
    the 64 patterns: (-1)^s 2^(e-3) (1 + m/4), subnormal m/16), independent of pack.py."""
    for b in range(64):
        s, e, m = b >> 5, (b >> 2) & 7, b & 3
        v = (m / 16.0) if e == 0 else 2.0 ** (e - 3) * (1 + m / 4.0)
        if (-v if s else v) == c and not (c == 0 and b != 0):
            return b
    raise AssertionError(f"{c} is not an E3M2 value")


def test_e3m2_value_table():
    """OCP FP6 E3M2 known values, and every INT4 code (including -8 and 8) is one."""
    from pi05_fast.w4a4 import pack

    vals = pack.e3m2_to_float(torch.arange(64)).tolist()
    assert vals[0x1F] == 28.0 and vals[0x01] == 0.0625 and vals[0x0C] == 1.0 and vals[0x04] == 0.25
    assert vals[0x18] == 8.0 and vals[0x38] == -8.0 and vals[0x17] == 7.0 and vals[0x15] == 5.0
    assert vals[0x20] == 0.0  # negative zero
    assert {_e3m2_encode_closed_form(c) for c in range(-8, 9)} == {
        0x00, 0x0C, 0x10, 0x12, 0x14, 0x15, 0x16, 0x17, 0x18, 0x2C, 0x30, 0x32, 0x34, 0x35, 0x36, 0x37, 0x38}


def _pack_slot(codes32) -> bytes:
    bits = 0
    for j, c in enumerate(codes32):
        bits |= _e3m2_encode_closed_form(int(c)) << (6 * j)
    return bits.to_bytes(24, "little")


def test_e3m2_decoders_against_an_independent_packer():
    """pack.codes_from_e3m2_weight / codes_from_e3m2_fragments read back what a packer
    written from the layout's definition (include/pi05_w4a4.h) lays down."""
    from pi05_fast.w4a4 import pack

    rng = np.random.default_rng(5)
    n, k = 64, 256
    kb = k // 128
    codes = rng.integers(-8, 9, size=(n, k))
    scales = rng.random(n).astype(np.float32)
    payload = np.zeros((n // 32, kb, 3, 64, 16), np.uint8)
    for p_ in range(n // 32):
        for b in range(kb):
            for lane in range(64):
                rec = b"".join(_pack_slot(codes[32 * p_ + 16 * h + lane % 16, 128 * b + 32 * (lane // 16):][:32])
                               for h in range(2))
                for c in range(3):
                    payload[p_, b, c, lane] = np.frombuffer(rec[16 * c:16 * c + 16], np.uint8)
    w6 = np.zeros(n * (3 * k // 16 + 16), np.int32)
    w6[: n * kb * 24] = payload.reshape(-1).view(np.int32)
    w6[n * kb * 24: n * kb * 24 + n] = scales.view(np.int32)
    got, sc = pack.codes_from_e3m2_weight(torch.from_numpy(w6.reshape(n, -1)), k)
    assert np.array_equal(got.numpy(), codes) and np.array_equal(sc.numpy(), scales)

    m = 20  # two row blocks, the second partly padding
    acts = rng.integers(-7, 8, size=(m, k))
    frags = np.zeros((2, kb, 1536), np.uint8)
    for mb in range(2):
        for b in range(kb):
            for lane in range(64):
                row = 16 * mb + lane % 16
                slot = _pack_slot(acts[row, 128 * b + 32 * (lane // 16):][:32]) if row < m else bytes(24)
                frags[mb, b, 16 * lane:16 * lane + 16] = np.frombuffer(slot[:16], np.uint8)
                frags[mb, b, 1024 + 8 * lane:1024 + 8 * lane + 8] = np.frombuffer(slot[16:], np.uint8)
    got = pack.codes_from_e3m2_fragments(torch.from_numpy(frags.reshape(-1)), m, k)
    assert np.array_equal(got.numpy(), acts)


def test_e3m2_sizes_and_layout_marker(lib):
    from pi05_fast.w4a4 import extension as ext
    from pi05_fast.w4a4.linear import W4A4Linear

    for m, k in ((1, 2048), (776, 2048), (17, 4096)):
        assert ext._q6_bytes(m, k) == lib.pi05w4a4_q_e3m2_bytes(m, k) == (m + 15) // 16 * (k // 128) * 1536
    for n, k in ((16384, 2048), (64, 4096)):
        assert lib.pi05w4a4_e3m2_words(n, k) == n * (k // 128) * 24 + n <= n * (3 * k // 16 + 16)

    def meta(n, w):
        return torch.empty((n, w), dtype=torch.int32, device="meta")

    assert ext.is_e3m2_layout(meta(16384, 3 * 2048 // 16 + 16), 2048)
    assert not ext.is_e3m2_layout(meta(16384, 2048 // 8 + 16), 2048)
    assert not ext.is_e3m2_layout(meta(48, 3 * 2048 // 16 + 16), 2048)  # N % 32
    assert not ext.is_mfma_layout(meta(16384, 3 * 2048 // 16 + 16), 2048)
    lin = W4A4Linear(torch.zeros(64, 3 * 2048 // 16 + 16, dtype=torch.int32), in_features=2048)
    assert lin.e3m2 and lin.mfma and "layout=e3m2" in lin.extra_repr()
    lin4 = W4A4Linear(torch.zeros(64, 2048 // 8 + 16, dtype=torch.int32), in_features=2048)
    assert lin4.mfma and not lin4.e3m2


def test_e3m2_abi_validation_without_gpu(lib):
    """Argument errors come back before any launch (no GPU needed)."""
    import ctypes

    vp = ctypes.c_void_p
    w = (vp * 2)(16, 16)
    n = (ctypes.c_int32 * 2)(64, 32)
    y = (vp * 2)(16, 16)
    assert lib.pi05w4a4_gemm_e3m2(16, 16, 8, 2048, 2, w, n, y, 1, None) != 0  # gate/up N differ
    assert b"same N" in lib.pi05w4a4_last_error()
    n2 = (ctypes.c_int32 * 2)(48, 48)
    assert lib.pi05w4a4_gemm_e3m2(16, 16, 8, 2048, 2, w, n2, y, 0, None) != 0
    assert b"N % 32" in lib.pi05w4a4_last_error()
    n3 = (ctypes.c_int32 * 2)(64, 64)
    assert lib.pi05w4a4_gemm_e3m2(16, 16, 8, 2000, 2, w, n3, y, 0, None) != 0
    assert b"K % 128" in lib.pi05w4a4_last_error()
    assert lib.pi05w4a4_quantize_e3m2(16, 8, 1024, 16, 16, None) != 0
    assert b"K = 2048" in lib.pi05w4a4_last_error()
    assert lib.pi05w4a4_repack_weight_e3m2(16, 64, 2048, 16, None) != 0  # in place
    assert lib.pi05w4a4_gemm_e3m2(16, 16, 0, 2048, 2, w, n3, y, 0, None) == 0  # M = 0: nothing to do


def test_int4_twin_registry():
    """register_int4_twin / int4_twin / gemm_weights_for_rows on CPU tensors of the two
    layouts' shapes: the twin is served while its E3M2 weight is unchanged, for at most
    E3M2_MAX_INT4_ROWS rows; an in-place write or a freed weight retires it."""
    import gc

    from pi05_fast.w4a4 import extension as ext

    k, n = 2048, 64
    w6 = torch.zeros(n, 3 * k // 16 + ext.E3M2_MARKER_WORDS, dtype=torch.int32)
    w4 = torch.zeros(n, k // 8 + ext.MFMA_MARKER_WORDS, dtype=torch.int32)
    assert ext.int4_twin(w6, k) is None
    ext.register_int4_twin(w6, w4, k)
    assert ext.int4_twin(w6, k) is w4
    assert ext.int4_twin(w6, 1024) is None
    rows = ext.E3M2_MAX_INT4_ROWS
    assert ext.gemm_weights_for_rows([w6], k, rows)[0] is w4
    assert ext.gemm_weights_for_rows([w6], k, rows + 1)[0] is w6
    other = torch.zeros_like(w6)  # no twin: the call keeps its E3M2 weights
    assert ext.gemm_weights_for_rows([w6, other], k, 1)[1] is other
    with pytest.raises(RuntimeError):
        ext.register_int4_twin(w4, w6, k)
    w6b = torch.zeros_like(w6)  # clear_weight_caches() drops the twins too
    ext.register_int4_twin(w6b, w4, k)
    ext.clear_weight_caches()
    assert ext.int4_twin(w6b, k) is None
    ext.register_int4_twin(w6, w4, k)
    w6.add_(1)
    assert ext.int4_twin(w6, k) is None
    key = id(w6)
    del w6
    gc.collect()
    assert key not in ext._INT4_TWINS
