"""GPU parity of the gfx950 W4A4 path against the CPU oracle (through the C ABI).

Bar: activation codes, scales, int32 accumulators and fp16 outputs bit-identical to the
oracle (which is itself pinned to the reference's golden vectors).  The path's looser
tolerances (codes +-1 on <= 0.01% of elements, fp16 rel-L2 <= 1e-2) are reported by the
assertion messages, but the tests require exact equality.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc
from tests import w4a4_inputs as inp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext(cuda):
    from pi05_fast.w4a4 import extension

    extension.preload()
    return extension


def _words(q: torch.Tensor, m: int, k: int) -> np.ndarray:
    """Fragment-major GPU codes -> row-major packed words [M, K/8]."""
    from pi05_fast.w4a4.pack import codes_from_fragment_major

    return inp.to_np(codes_from_fragment_major(q.cpu(), m, k))


def _codes(q: torch.Tensor, m: int, k: int) -> np.ndarray:
    return orc.unpack_nibbles(_words(q, m, k), k)


def _assert_qcorr(q: torch.Tensor, codes: np.ndarray, what: str) -> None:
    """The row corrections after the codes: -128 * (sum of the row's odd-k codes)."""
    from pi05_fast.w4a4.pack import qcorr_from_fragment_major

    m, k = codes.shape
    got = inp.to_np(qcorr_from_fragment_major(q.cpu(), m, k))
    want = -128 * codes[:, 1::2].astype(np.int64).sum(axis=1)
    assert np.array_equal(got, want), f"{what}: qcorr differs"


def _assert_codes_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    diff = got.astype(np.int32) - want.astype(np.int32)
    nbad = int(np.count_nonzero(diff))
    assert nbad == 0, (
        f"{what}: {nbad}/{diff.size} codes differ ({100.0 * nbad / diff.size:.4f}%), "
        f"max |diff| {int(np.abs(diff).max())}"
    )


def _assert_f16_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    same = np.array_equal(got.view(np.int16), want.view(np.int16))
    assert same, f"{what}: fp16 outputs differ, rel_l2={orc.rel_l2(got, want):.3e}"


# ----------------------------------------------------------------------------- quantize
@pytest.mark.parametrize("k", [64, 192, 512, 1024, 2048, 16384])
def test_quantize_matches_golden(golden, ext, cuda, k):
    x = torch.from_numpy(golden[f"act_x_{k}"]).to(cuda)
    q, sa = ext.quantize(x)
    torch.cuda.synchronize()
    _assert_codes_equal(_codes(q, x.shape[0], k), golden[f"act_q_{k}"], f"golden K={k}")
    _assert_qcorr(q, golden[f"act_q_{k}"], f"golden K={k}")
    assert np.array_equal(inp.to_np(sa).view(np.int32), golden[f"act_s_{k}"].view(np.int32))


@pytest.mark.parametrize(
    "m,k,kind",
    [(776, 2048, "act"), (776, 16384, "geglu"), (640, 1024, "act"), (3, 2048, "act"), (1, 16384, "act"),
     (33, 4096, "act"), (511, 2048, "act"), (513, 2048, "act")],
)
def test_quantize_matches_oracle(ext, cuda, m, k, kind):
    gen = inp.generator(m + k)
    x = inp.activations(gen, m, k) if kind == "act" else inp.geglu_activations(gen, m, k)
    q, sa = ext.quantize(x.to(cuda))
    torch.cuda.synchronize()
    q_ref, s_ref = orc.quant_activation(x.numpy())
    _assert_codes_equal(_codes(q, m, k), q_ref, f"M={m} K={k} {kind}")
    assert np.array_equal(_words(q, m, k), orc.pack_nibbles(q_ref)), "packed words differ"
    _assert_qcorr(q, q_ref, f"M={m} K={k}")
    assert np.array_equal(inp.to_np(sa).view(np.int32), s_ref.view(np.int32)), "scale bits differ"


@pytest.mark.parametrize("m", [776, 100, 512, 1])
def test_quantize_cache_warm_changes_nothing(ext, cuda, m):
    """The K = 16384 quantizer with cache warming (the slots the last round of rows leaves
    idle read further buffers: here 48 MB) writes the same codes and scales as the plain
    call and leaves the buffers it read unchanged; at M = 512 no slot is idle."""
    gen = inp.generator(40 + m)
    x = inp.geglu_activations(gen, m, 16384).to(cuda)
    big = [torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=cuda) for n in (4 << 20,) * 3]
    keep = [t.clone() for t in big]
    q0, s0 = ext.quantize(x)
    q1, s1 = ext.quantize(x, warm=big)
    torch.cuda.synchronize()
    # rows past M (the 16-row padding of the buffer) are never written: compare M rows
    c0, c1 = _codes(q0, m, 16384), _codes(q1, m, 16384)
    assert np.array_equal(c0, c1) and torch.equal(s0.view(torch.int32), s1.view(torch.int32))
    _assert_qcorr(q1, c1, "warm")
    for t, t0 in zip(big, keep):
        assert torch.equal(t, t0)


@pytest.mark.parametrize("k", [2048, 16384])
def test_quantize_exact_ties(ext, cuda, k):
    """Rows whose rotated values hit exact half-integer multiples of the scale: the GPU's
    reciprocal fast path must fall back to exact division and round half to even.

    x = FWHT(y) / K for y = 2^-4 * (7 e_0 + c_1 e_1 + c_2 e_2 ...) is exact in fp16, the fp32
    FWHT returns y exactly (H.H = K.I on dyadic values), amax = 7/16 makes sdiv = 1/16
    exactly (the 1e-12 is absorbed), and x'/sdiv = c_i are the chosen quotients.
    """
    quotients = [2.5, -2.5, 0.5, -0.5, 3.5, 1.5, -6.5, 4.5, 1.25, -3.75]
    m = 8
    y = np.zeros((m, k), np.float64)
    rng = np.random.default_rng(k)
    for r in range(m):
        y[r, 0] = 7.0 if r % 2 == 0 else -7.0
        cols = rng.choice(np.arange(1, k), size=len(quotients), replace=False)
        y[r, cols] = quotients
    y /= 16.0
    x = orc.fwht_unnormalized(y.astype(np.float32)).astype(np.float64) / k
    x16 = x.astype(np.float16)
    assert np.array_equal(x16.astype(np.float64), x), "inputs must be exact in fp16"
    q, sa = ext.quantize(torch.from_numpy(x16).to(cuda))
    torch.cuda.synchronize()
    q_ref, s_ref = orc.quant_activation(x16)
    got = _codes(q, m, k)
    _assert_codes_equal(got, q_ref, f"ties K={k}")
    _assert_qcorr(q, q_ref, f"ties K={k}")
    assert np.array_equal(inp.to_np(sa).view(np.int32), s_ref.view(np.int32))
    # half-even: 2.5 -> 2, -2.5 -> -2, 0.5 -> 0, 3.5 -> 4, 1.5 -> 2, -6.5 -> -6, 4.5 -> 4
    r0_cols = np.flatnonzero(y[0])
    assert sorted(np.unique(got[0, r0_cols]).tolist()) == sorted({7, 2, -2, 0, 4, -6, 1, -4})


@pytest.mark.parametrize("k", [2048, 16384])
def test_quantize_many_ties(ext, cuda, k):
    """As test_quantize_exact_ties with 48 exact half-integer quotients per row: lanes then
    hold several tied codes, in one or more of their code words, next to words with none,
    so the redo of only the flagged words (each redone in full) is checked against the
    exact division code for code."""
    halves = np.arange(-6.5, 7.0, 1.0)
    m = 16
    y = np.zeros((m, k), np.float64)
    rng = np.random.default_rng(1000 + k)
    for r in range(m):
        y[r, 0] = 7.0 if r % 2 == 0 else -7.0
        cols = rng.choice(np.arange(1, k), size=48, replace=False)
        y[r, cols] = rng.choice(halves, size=48)
    y /= 16.0
    x = orc.fwht_unnormalized(y.astype(np.float32)).astype(np.float64) / k
    x16 = x.astype(np.float16)
    assert np.array_equal(x16.astype(np.float64), x), "inputs must be exact in fp16"
    q, sa = ext.quantize(torch.from_numpy(x16).to(cuda))
    torch.cuda.synchronize()
    q_ref, s_ref = orc.quant_activation(x16)
    got = _codes(q, m, k)
    _assert_codes_equal(got, q_ref, f"many ties K={k}")
    _assert_qcorr(q, q_ref, f"many ties K={k}")
    assert np.array_equal(inp.to_np(sa).view(np.int32), s_ref.view(np.int32))
    for r in range(m):  # every tie went to the even neighbour
        cols = np.flatnonzero(y[r, 1:]) + 1
        assert np.all(got[r, cols] % 2 == 0)


# ----------------------------------------------------------------------------- repack
@pytest.mark.parametrize("n,k", [(16, 64), (48, 192), (256, 2048), (128, 16384)])
def test_repack_matches_cpu_layout(ext, cuda, n, k):
    from pi05_fast.w4a4 import pack

    packed = inp.random_packed(inp.generator(n * 7 + k), n, k)
    want = pack.pack_mfma_weight(packed, k)
    got_l1 = ext.repack_weight(packed.to(cuda), k=k).cpu()
    got_l2 = ext.repack_weight(torch.nn.functional.pad(packed, (0, 7)).to(cuda), k=k).cpu()
    assert torch.equal(got_l1, want)
    assert torch.equal(got_l2, want)
    if k % 16 == 0:
        tiled = pack.preshuffle_wmma_weight(packed, k)
        got_l3 = ext.repack_weight(tiled.to(cuda), k=k, tiled=True).cpu()
        assert torch.equal(got_l3, want)
    assert torch.equal(pack.unpack_mfma_weight(want, k), packed)


# ----------------------------------------------------------------------------- GEMM
GEMM_SHAPES = [
    (1, 2048, 2048),
    (5, 256, 64),
    (40, 160, 1024),
    (100, 48, 192),
    (64, 2048, 2048),
    (113, 256, 2048),
    (272, 512, 2048),
    (776, 2048, 2048),
    (3, 128, 16384),
    (776, 2048, 16384),
    # small M (the K-split streaming tiles: 16, 32 and 64 rows of 32 columns), ragged N
    (16, 48, 2048),
    (17, 2560, 2048),
    (32, 80, 1024),
    (48, 2048, 4096),
    (1, 2048, 16384),
    (64, 2048, 16384),
    # 112 x 64 tiles with four k parts (neither narrow tile fits two per CU): the k parts'
    # reduce-scatter leaves two row blocks to three of the waves and one to the fourth
    (2200, 2048, 2048),
    # the fixed-length K slices with a ragged last row tile: 64 x 64 tiles at K = 2048
    # (40 rows in the last tile) and the 16-block down tiles at K = 16384 (104 rows)
    (1000, 2048, 2048),
    (1000, 2048, 16384),
]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_acc_bit_exact(ext, cuda, m, n, k):
    gen = inp.generator(3 * m + n + k)
    x = inp.activations(gen, m, k)
    packed = inp.random_packed(gen, n, k)  # all 16 nibble values, including -8
    acc, q, _ = ext.int4_gemm_acc(x.to(cuda), packed.to(cuda))
    torch.cuda.synchronize()
    q_ref, _ = orc.quant_activation(x.numpy())
    w_codes, _, _ = orc.unpack_linear_weight(packed.numpy())
    _assert_codes_equal(_codes(q, m, k), q_ref, "codes")
    acc_ref = orc.gemm_acc_int32(q_ref, w_codes)
    got = inp.to_np(acc)
    nbad = int(np.count_nonzero(got != acc_ref))
    assert nbad == 0, f"{nbad}/{got.size} int32 accumulators differ"


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_int4_gemm_bit_exact(ext, cuda, m, n, k):
    gen = inp.generator(5 * m + n + k)
    x = inp.activations(gen, m, k) if k != 16384 else inp.geglu_activations(gen, m, k)
    packed = inp.packed_weight(gen, n, k)
    y_row = ext.int4_gemm(x.to(cuda), packed.to(cuda))
    y_mfma = ext.int4_gemm(x.to(cuda), ext.repack_weight(packed.to(cuda)))
    torch.cuda.synchronize()
    y_ref = orc.int4_gemm_ref(x.numpy(), packed.numpy())
    _assert_f16_equal(inp.to_np(y_mfma), y_ref, f"MFMA layout M={m} N={n} K={k}")
    assert torch.equal(y_row, y_mfma), "row-major and MFMA layouts disagree"


def test_leading_dims_preserved(ext, cuda):
    gen = inp.generator(11)
    x = inp.activations(gen, 2 * 3 * 5, 1024).view(2, 3, 5, 1024)
    packed = inp.packed_weight(gen, 32, 1024)
    y = ext.int4_gemm(x.to(cuda), packed.to(cuda))
    assert tuple(y.shape) == (2, 3, 5, 32) and y.dtype == torch.float16
    y_ref = orc.int4_gemm_ref(x.numpy(), packed.numpy())
    _assert_f16_equal(inp.to_np(y), y_ref, "leading dims")


def test_odd_n_row_major(ext, cuda):
    gen = inp.generator(12)
    x = inp.activations(gen, 9, 2048)
    packed = inp.random_packed(gen, 7, 2048)
    y = ext.int4_gemm(x.to(cuda), packed.to(cuda))
    _assert_f16_equal(inp.to_np(y), orc.int4_gemm_ref(x.numpy(), packed.numpy()), "N=7")


@pytest.mark.parametrize("m", [1, 64, 640, 776])
def test_int4_gemm3_qkv(ext, cuda, m):
    gen = inp.generator(100 + m)
    x = inp.activations(gen, m, 2048)
    ws = [inp.packed_weight(gen, n, 2048) for n in (2048, 256, 256)]
    ws_dev = [ext.repack_weight(w.to(cuda)) for w in ws]
    q, k, v = ext.int4_gemm3(x.to(cuda), *ws_dev)
    torch.cuda.synchronize()
    for name, got, w in zip("qkv", (q, k, v), ws):
        _assert_f16_equal(inp.to_np(got), orc.int4_gemm_ref(x.numpy(), w.numpy()), f"{name} M={m}")


@pytest.mark.parametrize("m", [776, 8])
def test_int4_gemm2_gate_up(ext, cuda, m):
    gen = inp.generator(200 + m)
    x = inp.activations(gen, m, 2048)
    wg = inp.random_packed(gen, 16384, 2048)
    wu = inp.random_packed(gen, 16384, 2048)
    g, u = ext.int4_gemm2(x.to(cuda), ext.repack_weight(wg.to(cuda)), ext.repack_weight(wu.to(cuda)))
    torch.cuda.synchronize()
    _assert_f16_equal(inp.to_np(g), orc.int4_gemm_ref(x.numpy(), wg.numpy()), "gate")
    _assert_f16_equal(inp.to_np(u), orc.int4_gemm_ref(x.numpy(), wu.numpy()), "up")


# Tile configurations of the fused epilogue: 4x2 (M = 776 and 64 at N = 2048), 2x2 (17),
# 1x2 with four k parts (16, 1), 7x4 with four k parts (200 and 113 x 16384: the second row
# tile of 113 rows holds one row), 7x4 with eight k parts, each wave finishing one row block
# (200 x 2048, K = 8192), and 7x4 over 1024 tiles whose last row tile holds one row
# (785 x 16384); the K-split ones stage the GELU correction table compactly, the others in
# its global layout.
@pytest.mark.parametrize("m,n,k", [(776, 2048, 2048), (64, 2048, 2048), (17, 2048, 2048), (16, 2048, 2048),
                                   (1, 2048, 2048), (200, 16384, 2048), (113, 16384, 2048), (200, 2048, 8192),
                                   (785, 16384, 2048)])
def test_int4_gemm2_gelu_matches_unfused(ext, cuda, m, n, k):
    gen = inp.generator(300 + m)
    x = inp.activations(gen, m, k).to(cuda)
    wg = ext.repack_weight(inp.packed_weight(gen, n, k).to(cuda))
    wu = ext.repack_weight(inp.packed_weight(gen, n, k).to(cuda))
    h = ext.int4_gemm2_gelu(x, wg, wu)
    g, u = ext.int4_gemm2(x, wg, wu)
    h_eager = torch.nn.functional.gelu(g, approximate="tanh") * u
    torch.cuda.synchronize()
    h64 = orc.gelu_tanh(inp.to_np(g).astype(np.float64)) * inp.to_np(u).astype(np.float64)
    err_fused = orc.rel_l2(inp.to_np(h), h64)
    assert err_fused <= 1e-3, f"fused rel_l2 {err_fused:.3e} against the float64 closed form"
    # The fused epilogue evaluates gelu and the product exactly as the eager ops do.
    nbad = int((h.view(torch.int16) != h_eager.view(torch.int16)).sum())
    assert nbad == 0, f"{nbad}/{h.numel()} fused outputs differ from eager gelu(gate) * up"


# ----------------------------------------------------------------------------- reference tests
def test_row_padding_is_exact_for_down_projection(ext, cuda):
    """tests/test_w4a4.py:55-65 of the reference."""
    torch.manual_seed(20260923)
    m, k, n = 3, 16384, 128
    x = torch.randn(m, k, dtype=torch.float16, device=cuda)
    packed = inp.random_packed(inp.generator(1), n, k).to(cuda)
    padded = torch.nn.functional.pad(packed, (0, 7))
    assert torch.equal(ext.int4_gemm(x, packed), ext.int4_gemm(x, padded))


def test_preshuffled_gate_weight_is_exact(ext, cuda):
    """tests/test_w4a4.py:67-78 of the reference (one 256-row tile plus a 16-row tail)."""
    from pi05_fast.w4a4.pack import preshuffle_wmma_weight

    torch.manual_seed(20260923)
    m, k, n = 272, 2048, 16384
    x = torch.randn(m, k, dtype=torch.float16, device=cuda)
    packed = inp.random_packed(inp.generator(2), n, k)
    tiled = preshuffle_wmma_weight(packed, k).to(cuda)
    reference = ext.int4_gemm(x, packed.to(cuda))
    candidate = ext.int4_gemm_tiled(x, tiled)
    assert torch.equal(reference, candidate)


def test_tiled_op_rejects_row_major_weight(ext, cuda):
    """tests/test_w4a4.py:80-85 of the reference."""
    x = torch.randn(1, 2048, dtype=torch.float16, device=cuda)
    packed = inp.random_packed(inp.generator(3), 16384, 2048).to(cuda)
    with pytest.raises(RuntimeError, match="K/8\\+9 marker stride"):
        ext.int4_gemm_tiled(x, packed)


def test_op_errors(ext, cuda):
    w = inp.random_packed(inp.generator(4), 16, 2048).to(cuda)
    with pytest.raises(RuntimeError, match="must be float16"):
        ext.int4_gemm(torch.randn(2, 2048, device=cuda), w)
    with pytest.raises(RuntimeError, match="K must be a multiple of 64, got 100"):
        ext.int4_gemm(torch.randn(2, 100, device=cuda).half(), w)
    with pytest.raises(RuntimeError, match="second dim must contain K/8 packed words plus a scale"):
        ext.int4_gemm(torch.randn(2, 4096, device=cuda).half(), w)
    with pytest.raises(RuntimeError, match="must be int32"):
        ext.int4_gemm(torch.randn(2, 2048, device=cuda).half(), w.float())


# ----------------------------------------------------------------------------- decoder RMSNorm
@pytest.mark.parametrize("m,k", [(776, 2048), (5, 2048), (33, 16384), (7, 64)])
def test_rms_norm_matches_gemma_module(ext, cuda, m, k):
    """The one-kernel RMSNorm against transformers' eager GemmaRMSNorm on the same fp16
    inputs: identical except where the sum of squares, reduced in another order, moves the
    result across an fp16 rounding boundary (one ulp, on a small fraction of elements)."""
    from transformers.models.gemma.modeling_gemma import GemmaRMSNorm

    gen = torch.Generator().manual_seed(m * 7 + k)
    x = (torch.randn(m, k, generator=gen) * 3.0).to(torch.float16).to(cuda)
    norm = GemmaRMSNorm(k, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(k, generator=gen) * 0.05)
    norm = norm.to(device=cuda, dtype=torch.float16)
    with torch.no_grad():
        want = norm(x)
        got = ext.rms_norm(x, norm.weight, 1e-6)
    torch.cuda.synchronize()
    ulps = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs()
    assert int(ulps.max()) <= 1, f"max difference {int(ulps.max())} fp16 ulps"
    frac = float((ulps > 0).float().mean())
    assert frac <= 5e-3, f"{100 * frac:.3f}% of outputs differ by one ulp"


@pytest.mark.parametrize("m,k,offset", [(776, 2048, True), (5, 2048, False), (33, 16384, True), (7, 64, True),
                                        (9, 192, True), (3, 4104, True)])
def test_rms_norm_matches_oracle_lane_order(ext, cuda, m, k, offset):
    """The one-kernel RMSNorm equals the oracle's rms_norm_lanes bit for bit: the kernel and
    the RMSNorm fused into the K = 2048 activation quant share one summation order and a
    correctly rounded 1/sqrt, which the oracle restates."""
    gen = torch.Generator().manual_seed(m * 11 + k)
    x = (torch.randn(m, k, generator=gen) * 3.0).to(torch.float16)
    w = (torch.randn(k, generator=gen) * (0.05 if offset else 1.0)).to(torch.float16)
    got = ext.rms_norm(x.to(cuda), w.to(cuda), 1e-6, unit_offset=offset)
    torch.cuda.synchronize()
    want = orc.rms_norm_lanes(x.numpy(), w.numpy(), 1e-6, unit_offset=offset)
    _assert_f16_equal(inp.to_np(got), want, f"rms_norm M={m} K={k}")


# ----------------------------------------------------------------------------- reference default gate/up route
@pytest.mark.parametrize("m", [776, 272])
def test_int4_gemm2_tiled_wmma_weights(ext, cuda, m):
    """The reference's default gate/up route (apply.py:134-135): int4_gemm2_tiled over
    WMMA-tiled (L3, [N, K/8+9]) gate and up weights, K = 2048, N = 16384, against the
    oracle on the row-major weights, bit for bit; int4_gemm_tiled on the same weights too."""
    from pi05_fast.w4a4.pack import preshuffle_wmma_weight

    k, n = 2048, 16384
    gen = inp.generator(400 + m)
    x = inp.activations(gen, m, k)
    wg = inp.random_packed(gen, n, k)
    wu = inp.random_packed(gen, n, k)
    tg, tu = (preshuffle_wmma_weight(w, k).to(cuda) for w in (wg, wu))
    assert tg.shape == (n, k // 8 + 9)
    g, u = ext.int4_gemm2_tiled(x.to(cuda), tg, tu)
    g1 = ext.int4_gemm_tiled(x.to(cuda), tg)
    torch.cuda.synchronize()
    want_g = orc.int4_gemm_ref(x.numpy(), wg.numpy())
    _assert_f16_equal(inp.to_np(g), want_g, f"gate M={m}")
    _assert_f16_equal(inp.to_np(u), orc.int4_gemm_ref(x.numpy(), wu.numpy()), f"up M={m}")
    _assert_f16_equal(inp.to_np(g1), want_g, f"int4_gemm_tiled M={m}")


def test_reference_layout_repack_runs_once_per_weight(ext, cuda, monkeypatch):
    """Weights kept in a reference layout (L1 row-major, L2 row-padded, L3 tiled) are
    repacked into the MFMA layout on their first call only; an in-place update of the
    weight invalidates the cached copy."""
    from pi05_fast.w4a4.pack import preshuffle_wmma_weight

    calls = []
    real = ext.repack_weight

    def counting(*a, **kw):
        calls.append(a[0].shape)
        return real(*a, **kw)

    monkeypatch.setattr(ext, "repack_weight", counting)
    gen = inp.generator(7)
    x = inp.activations(gen, 40, 2048).to(cuda)
    w1 = inp.random_packed(gen, 256, 2048).to(cuda)
    w2 = torch.nn.functional.pad(inp.random_packed(gen, 256, 2048), (0, 7)).to(cuda)
    w3 = preshuffle_wmma_weight(inp.random_packed(gen, 16384, 2048), 2048).to(cuda)
    y1 = [ext.int4_gemm(x, w1) for _ in range(3)]
    y2 = [ext.int4_gemm(x, w2) for _ in range(3)]
    y3 = [ext.int4_gemm_tiled(x, w3) for _ in range(3)]
    torch.cuda.synchronize()
    assert len(calls) == 3, calls
    for ys in (y1, y2, y3):
        assert all(torch.equal(ys[0], y) for y in ys[1:])
    w1.view(torch.int32)[0, 0] ^= 0x11  # in place: the cached copy is stale now
    y1b = ext.int4_gemm(x, w1)
    torch.cuda.synchronize()
    assert len(calls) == 4
    _assert_f16_equal(inp.to_np(y1b), orc.int4_gemm_ref(x.cpu().numpy(), w1.cpu().numpy()), "after update")


def test_reference_layout_cache_sees_data_updates(ext, cuda):
    """Weight updates that bypass the version counter: ``w.data = new`` is caught by the
    cache's data-pointer check; ``w.data.copy_(new)`` needs clear_weight_caches(), after
    which the output follows the new weight again (both against the oracle)."""
    gen = inp.generator(11)
    x = inp.activations(gen, 64, 2048).to(cuda)
    w = inp.random_packed(gen, 256, 2048).to(cuda)
    xn = x.cpu().numpy()
    y0 = ext.int4_gemm(x, w)
    torch.cuda.synchronize()
    _assert_f16_equal(inp.to_np(y0), orc.int4_gemm_ref(xn, w.cpu().numpy()), "first call")
    w.data = inp.random_packed(gen, 256, 2048).to(cuda)  # same object and version, new storage
    y1 = ext.int4_gemm(x, w)
    torch.cuda.synchronize()
    _assert_f16_equal(inp.to_np(y1), orc.int4_gemm_ref(xn, w.cpu().numpy()), "after w.data = new")
    w.data.copy_(inp.random_packed(gen, 256, 2048).to(cuda))  # bypasses the version counter
    ext.clear_weight_caches()
    y2 = ext.int4_gemm(x, w)
    torch.cuda.synchronize()
    _assert_f16_equal(inp.to_np(y2), orc.int4_gemm_ref(xn, w.cpu().numpy()), "after copy_ + clear_weight_caches")
