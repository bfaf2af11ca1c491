"""GPU parity of the small-M quant + GEMM launch (pi05w4a4_quant_gemm_small, 1..4 rows at
K = 2048): every workgroup quantizes the rows in its prologue (after the RMSNorm when a norm
weight is given) and multiplies them with its weights in the same launch.  Bar: outputs
bit-identical to the two-launch path (pi05w4a4_quantize / pi05w4a4_rmsnorm_quantize, then
pi05w4a4_gemm_multi / pi05w4a4_gemm_residual) and to the oracle's int4_gemm_ref, for one to
three weights, weights in the L1, L3 and MFMA layouts, N not a multiple of 32 or of 16,
with and without a residual, and the ops that route to it (int4_gemm, int4_gemm3,
rms_norm_int4_gemm3, int4_gemm_residual).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc
from tests import w4a4_inputs as inp

pytestmark = pytest.mark.gpu
K = 2048


@pytest.fixture(scope="module")
def ext(cuda):
    from pi05_fast.w4a4 import extension

    extension.preload()
    return extension


def _same_f16(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def _two_launch(ext, x, ws, norm=None, residual=None):
    """The two-launch path on the same inputs: quant (or norm + quant), then the GEMM."""
    dev = x.device
    q, sa = ext.quantize(x) if norm is None else ext.rms_norm_quantize(x, *norm)
    conv = [ext._as_mfma(w, K, False) for w in ws]
    with ext._on_device(dev):
        return ext._gemm_from_q(q, sa, K, conv, tuple(x.shape[:-1]), dev, "test", residual=residual)


def _fused(ext, x, ws, norm=None, residual=None):
    return ext._run_small(x, ws, K, x.numel() // K, False, "test", norm, residual)


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("use_norm", [False, True])
def test_small_m_matches_two_launches_and_oracle(ext, cuda, m, use_norm):
    gen = inp.generator(1300 + 10 * m + use_norm)
    x = inp.activations(gen, m, K)
    nw = (torch.randn(K, generator=gen) * 0.1).half()
    packed = [inp.packed_weight(gen, n, K) for n in (2048, 256, 256)]
    ws = [ext.repack_weight(p.to(cuda), k=K) for p in packed]
    norm = (nw.to(cuda), 1e-6, True) if use_norm else None
    got = _fused(ext, x.to(cuda), ws, norm)
    want = _two_launch(ext, x.to(cuda), ws, norm)
    torch.cuda.synchronize()
    h = orc.rms_norm_lanes(x.numpy(), nw.numpy(), 1e-6) if use_norm else x.numpy()
    for g, w, p in zip(got, want, packed):
        assert _same_f16(g, w), f"M={m}: {int((g.view(torch.int16) != w.view(torch.int16)).sum())} outputs differ"
        ref = orc.int4_gemm_ref(h, p.numpy())
        assert np.array_equal(inp.to_np(g).view(np.int16), ref.view(np.int16))


@pytest.mark.parametrize("n", [48, 40, 1000])
def test_small_m_odd_widths(ext, cuda, n):
    """N = 48 (tiles of 32 columns: a half tile), 40 (padded to 48 by the MFMA repack),
    1000 (padded to 1008): row-major L1 weights through the ops' per-tensor repack."""
    m = 3
    gen = inp.generator(1400 + n)
    x = inp.activations(gen, m, K).to(cuda)
    packed = inp.packed_weight(gen, n, K).to(cuda)
    (got,) = _fused(ext, x, [packed])
    (want,) = _two_launch(ext, x, [packed])
    torch.cuda.synchronize()
    assert tuple(got.shape) == (m, n) and _same_f16(got, want)
    ref = orc.int4_gemm_ref(x.cpu().numpy(), packed.cpu().numpy())
    assert np.array_equal(inp.to_np(got).view(np.int16), ref.view(np.int16))


def test_small_m_tiled_weights(ext, cuda):
    """L3 (WMMA-tiled) weights (the reference's tiled form exists at K = 2048, N = 16384
    only): the op int4_gemm_tiled at M = 2."""
    gen = inp.generator(1450)
    x = inp.activations(gen, 2, K).to(cuda)
    packed = inp.packed_weight(gen, 16384, K)
    from pi05_fast.w4a4.pack import preshuffle_wmma_weight

    tiled = preshuffle_wmma_weight(packed, K).to(cuda)
    got = ext.int4_gemm_tiled(x, tiled)
    want = ext._gemm_from_q(*ext.quantize(x), K, [ext._as_mfma(tiled, K, True)], (2,), x.device, "t")[0]
    torch.cuda.synchronize()
    assert _same_f16(got, want)


@pytest.mark.parametrize("m", [1, 4])
def test_small_m_residual(ext, cuda, m):
    gen = inp.generator(1500 + m)
    x = inp.activations(gen, m, K).to(cuda)
    w = ext.repack_weight(inp.packed_weight(gen, 2048, K).to(cuda), k=K)
    res = (torch.randn(m, 2048, generator=gen) * 4).half().to(cuda)
    (got,) = _fused(ext, x, [w], residual=res)
    (want,) = _two_launch(ext, x, [w], residual=res)
    via_op = ext.int4_gemm_residual(x, w, res)
    torch.cuda.synchronize()
    assert _same_f16(got, want) and _same_f16(via_op, want)


def test_small_m_ops_route_through_one_launch(ext, cuda):
    """int4_gemm, int4_gemm3 and rms_norm_int4_gemm3 at M <= 4 give the two-launch results;
    at M = 5 they take the two-launch path (same bits again)."""
    gen = inp.generator(1600)
    ws = [ext.repack_weight(inp.packed_weight(gen, n, K).to(cuda), k=K) for n in (2048, 256, 256)]
    nw = (torch.randn(K, generator=gen) * 0.1).half().to(cuda)
    for m in (1, 4, 5):
        x = inp.activations(gen, m, K).to(cuda).view(1, m, K)
        a = ext.int4_gemm(x, ws[0])
        b = ext.int4_gemm3(x, *ws)
        c = ext.rms_norm_int4_gemm3(x, nw, 1e-6, *ws)
        torch.cuda.synchronize()
        assert _same_f16(a, _two_launch(ext, x, ws[:1])[0])
        for got, want in zip(b, _two_launch(ext, x, ws)):
            assert _same_f16(got, want)
        for got, want in zip(c, _two_launch(ext, x, ws, norm=(nw, 1e-6, True))):
            assert _same_f16(got, want)


def test_small_m_argument_errors(ext, cuda):
    lib = ext.load_int4_gemm()
    gen = inp.generator(1700)
    w = ext.repack_weight(inp.packed_weight(gen, 64, K).to(cuda), k=K)
    y = torch.empty(8, 64, dtype=torch.float16, device=cuda)
    w_arr = (ctypes.c_void_p * 1)(w.data_ptr())
    y_arr = (ctypes.c_void_p * 1)(y.data_ptr())
    n_arr = (ctypes.c_int32 * 1)(64)
    st = torch.cuda.current_stream().cuda_stream
    for m, k in ((5, K), (0, K), (2, 1024)):
        x = torch.zeros(max(m, 1), k, dtype=torch.float16, device=cuda)
        rc = lib.pi05w4a4_quant_gemm_small(x.data_ptr(), None, 1e-6, 1, m, k, 1, w_arr, n_arr, y_arr, None, st)
        assert rc == 1, (m, k)
        assert b"small-M" in lib.pi05w4a4_last_error()
