"""The gate/up GEMM with the GELU-tanh*up epilogue and the down projection's activation
quant in one launch (pi05w4a4_gemm_gelu_up_quant, op rms_norm_int4_mlp), against the two
launches it replaces (pi05w4a4_gemm_gelu_up, then pi05w4a4_quantize of its output) and
the oracle: h, the codes (with the row corrections) and the scale bits must be identical.

Shapes: the forward's 776 tokens; 225 and 300 (three m-tiles: the smallest fused plan);
1000 (a partial last m-tile); batch 8 x 776 (M = 6208, 56 m-tiles, 7168 GEMM tiles); and
M = 1, 40, 100, 200 (other tile plans: the two-launch route of the same entry point).
Also: consecutive calls through one control block (left zeroed by each call), the cache
warming of the quant workgroups that find no row left, and the bounded wait: a call whose
waits can never be satisfied (wait_extra = 1) ends normally, sets the host-visible status
word and leaves the next call on a zeroed control block exact again.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc
from tests import w4a4_inputs as inp

pytestmark = pytest.mark.gpu

H, N = 2048, 16384


@pytest.fixture(scope="module")
def ext(cuda):
    from pi05_fast.w4a4 import extension

    extension.preload()
    return extension


@pytest.fixture(scope="module")
def weights(ext, cuda):
    gen = inp.generator(9100)
    wg = ext.repack_weight(inp.random_packed(gen, N, H).to(cuda))
    wu = ext.repack_weight(inp.random_packed(gen, N, H).to(cuda))
    return wg, wu


def _ptr_arr(ts):
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts]), \
        (ctypes.c_size_t * len(ts))(*[t.numel() * t.element_size() for t in ts])


def _two_launches(ext, q, sa, m, wg, wu):
    lib = ext.load_int4_gemm()
    h = torch.empty(m, N, dtype=torch.float16, device=q.device)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.pi05w4a4_gemm_gelu_up(q.data_ptr(), sa.data_ptr(), m, H, wg.data_ptr(), wu.data_ptr(), N,
                                     h.data_ptr(), None, 0, st) == 0, lib.pi05w4a4_last_error()
    dq, dsa = ext.quantize(h)
    return h, dq, dsa


def _fused(ext, q, sa, m, wg, wu, ctl, warm=(), spin_limit=0, wait_extra=0):
    lib = ext.load_int4_gemm()
    dev = q.device
    h = torch.empty(m, N, dtype=torch.float16, device=dev)
    dq = torch.empty(int(lib.pi05w4a4_q_words(m, N)), dtype=torch.int32, device=dev)
    dsa = torch.empty(m, dtype=torch.float32, device=dev)
    wp, wb = _ptr_arr(list(warm)) if warm else (None, None)
    rc = lib.pi05w4a4_gemm_gelu_up_quant(q.data_ptr(), sa.data_ptr(), m, H, wg.data_ptr(), wu.data_ptr(), N,
                                         h.data_ptr(), dq.data_ptr(), dsa.data_ptr(), ctl.data_ptr(), wp, wb,
                                         len(warm), spin_limit, wait_extra, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.pi05w4a4_last_error()
    return h, dq, dsa


def _new_ctl(ext, m, dev):
    lib = ext.load_int4_gemm()
    return torch.zeros(int(lib.pi05w4a4_mlp_ctl_words(m)), dtype=torch.int32, device=dev)


def _assert_same_codes(dq, dq_ref, m, what):
    """The codes and row corrections of the M valid rows (the pad rows of the last 16-row
    block are never written: the GEMM reads them but stores none of their outputs)."""
    from pi05_fast.w4a4.pack import codes_from_fragment_major, qcorr_from_fragment_major

    _assert_same(codes_from_fragment_major(dq, m, N), codes_from_fragment_major(dq_ref, m, N), f"{what} codes")
    _assert_same(qcorr_from_fragment_major(dq, m, N), qcorr_from_fragment_major(dq_ref, m, N),
                 f"{what} row corrections")


def _assert_same(got, want, what):
    a, b = got.view(torch.int16 if got.dtype == torch.float16 else torch.int32), \
        want.view(torch.int16 if want.dtype == torch.float16 else torch.int32)
    nbad = int((a != b).sum())
    assert nbad == 0, f"{what}: {nbad}/{a.numel()} differ"


@pytest.mark.parametrize("m", [776, 225, 300, 1000, 6208, 1, 40, 100, 200])
def test_fused_down_quant_equals_two_launches(ext, cuda, weights, m):
    print(f"gemm_gelu_up_quant: M={m}", flush=True)
    wg, wu = weights
    lib = ext.load_int4_gemm()
    assert lib.pi05w4a4_mlp_status(1) >= 0
    gen = inp.generator(9200 + m)
    x = inp.activations(gen, m, H).to(cuda)
    q, sa = ext.quantize(x)
    h_ref, dq_ref, dsa_ref = _two_launches(ext, q, sa, m, wg, wu)
    ctl = _new_ctl(ext, m, cuda)
    h, dq, dsa = _fused(ext, q, sa, m, wg, wu, ctl)
    torch.cuda.synchronize()
    assert lib.pi05w4a4_mlp_status(0) == 0
    _assert_same(h, h_ref, f"h M={m}")
    _assert_same_codes(dq, dq_ref, m, f"M={m}")
    _assert_same(dsa, dsa_ref, f"scales M={m}")
    assert int(ctl.abs().sum()) == 0, "the control block is not left zeroed"
    # the oracle's quant of the fp16 h, on a sample of rows (codes and scale bits)
    rows = sorted(set([0, m // 2, m - 1] + list(range(0, m, max(1, m // 12)))))
    hn = h[rows].cpu().numpy()
    q_ref, s_ref = orc.quant_activation(hn)
    from pi05_fast.w4a4.pack import codes_from_fragment_major

    words = codes_from_fragment_major(dq.cpu(), m, N).numpy()[rows]
    assert np.array_equal(orc.unpack_nibbles(words, N), q_ref.astype(np.int32)), f"codes vs oracle M={m}"
    assert np.array_equal(dsa.cpu().numpy()[rows].view(np.int32), s_ref.view(np.int32)), f"scales vs oracle M={m}"


def test_fused_down_quant_h_matches_oracle(ext, cuda, weights):
    """h itself: the oracle's gate and up outputs through torch's eager gelu * up."""
    wg, wu = weights
    m = 300
    gen = inp.generator(9300)
    x = inp.activations(gen, m, H)
    q, sa = ext.quantize(x.to(cuda))
    h, _, _ = _fused(ext, q, sa, m, wg, wu, _new_ctl(ext, m, cuda))
    torch.cuda.synchronize()
    from pi05_fast.w4a4.pack import unpack_mfma_weight

    g = orc.int4_gemm_ref(x.numpy(), unpack_mfma_weight(wg.cpu(), H).numpy())
    u = orc.int4_gemm_ref(x.numpy(), unpack_mfma_weight(wu.cpu(), H).numpy())
    gt, ut = torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)
    _assert_same(h, torch.nn.functional.gelu(gt, approximate="tanh") * ut, "h vs oracle gate/up + eager gelu*up")


def test_fused_down_quant_consecutive_calls_and_warming(ext, cuda, weights):
    """One control block through calls of changing M (it is left zeroed each time), with
    the quant workgroups that find no row left warming 48 MB of other buffers (read only)."""
    wg, wu = weights
    ctl = _new_ctl(ext, 6208, cuda)
    big = [torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=cuda) for n in (4 << 20,) * 3]
    keep = [t.clone() for t in big]
    for i, m in enumerate((776, 300, 1000, 776)):
        print(f"call {i}: M={m}", flush=True)
        gen = inp.generator(9400 + i)
        q, sa = ext.quantize(inp.activations(gen, m, H).to(cuda))
        h_ref, dq_ref, dsa_ref = _two_launches(ext, q, sa, m, wg, wu)
        h, dq, dsa = _fused(ext, q, sa, m, wg, wu, ctl, warm=big if i % 2 == 0 else ())
        torch.cuda.synchronize()
        _assert_same(h, h_ref, f"call {i} h")
        _assert_same_codes(dq, dq_ref, m, f"call {i}")
        _assert_same(dsa, dsa_ref, f"call {i} scales")
        assert int(ctl.abs().sum()) == 0
    assert all(torch.equal(a, b) for a, b in zip(big, keep))


def test_fused_down_quant_bounded_wait_reports_to_host(ext, cuda, weights):
    """wait_extra = 1: every row block waits for one completion more than the launch makes.
    The waits run out after spin_limit rounds, the kernel still ends, the status word is
    set; after the host zeroes the control block the next call is exact."""
    wg, wu = weights
    lib = ext.load_int4_gemm()
    m = 776
    gen = inp.generator(9500)
    q, sa = ext.quantize(inp.activations(gen, m, H).to(cuda))
    ctl = _new_ctl(ext, m, cuda)
    lib.pi05w4a4_mlp_status(1)
    h, _, _ = _fused(ext, q, sa, m, wg, wu, ctl, spin_limit=4, wait_extra=1)
    torch.cuda.synchronize()
    assert lib.pi05w4a4_mlp_status(0) > 0, "no timed-out wait reached the host"
    h_ref, dq_ref, dsa_ref = _two_launches(ext, q, sa, m, wg, wu)
    _assert_same(h, h_ref, "h (the GEMM tiles never wait)")
    lib.pi05w4a4_mlp_status(1)
    ctl.zero_()
    h, dq, dsa = _fused(ext, q, sa, m, wg, wu, ctl)
    torch.cuda.synchronize()
    assert lib.pi05w4a4_mlp_status(0) == 0
    _assert_same_codes(dq, dq_ref, m, "after the reset")
    _assert_same(dsa, dsa_ref, "scales after the reset")


def test_mlp_op_equals_unfused_ops(ext, cuda, weights):
    """rms_norm_int4_mlp = rms_norm_int4_gemm2_gelu then int4_gemm_residual, bit for bit
    (y and h), at batch 2 x 776 with a down weight; and the status check raises after a
    forced timeout."""
    wg, wu = weights
    gen = inp.generator(9600)
    wd = ext.repack_weight(inp.random_packed(gen, H, N).to(cuda))
    x = (torch.randn(2, 776, H, generator=gen) * 0.5).half().to(cuda)
    nw = (torch.randn(H, generator=gen) * 0.1).half().to(cuda)
    y, h = ext.rms_norm_int4_mlp(x, nw, 1e-6, wg, wu, wd, x, warm=[wd])
    h_ref = ext.rms_norm_int4_gemm2_gelu(x, nw, 1e-6, wg, wu)
    y_ref = ext.int4_gemm_residual(h_ref, wd, x)
    torch.cuda.synchronize()
    _assert_same(h, h_ref, "h")
    _assert_same(y, y_ref, "y")
    with pytest.raises(RuntimeError, match="different|MFMA-layout"):
        ext.rms_norm_int4_mlp(x, nw, 1e-6, wg, wu, inp.random_packed(gen, H, N).to(cuda), x)
