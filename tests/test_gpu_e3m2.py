"""GPU parity of the E3M2 (FP6-MFMA) form of the gate/up GEMM.

The E3M2 path holds the same INT4 codes as FP6 E3M2 values and multiplies them with
v_mfma_f32_16x16x128_f8f6f4, whose fp32 sums of integer products are exact.  Bar:
  * the E3M2 quantizers write the same codes and scale bits as the INT4 quantizers (which
    are pinned to the oracle) and as the oracle itself;
  * the E3M2 weight repack holds the same codes and scales as its source;
  * every GEMM output (plain groups, the GELU-tanh*up pair) is bit-identical to the INT4
    path's on the same inputs and to the oracle's int4_gemm_ref;
  * whole forwards with E3M2 gate/up weights equal the INT4 forward bit for bit.
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


def _int4_codes(q: torch.Tensor, m: int, k: int) -> np.ndarray:
    from pi05_fast.w4a4.pack import codes_from_fragment_major

    return orc.unpack_nibbles(inp.to_np(codes_from_fragment_major(q.cpu(), m, k)), k)


def _e3m2_codes(q6: torch.Tensor, m: int, k: int) -> np.ndarray:
    from pi05_fast.w4a4.pack import codes_from_e3m2_fragments

    return inp.to_np(codes_from_e3m2_fragments(q6.cpu(), m, k)).astype(np.int32)


def _same_f16(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("m", [1, 5, 40, 776, 2200])
def test_quantize_e3m2_matches_int4_and_oracle(ext, cuda, m):
    k = 2048
    x = inp.activations(inp.generator(500 + m), m, k)
    q, sa = ext.quantize(x.to(cuda))
    q6, sa6 = ext.quantize_e3m2(x.to(cuda))
    torch.cuda.synchronize()
    c4 = _int4_codes(q, m, k)
    c6 = _e3m2_codes(q6, m, k)
    assert np.array_equal(c6, c4), f"M={m}: {np.count_nonzero(c6 != c4)} codes differ from the INT4 quantizer"
    assert torch.equal(sa.view(torch.int32), sa6.view(torch.int32))
    if m <= 776:
        q_ref, s_ref = orc.quant_activation(x.numpy())
        assert np.array_equal(c6, q_ref.astype(np.int32))
        assert np.array_equal(inp.to_np(sa6).view(np.int32), s_ref.view(np.int32))


def test_quantize_e3m2_many_ties(ext, cuda):
    """Exact half-integer quotients (the reciprocal fast path's exact-division redo)."""
    k, m = 2048, 16
    halves = np.arange(-6.5, 7.0, 1.0)
    y = np.zeros((m, k), np.float64)
    rng = np.random.default_rng(77)
    for r in range(m):
        y[r, 0] = 7.0 if r % 2 == 0 else -7.0
        cols = rng.choice(np.arange(1, k), size=48, replace=False)
        y[r, cols] = rng.choice(halves, size=48)
    y /= 16.0
    x16 = (orc.fwht_unnormalized(y.astype(np.float32)).astype(np.float64) / k).astype(np.float16)
    q6, sa6 = ext.quantize_e3m2(torch.from_numpy(x16).to(cuda))
    torch.cuda.synchronize()
    q_ref, s_ref = orc.quant_activation(x16)
    assert np.array_equal(_e3m2_codes(q6, m, k), q_ref.astype(np.int32))
    assert np.array_equal(inp.to_np(sa6).view(np.int32), s_ref.view(np.int32))


@pytest.mark.parametrize("m", [3, 776])
def test_rms_norm_quantize_e3m2_matches_int4(ext, cuda, m):
    k = 2048
    gen = inp.generator(600 + m)
    x = inp.activations(gen, m, k).to(cuda)
    w = (torch.randn(k, generator=gen) * 0.1).to(torch.float16).to(cuda)
    q, sa = ext.rms_norm_quantize(x, w, 1e-6, True)
    q6, sa6 = ext.quantize_e3m2(x, (w, 1e-6, True))
    torch.cuda.synchronize()
    assert np.array_equal(_e3m2_codes(q6, m, k), _int4_codes(q, m, k))
    assert torch.equal(sa.view(torch.int32), sa6.view(torch.int32))


@pytest.mark.parametrize("m", [3, 776])
def test_rms_norm_quantize_e3m2_cache_warm_changes_nothing(ext, cuda, m):
    """The E3M2 norm + quant with cache warming (a workgroup for each CU the rows leave idle
    reads further buffers) writes the same codes and scales as without, and leaves the
    buffers unchanged."""
    k = 2048
    gen = inp.generator(650 + m)
    x = inp.activations(gen, m, k).to(cuda)
    w = (torch.randn(k, generator=gen) * 0.1).to(torch.float16).to(cuda)
    big = [torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=cuda) for n in (1 << 20,) * 2]
    keep = [t.clone() for t in big]
    q0, s0 = ext.quantize_e3m2(x, (w, 1e-6, True))
    q1, s1 = ext.quantize_e3m2(x, (w, 1e-6, True), warm=big)
    torch.cuda.synchronize()
    assert np.array_equal(_e3m2_codes(q1, m, k), _e3m2_codes(q0, m, k))
    assert torch.equal(s0.view(torch.int32), s1.view(torch.int32))
    for t, t0 in zip(big, keep):
        assert torch.equal(t, t0)


def test_gate_up_op_warming_changes_nothing(ext, cuda, monkeypatch):
    """rms_norm_int4_gemm2_gelu on E3M2 weights at 776 rows, whose norm + quant launch warms
    the up weight's tail, equals the call without warming (PI05_W4A4_CACHE_WARM=0)."""
    m, k, n = 776, 2048, 16384
    gen = inp.generator(660)
    x = inp.activations(gen, m, k).to(cuda)
    nw = (torch.randn(k, generator=gen) * 0.1).to(torch.float16).to(cuda)
    g6, u6 = (ext.repack_weight_e3m2(inp.random_packed(gen, n, k).to(cuda), k=k) for _ in range(2))
    head, tail = ext.gate_up_warm_split(u6)
    assert tail is not None and head.numel() + tail.numel() == u6.numel()
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("PI05_W4A4_CACHE_WARM", flag)
        outs.append(ext.rms_norm_int4_gemm2_gelu(x, nw, 1e-6, g6, u6))
    torch.cuda.synchronize()
    assert _same_f16(outs[0], outs[1])


@pytest.mark.parametrize("n,k", [(64, 2048), (16384, 2048), (96, 4096)])
def test_repack_e3m2_keeps_codes_and_scales(ext, cuda, n, k):
    from pi05_fast.w4a4.pack import codes_from_e3m2_weight

    packed = inp.random_packed(inp.generator(700 + n), n, k)  # all 16 nibbles, -8 included
    w6 = ext.repack_weight_e3m2(packed.to(cuda), k=k)
    torch.cuda.synchronize()
    assert tuple(w6.shape) == (n, 3 * k // 16 + 16) and ext.is_e3m2_layout(w6, k)
    codes, scales = codes_from_e3m2_weight(w6.cpu(), k)
    want_codes = orc.unpack_nibbles(inp.to_np(packed[:, : k // 8]), k)
    assert np.array_equal(inp.to_np(codes).astype(np.int32), want_codes.astype(np.int32))
    assert torch.equal(scales.view(torch.int32), packed[:, k // 8])
    # from the MFMA layout as well
    w6b = ext.repack_weight_e3m2(ext.repack_weight(packed.to(cuda), k=k), k=k)
    assert torch.equal(w6, w6b)


GEMM_M = [1, 17, 64, 113, 200, 776, 2200]


@pytest.mark.parametrize("m", GEMM_M)
def test_gemm2_gelu_e3m2_matches_int4(ext, cuda, m):
    """gate/up + GELU-tanh*up: E3M2 weights against MFMA-layout INT4 weights, bit for bit."""
    k, n = 2048, 16384 if m in (200, 776) else 1024
    gen = inp.generator(800 + m)
    x = inp.activations(gen, m, k).to(cuda)
    wg, wu = (inp.random_packed(gen, n, k).to(cuda) for _ in range(2))
    g4, u4 = ext.repack_weight(wg, k=k), ext.repack_weight(wu, k=k)
    g6, u6 = ext.repack_weight_e3m2(g4, k=k), ext.repack_weight_e3m2(u4, k=k)
    h4 = ext.int4_gemm2_gelu(x, g4, u4)
    h6 = ext.int4_gemm2_gelu(x, g6, u6)
    torch.cuda.synchronize()
    assert _same_f16(h6, h4), f"M={m}: {int((h6.view(torch.int16) != h4.view(torch.int16)).sum())} outputs differ"


@pytest.mark.parametrize("m", GEMM_M)
def test_gemm2_e3m2_matches_int4(ext, cuda, m):
    """Plain gate and up outputs (two groups of one launch), and int4_gemm on one weight."""
    k, n = 2048, 2048
    gen = inp.generator(900 + m)
    x = inp.activations(gen, m, k).to(cuda)
    wa, wb = (inp.random_packed(gen, n, k).to(cuda) for _ in range(2))
    a4, b4 = ext.int4_gemm2(x, ext.repack_weight(wa, k=k), ext.repack_weight(wb, k=k))
    a6w, b6w = ext.repack_weight_e3m2(wa, k=k), ext.repack_weight_e3m2(wb, k=k)
    a6, b6 = ext.int4_gemm2(x, a6w, b6w)
    y6 = ext.int4_gemm(x, a6w)
    torch.cuda.synchronize()
    assert _same_f16(a6, a4) and _same_f16(b6, b4) and _same_f16(y6, a4)


@pytest.mark.parametrize("m,n", [(40, 256), (776, 2048)])
def test_gemm_e3m2_matches_oracle(ext, cuda, m, n):
    """Straight against the CPU oracle: N(0, 0.02) weights, outlier activations."""
    k = 2048
    gen = inp.generator(1000 + m)
    x = inp.activations(gen, m, k)
    packed = inp.packed_weight(gen, n, k)
    y = ext.int4_gemm(x.to(cuda), ext.repack_weight_e3m2(packed.to(cuda), k=k))
    torch.cuda.synchronize()
    want = orc.int4_gemm_ref(x.numpy(), packed.numpy())
    got = inp.to_np(y)
    assert np.array_equal(got.view(np.int16), want.view(np.int16)), f"rel_l2={orc.rel_l2(got, want):.3e}"


def test_gemm3_e3m2_groups(ext, cuda):
    """Three groups of different widths in one launch (tile boundaries between groups)."""
    k, m = 2048, 300
    gen = inp.generator(1100)
    x = inp.activations(gen, m, k).to(cuda)
    ws = [inp.random_packed(gen, n, k).to(cuda) for n in (512, 96, 160)]
    want = ext.int4_gemm3(x, *[ext.repack_weight(w, k=k) for w in ws])
    got = ext.int4_gemm3(x, *[ext.repack_weight_e3m2(w, k=k) for w in ws])
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert _same_f16(g, w)


def test_e3m2_argument_errors(ext, cuda):
    k = 2048
    gen = inp.generator(1200)
    x = inp.activations(gen, 8, k).to(cuda)
    w = inp.random_packed(gen, 64, k).to(cuda)
    w4, w6 = ext.repack_weight(w, k=k), ext.repack_weight_e3m2(w, k=k)
    with pytest.raises(RuntimeError, match="E3M2-layout"):
        ext.int4_gemm2(x, w6, w4)
    with pytest.raises(RuntimeError, match="residual"):
        ext.int4_gemm_residual(x, w6, torch.zeros(8, 64, dtype=torch.float16, device=cuda))
    with pytest.raises(RuntimeError, match="K = 2048"):
        ext.quantize_e3m2(inp.activations(gen, 8, 1024).to(cuda))
    with pytest.raises(RuntimeError, match="N % 32"):
        ext.repack_weight_e3m2(inp.random_packed(gen, 48, k).to(cuda), k=k)


def test_forward_e3m2_equals_int4(cuda, monkeypatch):
    """Two decoder layers at 776 tokens (the fused layer path): gate/up weights in the E3M2
    form (the load-time default) against the INT4 MFMA layout, bit for bit."""
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm, prefix_inputs

    x = prefix_inputs(1, 776, cuda)
    outs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("PI05_W4A4_E3M2", flag)
        model, _ = build_prefix_lm(cuda, num_layers=2)
        gate = model.layers[0].mlp.gate_proj.packed
        assert (int(gate.size(1)) == 3 * 2048 // 16 + 16) == (flag == "1")
        with torch.no_grad():
            outs.append(model(x))
        del model
    torch.cuda.synchronize()
    assert _same_f16(outs[1], outs[0])


@pytest.mark.parametrize("m", [1, 64, 128, 129, 776])
def test_gate_up_loaded_weights_run_int4_twins_at_few_rows(ext, cuda, monkeypatch, m):
    """The loader gives the MLP's gate/up weights the E3M2 form and registers their INT4
    form as its twin: calls of at most E3M2_MAX_INT4_ROWS rows run the INT4 kernels on the
    twins, larger ones the E3M2 kernels; the fp16 outputs equal the INT4-only weights' bit
    for bit either way (plain pair and GELU-tanh*up)."""
    from pi05_fast.w4a4 import apply

    k, n = 2048, 1024
    gen = inp.generator(7100 + m)
    x = inp.activations(gen, m, k).to(cuda)
    wg_ref, wu_ref = inp.packed_weight(gen, n, k), inp.packed_weight(gen, n, k)
    wg, _ = apply.load_time_weight(wg_ref, "model.layers.0.mlp.gate_proj", k, n, cuda)
    wu, _ = apply.load_time_weight(wu_ref, "model.layers.0.mlp.up_proj", k, n, cuda)
    assert ext.is_e3m2_layout(wg, k) and ext.is_e3m2_layout(wu, k)
    assert ext.is_mfma_layout(ext.int4_twin(wg, k), k) and ext.is_mfma_layout(ext.int4_twin(wu, k), k)
    wg4, wu4 = ext.repack_weight(wg_ref.to(cuda)), ext.repack_weight(wu_ref.to(cuda))
    calls = {"e3m2": 0}
    real = ext._run_e3m2

    def counting(*a, **kw):
        calls["e3m2"] += 1
        return real(*a, **kw)

    monkeypatch.setattr(ext, "_run_e3m2", counting)
    y = ext.int4_gemm2_gelu(x, wg, wu)
    g, u = ext.int4_gemm2(x, wg, wu)
    y_ref = ext.int4_gemm2_gelu(x, wg4, wu4)
    g_ref, u_ref = ext.int4_gemm2(x, wg4, wu4)
    torch.cuda.synchronize()
    assert _same_f16(y, y_ref) and _same_f16(g, g_ref) and _same_f16(u, u_ref)
    assert calls["e3m2"] == (0 if m <= ext.E3M2_MAX_INT4_ROWS else 2)
    # an in-place write to the E3M2 weight retires its twin: the call runs on E3M2 weights
    wg.add_(0)
    calls["e3m2"] = 0
    ext.int4_gemm2_gelu(x, wg, wu)
    assert calls["e3m2"] == 1
