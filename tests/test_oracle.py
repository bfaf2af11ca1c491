"""Pinning of the CPU oracle (oracle/w4a4_oracle.py) -- CPU only.

Each oracle function is checked against (a) golden vectors written by the reference's
own CPU code (tests/golden/make_golden.py -> pi05_fast/w4a4/pack.py), and (b) what the
mathematics fixes independently of any implementation: the closed form of the
Sylvester-Hadamard matrix, H.H = K.I, exact integer arithmetic, hand-built known
answers for nibble packing and half-even ties, and int64 brute force for the GEMM.
Each check is chosen so that a dropped term, a wrong sign/index or a transposed
operand fails it (see the planted-mistake tests at the end).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import w4a4_oracle as orc


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.int32 if a.dtype == np.float32 else np.int16)


# ----------------------------------------------------------------------------- FWHT
@pytest.mark.parametrize("n", [8, 64, 2048])
def test_fwht_golden(golden, n):
    got = orc.fwht_unnormalized(golden[f"fwht_in_{n}"])
    assert np.array_equal(_bits(got), _bits(golden[f"fwht_out_{n}"]))


@pytest.mark.parametrize("n", [1, 2, 4, 16, 128, 256])
def test_fwht_closed_form(n):
    """FWHT(x) = H x with H[i, j] = (-1)^popcount(i & j) (float64 brute force)."""
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n)).astype(np.float32)
    i = np.arange(n)
    h = np.where(np.vectorize(lambda v: bin(v).count("1") % 2)(i[:, None] & i[None, :]) == 0, 1.0, -1.0)
    want = x.astype(np.float64) @ h.T
    got = orc.fwht_unnormalized(x).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.sqrt(n))


@pytest.mark.parametrize("n", [2, 32, 1024, 16384])
def test_fwht_involution_and_basis(n):
    """H.H = n.I exactly on small integers; FWHT(e_i) = column i of H."""
    rng = np.random.default_rng(7)
    x = rng.integers(-8, 8, size=(2, n)).astype(np.float32)  # |values| stay < 2^24: exact
    twice = orc.fwht_unnormalized(orc.fwht_unnormalized(x))
    assert np.array_equal(twice, x * n)
    i = int(rng.integers(0, n))
    e = np.zeros((1, n), np.float32)
    e[0, i] = 1.0
    col = orc.fwht_unnormalized(e)[0]
    j = np.arange(n)
    want = np.where(np.array([bin(v).count("1") % 2 for v in (j & i)]) == 0, 1.0, -1.0)
    assert np.array_equal(col, want)


def test_fwht_rejects_non_power_of_two():
    with pytest.raises(ValueError):
        orc.fwht_unnormalized(np.zeros((1, 12), np.float32))


# ----------------------------------------------------------------------------- nibbles
def test_nibble_known_answers():
    codes = np.array([[0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]], np.int32)
    words = orc.pack_nibbles(codes)
    assert words.dtype == np.int32
    assert words[0, 0] == 0x76543210
    assert np.uint32(words[0, 1].view(np.uint32)) == 0xFEDCBA98
    assert np.array_equal(orc.unpack_nibbles(words, 16), codes)


def test_nibble_golden(golden):
    assert np.array_equal(orc.pack_nibbles(golden["nib_codes"]), golden["nib_packed"])
    assert np.array_equal(orc.unpack_nibbles(golden["nib_words"], 40), golden["nib_unpacked"])


def test_nibble_round_trip_all_words():
    rng = np.random.default_rng(3)
    words = rng.integers(-(2**31), 2**31 - 1, size=(4, 64), dtype=np.int64).astype(np.int32)
    assert np.array_equal(orc.pack_nibbles(orc.unpack_nibbles(words, 512)), words)


# ----------------------------------------------------------------------------- activation quant
@pytest.mark.parametrize("k", [64, 192, 512, 1024, 2048, 16384])
def test_quant_activation_golden(golden, k):
    q, s = orc.quant_activation(golden[f"act_x_{k}"])
    assert np.array_equal(q, golden[f"act_q_{k}"])
    assert np.array_equal(_bits(s), _bits(golden[f"act_s_{k}"]))


def test_quant_rotation_set():
    assert orc.should_rotate(1024) and orc.should_rotate(2048) and orc.should_rotate(16384)
    assert not orc.should_rotate(4096) and not orc.should_rotate(64)
    assert orc.should_rotate(64, True) and not orc.should_rotate(2048, False)


def test_quant_half_even_ties():
    """amax = 7 * 2^e makes sdiv = 2^e exactly (the 1e-12 is absorbed); values at (k + 1/2)
    * 2^e are exact ties and must round half to even."""
    e = -3
    step = 2.0**e
    row = np.array([7, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 4.5, 5.5, 6.5, -6.5, 0, 1, -7, 0.25],
                   np.float64) * step
    x = np.tile(row, 4)[None, :].astype(np.float16)  # K = 64, unrotated
    q, s = orc.quant_activation(x)
    assert s[0] == np.float32(step)
    want = np.array([7, 0, 2, 2, 0, -2, -2, 4, 4, 6, 6, -6, 0, 1, -7, 0], np.int8)
    assert np.array_equal(q[0, :16], want)


def test_quant_zero_and_one_hot_rows():
    x = np.zeros((2, 2048), np.float16)
    x[1, 5] = 3.0
    q, s = orc.quant_activation(x)
    assert np.all(q[0] == 0) and s[0] == np.float32(np.float32(1e-12) * orc.inv_sqrt_k(2048))
    # one-hot rotates to a +-3 constant row: every code is +-7 and sdiv = 3/7 + 1e-12
    assert np.all(np.abs(q[1]) == 7)
    sdiv = np.float32(np.float32(3.0) / np.float32(7.0) + np.float32(1e-12))
    assert s[1] == np.float32(sdiv * orc.inv_sqrt_k(2048))


def test_quant_never_emits_minus_eight():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((16, 2048)) * 50).astype(np.float16)
    q, _ = orc.quant_activation(x)
    assert q.min() >= -7 and q.max() <= 7


# ----------------------------------------------------------------------------- weight pack
@pytest.mark.parametrize("shape", [(8, 64), (8, 192), (8, 1024), (16, 2048), (2, 16384)])
def test_pack_linear_weight_golden(golden, shape):
    n, k = shape
    got = orc.pack_linear_weight(golden[f"w_in_{n}x{k}"])
    assert np.array_equal(got, golden[f"w_packed_{n}x{k}"])


def test_pack_linear_weight_reconstructs():
    """Dequantised codes reproduce the (rotated) weight to within half a step."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((4, 1024)) * 0.02).astype(np.float32)
    packed = orc.pack_linear_weight(w)
    q, s, k = orc.unpack_linear_weight(packed)
    assert k == 1024
    wr = orc.fwht_unnormalized(w) * orc.inv_sqrt_k(1024)
    err = np.abs(q * s[:, None] - wr).max(axis=1)
    assert np.all(err <= s * 0.5 * (1 + 1e-5))


# ----------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("m,n,k", [(6, 8, 64), (8, 16, 2048), (4, 2, 16384), (6, 8, 1024)])
def test_int4_gemm_ref_golden(golden, m, n, k):
    y = orc.int4_gemm_ref(golden[f"act_x_{k}"][:m], golden[f"w_packed_{n}x{k}"])
    assert np.array_equal(_bits(y), _bits(golden[f"gemm_y_{m}x{n}x{k}"]))


def test_gemm_acc_brute_force():
    rng = np.random.default_rng(11)
    a = rng.integers(-7, 8, size=(5, 192)).astype(np.int8)
    b = rng.integers(-8, 8, size=(7, 192)).astype(np.int8)
    want = np.array([[int(sum(int(a[i, t]) * int(b[j, t]) for t in range(192))) for j in range(7)]
                     for i in range(5)])
    assert np.array_equal(orc.gemm_acc_int32(a, b), want)


def test_dequant_order():
    """fp16((acc * sa) * sw): two fp32 roundings then one fp16 rounding."""
    acc = np.array([[123457, -99991]], np.int32)
    sa = np.array([np.float32(0.0123)], np.float32)
    sw = np.array([np.float32(0.0371), np.float32(0.0029)], np.float32)
    y = orc.dequant_fp16(acc, sa, sw)
    want = ((acc.astype(np.float32) * sa[0]).astype(np.float32) * sw).astype(np.float16)
    assert np.array_equal(_bits(y), _bits(want))


# ----------------------------------------------------------------------------- layouts
def test_preshuffle_golden_and_round_trip(golden):
    pre = orc.preshuffle_wmma_weight(golden["pre_in"], 64)
    assert np.array_equal(pre, golden["pre_out"])
    assert pre.shape == (7, 64 // 8 + 9)
    assert np.array_equal(orc.unshuffle_wmma_weight(pre, 64), golden["pre_in"])


def test_inv_sqrt_k_constants(golden):
    got = np.array([orc.inv_sqrt_k(k) for k in (1024, 2048, 16384)], np.float32)
    assert np.array_equal(got, golden["inv_sqrt_k"])
    assert orc.inv_sqrt_k(2048) == np.float32(1.0 / math.sqrt(2048))


# ----------------------------------------------------------------------------- planted mistakes
def test_checks_catch_planted_mistakes(golden):
    """Plausible mistakes in the oracle must fail the pinning checks above."""
    x = golden["act_x_2048"]
    q_ref, s_ref = golden["act_q_2048"], golden["act_s_2048"]

    def quant_with(fwht, scale_op):
        xf = fwht(x.astype(np.float32))
        sdiv = (np.abs(xf).max(axis=-1) / np.float32(7.0) + np.float32(1e-12)).astype(np.float32)
        return np.clip(np.rint(xf / sdiv[:, None]), -7, 7).astype(np.int8), scale_op(sdiv)

    def fwht_descending(v):  # stages in the wrong order
        n = v.shape[-1]
        out = v.copy()
        h = n // 2
        while h >= 1:
            w = out.reshape(*v.shape[:-1], n // (2 * h), 2, h)
            out = np.stack((w[..., 0, :] + w[..., 1, :], w[..., 0, :] - w[..., 1, :]), -2).reshape(v.shape)
            h //= 2
        return out

    def fwht_sign_flip(v):  # (a - b, a + b) instead of (a + b, a - b)
        return -orc.fwht_unnormalized(-v)[..., ::-1].copy()

    good_scale = lambda sd: (sd * orc.inv_sqrt_k(2048)).astype(np.float32)  # noqa: E731
    rsqrt_scale = lambda sd: (sd * np.float32(1.0) / np.sqrt(np.float32(2048))).astype(np.float32)  # noqa: E731
    q, s = quant_with(orc.fwht_unnormalized, good_scale)
    assert np.array_equal(q, q_ref) and np.array_equal(_bits(s), _bits(s_ref))
    q, _ = quant_with(fwht_sign_flip, good_scale)
    assert not np.array_equal(q, q_ref)
    w = golden["fwht_in_2048"]
    assert not np.array_equal(_bits(fwht_descending(w)), _bits(golden["fwht_out_2048"]))
    _, s = quant_with(orc.fwht_unnormalized, lambda sd: sd)  # dropped 1/sqrt(K)
    assert not np.array_equal(_bits(s), _bits(s_ref))
    del rsqrt_scale
    # transposed weight codes in the GEMM
    y = orc.int4_gemm_ref(golden["act_x_2048"][:8], golden["w_packed_16x2048"])
    q_w, s_w, _ = orc.unpack_linear_weight(golden["w_packed_16x2048"])
    qa, sa = orc.quant_activation(golden["act_x_2048"][:8])
    y_bad = orc.dequant_fp16(orc.gemm_acc_int32(qa, q_w[:, ::-1]), sa, s_w)
    assert np.array_equal(_bits(y), _bits(golden["gemm_y_8x16x2048"]))
    assert not np.array_equal(_bits(y_bad), _bits(golden["gemm_y_8x16x2048"]))


# ----------------------------------------------------------------------------- GELU
def _gelu_inputs() -> np.ndarray:
    x = np.concatenate([np.linspace(-12.0, 12.0, 240001), np.random.default_rng(5).standard_normal(50000) * 3.0,
                        [0.0, -0.0, 1e-30, -1e-30, 6e-8, -6e-8, 40.0, -40.0, 65504.0, -65504.0]])
    # every finite fp16 value too: the GPU epilogue's inputs are fp16 gates
    f16 = np.arange(2**16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return np.concatenate([x, f16[np.isfinite(f16)].astype(np.float64)])


def _gelu_close(a: np.ndarray, b: np.ndarray, x: np.ndarray) -> np.ndarray:
    """float64 agreement: gelu = 0.5 x (1 + tanh(u)) loses absolute precision in 1 + tanh(u)
    near tanh = -1 (about 2^-53 |x| per rounding), hence the |x|-scaled absolute term."""
    return np.abs(a - b) <= 1e-14 * np.abs(b) + 1e-15 * np.abs(x)


def test_gelu_tanh_matches_torch_float64():
    """gelu_tanh is torch.nn.functional.gelu(approximate="tanh") (transformers' GELUTanh,
    the act_fn of the reference MLP, apply.py:138) in float64 on the CPU."""
    import torch

    x = _gelu_inputs()
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    got = orc.gelu_tanh(x)
    assert _gelu_close(got, want, x).all()
    assert np.array_equal(np.signbit(got[x == 0]), np.signbit(x[x == 0]))  # gelu(-0) = -0


def test_gelu_tanh_closed_forms():
    """gelu(0) = 0, gelu(x) -> x for large x and -> 0 for large negative x, and the odd
    part: gelu(x) - gelu(-x) = x exactly in real arithmetic (tanh is odd)."""
    assert orc.gelu_tanh(np.array([0.0]))[0] == 0.0
    assert orc.gelu_tanh(np.array([30.0]))[0] == 30.0
    assert abs(orc.gelu_tanh(np.array([-30.0]))[0]) < 1e-300 or orc.gelu_tanh(np.array([-30.0]))[0] == 0.0
    x = np.linspace(-6.0, 6.0, 1201)
    assert np.allclose(orc.gelu_tanh(x) - orc.gelu_tanh(-x), x, rtol=0, atol=1e-14)


def test_gelu_planted_mistakes_fail():
    """A wrong cubic coefficient, the erf form or a dropped 1/2 each fail the torch check."""
    import torch

    x = _gelu_inputs()
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    c = math.sqrt(2.0 / math.pi)
    bad_coeff = 0.5 * x * (1.0 + np.tanh(c * (x + 0.0447 * x**3)))
    bad_erf = torch.nn.functional.gelu(torch.from_numpy(x)).numpy()
    bad_half = x * (1.0 + np.tanh(c * (x + 0.044715 * x**3)))
    for bad in (bad_coeff, bad_erf, bad_half):
        assert not _gelu_close(bad, want, x).all()


# ----------------------------------------------------------------------------- RMSNorm
def _torch_gemma_rms_norm(x16: np.ndarray, w16: np.ndarray, eps: float) -> np.ndarray:
    """transformers' GemmaRMSNorm on the CPU (fp32 inside, (1 + w), fp16 out)."""
    import torch
    from transformers.models.gemma.modeling_gemma import GemmaRMSNorm

    k = x16.shape[-1]
    mod = GemmaRMSNorm(k, eps=eps)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w16.astype(np.float32)))
        return mod(torch.from_numpy(x16)).numpy()  # fp16 in -> fp16 out (type_as)


@pytest.mark.parametrize("m,k,scale", [(64, 2048, 1.0), (16, 2048, 30.0), (8, 1024, 0.01)])
def test_rms_norm_lanes_matches_gemma_module(m, k, scale):
    """Within one fp16 ulp of transformers' module (only the fp32 summation order and
    rsqrt vs 1/sqrt differ), on a small fraction of elements."""
    rng = np.random.default_rng(m + k)
    x = (rng.standard_normal((m, k)) * scale).astype(np.float16)
    w = (rng.standard_normal(k) * 0.1).astype(np.float16)
    got = orc.rms_norm_lanes(x, w, 1e-6)
    want = _torch_gemma_rms_norm(x, w, 1e-6)
    ulps = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert int(ulps.max()) <= 1
    assert float((ulps > 0).mean()) <= 5e-3


def test_rms_norm_lanes_closed_forms():
    """Rows of one repeated value c: mean(x^2) = c^2 exactly, so h = fp16(c * r * g) with
    r = 1 / sqrt(c^2 + eps) computed in float64 and rounded like the fp32 steps; zero rows
    give zeros; the unit offset is (1 + w)."""
    k = 2048
    eps = 1e-6
    for c in (1.0, -2.0, 0.5, 3.0):
        x = np.full((1, k), c, np.float16)
        w = np.zeros(k, np.float16)
        got = orc.rms_norm_lanes(x, w, eps).astype(np.float64)
        assert np.allclose(got, c / math.sqrt(c * c + eps), rtol=2**-10)
        w_half = np.full(k, -0.5, np.float16)  # g = 1 + w = 0.5
        got_half = orc.rms_norm_lanes(x, w_half, eps).astype(np.float64)
        assert np.allclose(got_half, 0.5 * c / math.sqrt(c * c + eps), rtol=2**-10)
        got_plain = orc.rms_norm_lanes(x, np.full(k, 2.0, np.float16), eps, unit_offset=False)
        assert np.allclose(got_plain.astype(np.float64), 2.0 * c / math.sqrt(c * c + eps), rtol=2**-10)
    assert not orc.rms_norm_lanes(np.zeros((2, k), np.float16), np.ones(k, np.float16), eps).any()


def test_rms_norm_lanes_sum_order():
    """The lane-order sum of squares stays within fp32 summation error of float64 (a
    dropped lane or a wrong butterfly partner would be off by a whole lane's share)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((32, 2048)).astype(np.float16)
    v = x.astype(np.float64)
    w = np.zeros(2048, np.float16)
    h = orc.rms_norm_lanes(x, w, 0.0).astype(np.float64)
    r = 1.0 / np.sqrt((v * v).mean(axis=1))
    assert np.allclose(h, v * r[:, None], rtol=2**-10, atol=2**-14)


@pytest.mark.parametrize("m,k,n", [(5, 64, 16), (17, 2048, 48), (3, 16384, 16), (24, 192, 8), (40, 1024, 32)])
def test_torch_cpu_baseline_matches_numpy_oracle(m, k, n):
    """The PyTorch-CPU restatement that bench.py times (both integer matmul forms) gives the
    numpy oracle's codes, scale bits and fp16 outputs bit for bit."""
    import torch

    from oracle import w4a4_torch_cpu as tcpu

    rng = np.random.default_rng(m * 131 + k + n)
    x = rng.standard_normal((m, k), dtype=np.float32)
    x[:, rng.permutation(k)[: max(1, k // 100)]] *= 20.0
    x = x.astype(np.float16)
    packed = orc.pack_linear_weight(rng.standard_normal((n, k), dtype=np.float32) * 0.02)
    q_ref, s_ref = orc.quant_activation(x)
    q, s = tcpu.quant_activation(torch.from_numpy(x))
    assert np.array_equal(q.numpy(), q_ref)
    assert np.array_equal(s.numpy().view(np.int32), s_ref.view(np.int32))
    want = orc.int4_gemm_ref(x, packed)
    for method in ("fp32", "int_mm"):
        if method == "int_mm" and m <= 16:
            continue  # torch._int_mm takes more than 16 rows
        (y,) = tcpu.int4_gemm_ref(torch.from_numpy(x), [torch.from_numpy(packed)], method)
        assert np.array_equal(y.numpy().view(np.int16), want.view(np.int16)), method


def test_torch_cpu_unpack_all_nibbles():
    """Every nibble value (including -8) unpacks as the numpy oracle does."""
    import torch

    from oracle import w4a4_torch_cpu as tcpu

    words = np.arange(-(2**31), 2**31, 2**20 + 12345, dtype=np.int64).astype(np.int32)[:256].reshape(16, 16)
    packed = np.concatenate([words, np.full((16, 1), np.float32(0.5).view(np.int32), np.int32)], axis=1)
    q, s = tcpu.unpack_weight(torch.from_numpy(packed))
    q_ref, s_ref, _ = orc.unpack_linear_weight(packed)
    assert np.array_equal(q.numpy(), q_ref) and np.array_equal(s.numpy(), s_ref)
