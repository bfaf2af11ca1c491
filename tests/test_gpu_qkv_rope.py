"""The QKV GEMM with the attention prep in its epilogue (pi05w4a4_gemm_qkv_rope, ops
rms_norm_int4_gemm3_rope / prefix_attention_o_proj_kv) against the separate path it
replaces: rms_norm_int4_gemm3, then the K/V prep kernel (pinned to transformers'
apply_rotary_pos_emb in test_gpu_attention.py), then the attention.  Everything must be
equal bit for bit: q, v, the key states and the fragment-major K/V^T (pad keys included),
and the attention + o-proj output that reads them.  Shapes: the forward's 776 tokens, batch
2 and 8 (rows of one 8-row group never straddle two batches), short and long sequences, and
sequence lengths that are not multiples of 64 (zeroed pad keys) or of 32."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc
from tests.test_gpu_prefix_lm import ROPE_PAIR_DIM, _row_major

pytestmark = pytest.mark.gpu

H = 2048


@pytest.fixture(scope="module")
def ext():
    from pi05_fast.w4a4 import extension

    extension.load_int4_gemm()
    return extension


def _weights(ext, cuda, gen):
    out = []
    for n in (2048, 256, 256):
        w = torch.randn(n, H, generator=gen) * 0.02
        out.append(ext.repack_weight(torch.from_numpy(orc.pack_linear_weight(w.numpy())).to(cuda)))
    return out


def _rope_tables(gen, b, s, cuda):
    pos = torch.arange(s, dtype=torch.float32)[None, :].repeat(b, 1) + torch.randint(0, 5, (b, 1), generator=gen)
    inv = 1.0 / (10000 ** (torch.arange(0, 256, 2, dtype=torch.float32) / 256))
    f = pos[..., None] * inv
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().half().to(cuda), emb.sin().half().to(cuda)


# Tile layouts reached (capi.hip make_plan, N = 2560, 256 CUs): 7x4K4 (four waves split K,
# reduce-scatter before the RoPE / V^T epilogue) at 3 x 776; 4x4K4 (64 x 64, four waves
# split K) at 1 x 776 and 8 x 776 (M = 6208); 4x2 at 2 x 776, 1 x 1000 and 1 x 1024;
# 2x2 at 3 x 24 and 2 x 40; the small-M K-split tiles 1x2K4 at 1 x 8, 2x2K4 at 1 x 24 and
# 4 x 8, 4x2K4 at 1 x 64.
CASES = [(1, 776), (2, 776), (8, 776), (3, 776), (1, 8), (1, 24), (4, 8), (3, 24), (1, 64), (2, 40), (1, 1000),
         (1, 1024)]


@pytest.mark.parametrize("b,s", CASES)
def test_qkv_rope_equals_separate_prep(ext, cuda, b, s):
    print(f"qkv rope: B={b} S={s}", flush=True)
    gen = torch.Generator().manual_seed(4100 + 7 * b + s)
    wq, wk, wv = _weights(ext, cuda, gen)
    x = (torch.randn(b, s, H, generator=gen) * 0.5).half().to(cuda)
    nw = (torch.randn(H, generator=gen) * 0.1).half().to(cuda)
    cos, sin = _rope_tables(gen, b, s, cuda)
    wk_rope = ext.rope_pair_weight(wk)
    q1, k1, v1 = ext.rms_norm_int4_gemm3(x, nw, 1e-6, wq, wk, wv)
    kr1 = torch.empty(b, 1, s, 256, dtype=torch.float16, device=cuda)
    lib = ext.load_int4_gemm()
    kv1 = torch.empty(int(lib.pi05w4a4_attn_kv_mfma_elems(b, s, 1, 256)), dtype=torch.float16, device=cuda)
    kv1.fill_(1.0)  # every element is written (pad keys with zeros)
    cs, sn = ext._rope_tables(cos, sin, b, s)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.pi05w4a4_attn_kv_prep(k1.data_ptr(), v1.data_ptr(), 256, cs.data_ptr(), sn.data_ptr(), b, s, 1, 256,
                                     kr1.data_ptr(), kv1.data_ptr(), st) == 0
    q2, kr2, v2, kv2 = ext.rms_norm_int4_gemm3_rope(x, nw, 1e-6, wq, wk_rope, wv, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(v1, v2)
    assert torch.equal(kr1, kr2), "key states"
    assert kv2.shape == kv1.shape
    nbad = int((kv1.view(torch.int16) != kv2.view(torch.int16)).sum())
    assert nbad == 0, f"{nbad}/{kv1.numel()} fragment-major K/V^T elements differ"


@pytest.mark.parametrize("b,s", [(1, 776), (2, 136)])
def test_attention_from_epilogue_layout_equals_separate_prep(ext, cuda, b, s):
    gen = torch.Generator().manual_seed(4200 + s)
    wq, wk, wv = _weights(ext, cuda, gen)
    w_o = _weights(ext, cuda, gen)[0]
    x = (torch.randn(b, s, H, generator=gen) * 0.5).half().to(cuda)
    nw = (torch.randn(H, generator=gen) * 0.1).half().to(cuda)
    cos, sin = _rope_tables(gen, b, s, cuda)
    mask = torch.zeros(b, 1, s, s, dtype=torch.float16, device=cuda)
    mask[:, :, :, s - 5:] = float("-inf")
    scaling = 256 ** -0.5
    q1, k1, v1 = ext.rms_norm_int4_gemm3(x, nw, 1e-6, wq, wk, wv)
    y1, kr1, out1 = ext.prefix_attention_o_proj(q1, k1, v1, cos, sin, mask, scaling, 8, 1, w_o, x)
    q2, kr2, v2, kv2 = ext.rms_norm_int4_gemm3_rope(x, nw, 1e-6, wq, ext.rope_pair_weight(wk), wv, cos, sin)
    y2, out2 = ext.prefix_attention_o_proj_kv(q2, v2, kv2, cos, sin, mask, scaling, 8, w_o, x)
    y3, out3 = ext.prefix_attention_o_proj_kv(q2, v2, kv2, cos, sin, mask, scaling, 8, w_o, x, return_out=False)
    torch.cuda.synchronize()
    assert torch.equal(kr1, kr2)
    assert torch.equal(out1, out2)
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    assert out3.numel() == 0


def test_rope_pair_weight_permutes_blocks(ext, cuda):
    gen = torch.Generator().manual_seed(4300)
    w = torch.randn(256, H, generator=gen) * 0.02
    packed = torch.from_numpy(orc.pack_linear_weight(w.numpy()))
    wm = ext.repack_weight(packed.to(cuda))
    wp = ext.rope_pair_weight(wm)
    torch.cuda.synchronize()
    rm, rp = _row_major(wm, H), _row_major(wp, H)
    # output channel gc of the permuted weight is channel ROPE_PAIR_DIM[gc] of the source
    assert np.array_equal(rp, rm[ROPE_PAIR_DIM])
    x = (torch.randn(40, H, generator=gen)).half()
    a = orc.int4_gemm_ref(x.numpy(), rm)
    bp = orc.int4_gemm_ref(x.numpy(), rp)
    assert np.array_equal(a[:, ROPE_PAIR_DIM], bp)


def test_qkv_rope_rejects_bad_calls(ext, cuda):
    gen = torch.Generator().manual_seed(4400)
    wq, wk, wv = _weights(ext, cuda, gen)
    wk_rope = ext.rope_pair_weight(wk)
    nw = torch.ones(H, dtype=torch.float16, device=cuda)
    x = torch.randn(1, 20, H, generator=gen).half().to(cuda)  # 20 tokens: not a multiple of 8
    cos, sin = _rope_tables(gen, 1, 20, cuda)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ext.rms_norm_int4_gemm3_rope(x, nw, 1e-6, wq, wk_rope, wv, cos, sin)
    x = torch.randn(1, 16, H, generator=gen).half().to(cuda)
    cos, sin = _rope_tables(gen, 1, 16, cuda)
    with pytest.raises(RuntimeError, match="one KV head of 256"):
        ext.rms_norm_int4_gemm3_rope(x, nw, 1e-6, wq, wq, wv, cos, sin)
    with pytest.raises(RuntimeError, match="rope_pair_weight takes"):
        ext.rope_pair_weight(wq)
