"""The allocation-free entry point pi05w4a4_int4_gemm_noalloc on the GPU, through the C ABI:
its output equals pi05w4a4_int4_gemm's (caller-allocated codes, scales and split-K
workspace) bit for bit, and the oracle's, over consecutive calls that reuse the library's
device scratch -- a large call, then smaller ones (one of them through the split-K
partials), so that stale scratch contents from the previous call are present.  A call
that needs more scratch than the library holds is refused before any launch."""

from __future__ import annotations

import ctypes

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


def _with_buffers(ext, lib, x, w, n, stream):
    """pi05w4a4_int4_gemm with torch-allocated codes, scales and workspace."""
    m, k = x.shape
    q = torch.empty(int(lib.pi05w4a4_q_words(m, k)), dtype=torch.int32, device=x.device)
    sa = torch.empty(m, dtype=torch.float32, device=x.device)
    wsb = int(lib.pi05w4a4_gemm_workspace_bytes(m, k, 1, (ctypes.c_int32 * 1)(n), 0))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=x.device)
    y = torch.empty(m, n, dtype=torch.float16, device=x.device)
    rc = lib.pi05w4a4_int4_gemm(x.data_ptr(), m, k, w.data_ptr(), n, y.data_ptr(), q.data_ptr(), sa.data_ptr(),
                                ws.data_ptr(), wsb, stream)
    assert rc == 0, lib.pi05w4a4_last_error()
    return y, wsb


def test_noalloc_matches_int4_gemm(ext, cuda):
    lib = ext.load_int4_gemm()
    stream = torch.cuda.current_stream().cuda_stream
    # large, then smaller; (3, 16384, 2048) runs through the split-K partials
    shapes = [(776, 16384, 2048), (40, 2048, 256), (3, 16384, 2048), (1, 2048, 2560)]
    used_split = False
    for i, (m, k, n) in enumerate(shapes):
        print(f"noalloc call {i}: M={m} K={k} N={n}", flush=True)
        gen = inp.generator(600 + i)
        x = (inp.activations(gen, m, k) if k == 2048 else inp.geglu_activations(gen, m, k))
        packed = inp.random_packed(gen, n, k)
        w = ext.repack_weight(packed.to(cuda), k=k)
        xd = x.to(cuda)
        want, wsb = _with_buffers(ext, lib, xd, w, n, stream)
        used_split |= wsb > 0
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
        rc = lib.pi05w4a4_int4_gemm_noalloc(xd.data_ptr(), m, k, w.data_ptr(), n, y.data_ptr(), stream)
        assert rc == 0, lib.pi05w4a4_last_error()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), f"call {i}: differs from pi05w4a4_int4_gemm"
        ref = orc.int4_gemm_ref(x.numpy(), packed.numpy())
        assert np.array_equal(y.cpu().numpy().view(np.int16), ref.view(np.int16)), f"call {i}: differs from the oracle"
    assert used_split, "no call went through the split-K partials"


def test_noalloc_refuses_oversized_calls(ext, cuda):
    lib = ext.load_int4_gemm()
    m, k, n = 8192, 16384, 2048  # 64 MiB of codes alone
    w = torch.zeros(n, k // 8 + 16, dtype=torch.int32, device=cuda)
    x = torch.zeros(1, dtype=torch.float16, device=cuda)
    rc = lib.pi05w4a4_int4_gemm_noalloc(x.data_ptr(), m, k, w.data_ptr(), n, x.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
    assert rc != 0
    assert b"bytes of scratch" in lib.pi05w4a4_last_error()
