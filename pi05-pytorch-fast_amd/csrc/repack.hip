// One-time repack of packed INT4 weights into the gfx950 MFMA-fragment-major layout.
//
// Source layouts (reference addressing, pi05_fast/w4a4/csrc/int4_gemm.cu:44-61):
//   row-major  L1 [N, K/8+1] / L2 [N, K/8+P]: word (n, kw) at n*stride + kw, scale at
//              n*stride + K/8 (pack.py:85-101, apply.py:68-69);
//   WMMA-tiled L3 [N, K/8+9] read flat: word (n, kw) at ((kw>>1)*N + n)*2 + (kw&1),
//              scale at N*K/8 + n (pack.py:45-68).
//
// Destination (this library's layout): the B operand of v_mfma_i32_16x16x64_i8 for a
// 16-column block nb and a 64-deep k block kb is one contiguous 512-byte fragment;
// lane L of the wave reads words 2L, 2L+1 of it, which hold the 16 codes of column
// 16*nb + L%16 at k = 64*kb + 16*(L/16) .. +15.  Fragments of one column block are
// consecutive along K, so a wave streams its weights with fully coalesced 8-byte-per-
// lane loads.  The fp32 column scales follow the payload.

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

__global__ __launch_bounds__(256) void repack_kernel(const int32_t* __restrict__ src, int32_t layout,
                                                     int32_t n, int32_t k, int64_t stride,
                                                     int32_t* __restrict__ dst) {
  const int64_t kw_total = k / 8;
  const int64_t payload = static_cast<int64_t>(n) * kw_total;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx < payload) {
    const int64_t pair = idx >> 1;
    const int j = static_cast<int>(idx & 1);
    const int lane = static_cast<int>(pair & 63);
    const int64_t blk = pair >> 6;
    const int64_t kb64 = k / 64;
    const int64_t kb = blk % kb64;
    const int64_t nb = blk / kb64;
    const int64_t col = nb * 16 + (lane & 15);
    const int64_t kw = kb * 8 + 2 * (lane >> 4) + j;
    const int64_t s = (layout == 0) ? col * stride + kw : ((kw >> 1) * n + col) * 2 + (kw & 1);
    dst[idx] = src[s];
  } else if (idx < payload + n) {
    const int64_t col = idx - payload;
    const int64_t s = (layout == 0) ? col * stride + kw_total : payload + col;
    dst[idx] = src[s];
  }
}

}  // namespace

hipError_t launch_repack(const int32_t* src, int32_t layout, int32_t n, int32_t k,
                         int64_t src_stride, int32_t* dst, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n) * (k / 8) + n;
  const int64_t blocks = (total + 255) / 256;
  repack_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, stream>>>(src, layout, n, k,
                                                                         src_stride, dst);
  return hipGetLastError();
}

}  // namespace w4a4
