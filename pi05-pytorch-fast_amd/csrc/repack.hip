// One-time repack of packed INT4 weights into the gfx950 MFMA-fragment-major layout.
//
// Source layouts (reference addressing, pi05_fast/w4a4/csrc/int4_gemm.cu:44-61):
//   row-major  L1 [N, K/8+1] / L2 [N, K/8+P]: word (n, kw) at n*stride + kw, scale at
//              n*stride + K/8 (pack.py:85-101, apply.py:68-69);
//   WMMA-tiled L3 [N, K/8+9] read flat: word (n, kw) at ((kw>>1)*N + n)*2 + (kw&1),
//              scale at N*K/8 + n (pack.py:45-68).
//
// Destination (this library's layout, frag_word_index in w4a4_internal.h): for every
// 16-column block and 128-deep k block one contiguous 1 KB fragment of 64 16-byte slots,
// slot L = codes 32*(L/16) .. +31 of column 16*nb + L%16.  Fragments of one column block
// are consecutive along K, so a wave streams its weights with fully coalesced
// 16-byte-per-lane loads.  K is padded to a multiple of 128 with zero codes; the fp32
// column scales follow the payload.
//
// One thread per destination word: the writes are coalesced, the reads are gathers from
// a layout that is only read once (this runs at load time, not per call).

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

__global__ __launch_bounds__(256) void repack_kernel(const int32_t* __restrict__ src, int32_t layout,
                                                     int32_t n, int32_t k, int64_t stride,
                                                     int32_t* __restrict__ dst) {
  const int32_t kw_total = k / 8;
  const int32_t kb128 = kblocks128(k);
  const int64_t payload = static_cast<int64_t>(n) * kb128 * 16;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx < payload) {
    // Invert frag_word_index: idx = (nb*kb128 + kb2)*256 + slot*4 + kw%4, slot = col%16 +
    // 16*((kw%16)/4).
    const int64_t frag = idx >> 8;
    const int64_t kb2 = frag % kb128;
    const int64_t nb = frag / kb128;
    const int slot = static_cast<int>((idx >> 2) & 63);
    const int64_t col = nb * 16 + (slot & 15);
    const int64_t kw = kb2 * 16 + (slot >> 4) * 4 + (idx & 3);
    int32_t v = 0;
    if (kw < kw_total) {
      const int64_t s = (layout == 0) ? col * stride + kw : ((kw >> 1) * n + col) * 2 + (kw & 1);
      v = src[s];
    }
    dst[idx] = v;
  } else if (idx < payload + n) {
    const int64_t col = idx - payload;
    const int64_t s = (layout == 0) ? col * stride + kw_total
                                    : static_cast<int64_t>(n) * kw_total + col;
    dst[idx] = src[s];
  }
}

}  // namespace

hipError_t launch_repack(const int32_t* src, int32_t layout, int32_t n, int32_t k,
                         int64_t src_stride, int32_t* dst, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n) * kblocks128(k) * 16 + n;
  const int64_t blocks = (total + 255) / 256;
  repack_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, stream>>>(src, layout, n, k,
                                                                         src_stride, dst);
  return hipGetLastError();
}

}  // namespace w4a4
