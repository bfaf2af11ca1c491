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
// 16-byte-per-lane loads.  Each byte is re-encoded for the GEMM's one-AND unpack (the
// weight encoding of w4a4_internal.h): the even-k code moves to the high nibble (two's
// complement) and the odd-k code to the low nibble (offset binary).  K is padded to a
// multiple of 128 with zero words.  The fp32 column scales follow the payload, and the
// column corrections wcorr[n] = -128 * (sum of the even-k codes of column n) follow the
// scales.
//
// One thread per destination word: the writes are coalesced, the reads are gathers from
// a layout that is only read once (this runs at load time, not per call).

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

// Reference word (code 8kw+e in nibble e, two's complement) -> weight encoding.
__device__ __forceinline__ int32_t encode_weight_word(int32_t w) {
  const uint32_t u = static_cast<uint32_t>(w);
  return static_cast<int32_t>(((u & kLoNib) << 4) | (((u >> 4) & kLoNib) ^ kObFlipLo));
}

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
      v = encode_weight_word(src[s]);
    }
    dst[idx] = v;
  } else if (idx < payload + n) {
    const int64_t col = idx - payload;
    const int64_t s = (layout == 0) ? col * stride + kw_total
                                    : static_cast<int64_t>(n) * kw_total + col;
    dst[idx] = src[s];
  }
}

// wcorr of one column per wave: 16 * (even-k code sum) of a reference word is the signed
// dot product of its low-nibble bytes 16c with ones.
__global__ __launch_bounds__(256) void weight_corr_kernel(const int32_t* __restrict__ src,
                                                          int32_t layout, int32_t n, int32_t k,
                                                          int64_t stride, int32_t* __restrict__ dst) {
  const int32_t col = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (col >= n) return;
  const int32_t kw_total = k / 8;
  int s16 = 0;
  for (int32_t kw = lane; kw < kw_total; kw += 64) {
    const int64_t s = (layout == 0) ? col * stride + kw : ((kw >> 1) * static_cast<int64_t>(n) + col) * 2 + (kw & 1);
    const uint32_t w = static_cast<uint32_t>(src[s]);
    s16 = __builtin_amdgcn_sdot4(static_cast<int>((w << 4) & kHiNib), 0x01010101, s16, false);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s16 += __shfl_xor(s16, o, 64);
  if (lane == 0) dst[static_cast<int64_t>(n) * kblocks128(k) * 16 + n + col] = -8 * s16;
}

// E3M2 bits of an integer code in [-8, 8]: magnitudes 0, 1, 2, 3, 4, 5, 6, 7, 8 are
// 0, 2^0, 2^1, 1.5 * 2^1, 2^2, 1.25 * 2^2, 1.5 * 2^2, 1.75 * 2^2, 2^3 (exponent field
// e + 3, two mantissa bits), the sign in bit 5.
__device__ __forceinline__ uint32_t e3m2_bits(int c) {
  constexpr uint32_t kMag[9] = {0x00, 0x0c, 0x10, 0x12, 0x14, 0x15, 0x16, 0x17, 0x18};
  return c < 0 ? (0x20u | kMag[-c]) : kMag[c];
}

// INT4 MFMA layout -> E3M2 pair layout (w4a4_internal.h).  One thread per (column, k
// block, 32-code group): it reads the column's 16-byte slot of the INT4 fragment, decodes
// the weight nibbles (even k: high nibble, two's complement; odd k: low nibble, offset
// binary), re-encodes the 32 codes as E3M2 (code j in bits 6j .. 6j+5 of six dwords) and
// writes the dwords into the column pair's 48-byte lane record.  The last N threads copy
// the column scales.  Load time only.
__global__ __launch_bounds__(256) void repack_e3m2_kernel(const int32_t* __restrict__ src, int32_t n, int32_t k,
                                                          int32_t* __restrict__ dst) {
  const int32_t kb128 = kblocks128(k);
  const int64_t slots = static_cast<int64_t>(n) * kb128 * 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx < slots) {
    const int g = static_cast<int>(idx & 3);
    const int64_t kb = (idx >> 2) % kb128;
    const int64_t col = (idx >> 2) / kb128;
    uint32_t d[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = static_cast<uint32_t>(src[frag_word_index(col, static_cast<int32_t>(kb * 16 + 4 * g + i), kb128)]);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (w >> (8 * b)) & 0xffu;
        const int even = static_cast<int>((byte >> 4) ^ 8u) - 8;  // two's complement nibble
        const int odd = static_cast<int>(byte & 15u) - 8;          // offset binary nibble
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int j = 8 * i + 2 * b + h;  // code index in the slot's 32
          const uint32_t f = e3m2_bits(h ? odd : even);
          const int bit = 6 * j;
          d[bit >> 5] |= f << (bit & 31);
          if ((bit & 31) > 26) d[(bit >> 5) + 1] |= f >> (32 - (bit & 31));
        }
      }
    }
    const int64_t pair = col >> 5;
    const int h = static_cast<int>((col >> 4) & 1);
    const int lane = static_cast<int>(col & 15) + 16 * g;
    uint8_t* const base = reinterpret_cast<uint8_t*>(dst) + (pair * kb128 + kb) * kE3m2PairBytes;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int byte_in_record = 4 * (6 * h + i);
      *reinterpret_cast<uint32_t*>(base + (byte_in_record >> 4) * 1024 + 16 * lane + (byte_in_record & 15)) = d[i];
    }
  } else if (idx < slots + n) {
    const int64_t col = idx - slots;
    dst[w6_payload_words(n, kb128) + col] = src[static_cast<int64_t>(n) * kb128 * 16 + col];
  }
}

}  // namespace

hipError_t launch_repack_e3m2(const int32_t* w_mfma, int32_t n, int32_t k, int32_t* dst, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n) * kblocks128(k) * 4 + n;
  repack_e3m2_kernel<<<dim3(static_cast<unsigned>((total + 255) / 256)), 256, 0, stream>>>(w_mfma, n, k, dst);
  return hipGetLastError();
}

hipError_t launch_repack(const int32_t* src, int32_t layout, int32_t n, int32_t k,
                         int64_t src_stride, int32_t* dst, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n) * kblocks128(k) * 16 + n;
  const int64_t blocks = (total + 255) / 256;
  repack_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, stream>>>(src, layout, n, k,
                                                                         src_stride, dst);
  weight_corr_kernel<<<dim3(static_cast<unsigned>((n + 3) / 4)), 256, 0, stream>>>(src, layout, n, k,
                                                                               src_stride, dst);
  return hipGetLastError();
}

}  // namespace w4a4
