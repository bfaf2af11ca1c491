// Shared device code of the activation quantizers: the Sylvester FWHT of one row held in
// registers (passes of register butterflies with LDS transposes between them), the
// per-token INT4 quantization and the stores of the codes, the scale and the row
// correction.  Used by quant_rot.hip (one row per workgroup or per wave) and by the
// prefix attention kernel, whose workgroup quantizes the o-proj input rows it produced.
#pragma once

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// 16 * (sum of the four codes in the high nibbles of w, the odd-k codes): a signed dot
// product of the bytes 16c with ones.
__device__ __forceinline__ int odd_code_sum16(uint32_t w) {
  return __builtin_amdgcn_sdot4(static_cast<int>(w & kHiNib), 0x01010101, 0, false);
}

// Sum over the T threads of a row (T / 64 waves); the result is valid in thread 0.
template <int T>
__device__ __forceinline__ int row_sum(int v, int* red) {
  v = wave_sum(v);
  if constexpr (T > 64) {
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int i = 1; i < T / 64; ++i) v += red[i];
  }
  return v;
}

// Eight codes clamp(rint(v / sdiv), -7, 7) packed as nibbles 0..7 of one word (two's
// complement; the stores flip the low nibbles to offset binary).
__device__ __forceinline__ int32_t quant_pack8(const float (&v)[8], float sdiv) {
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = __builtin_rintf(__fdiv_rn(v[e], sdiv));
    r = fminf(fmaxf(r, -7.0f), 7.0f);
    word |= (static_cast<uint32_t>(static_cast<int>(r)) & 0xFu) << (4 * e);
  }
  return static_cast<int32_t>(word);
}

// Same eight codes without a division per element.  qa = v * rcp(sdiv) differs from the
// exact quotient q = v / sdiv by less than 2e-6 (|q| <= 7 and the hardware reciprocal
// and the product each round within an ulp or two), so rint(qa) == rint(q) unless q lies
// within 2e-6 of a half-integer.  Any lane that sees qa within 1e-5 of one raises
// `near_tie`; the caller then redoes the row's codes with quant_pack8 (exact division).
// Both paths therefore produce the reference's round-half-even codes bit for bit.
__device__ __forceinline__ int32_t quant_pack8_rcp(const float (&v)[8], float rcp,
                                                   bool& near_tie) {
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float qa = v[e] * rcp;
    float r = __builtin_rintf(qa);
    near_tie |= fabsf(qa - r) > 0.49999f;
    r = fminf(fmaxf(r, -7.0f), 7.0f);
    word |= (static_cast<uint32_t>(static_cast<int>(r)) & 0xFu) << (4 * e);
  }
  return static_cast<int32_t>(word);
}

// Rotation, quantization and stores of one row of K = 2^LOGK values held by T = 2^LOGT
// threads, R = K/T consecutive values per thread (thread t: elements t*R .. t*R + R - 1).
// The log2(K) butterfly stages run in passes of r = log2(R) consecutive stride bits, each
// pass entirely in registers, with an LDS transpose between passes that re-deals the row
// so that the next pass's stride bits index a thread's registers.  Stages still run in
// increasing order of the stride h and each one writes (a + b, a - b), so the rotated
// values are bit-identical to the CPU transform.  Pass p covers element bits
// [lo, lo + w): register j of thread t holds element e_p(t, j), whose bits [lo, lo + w)
// are j mod 2^w and whose other bits, in increasing order, are (t << (r - w)) | (j >> w).
// After the last pass each thread holds runs of 2^(r - w) >= 8 consecutive elements,
// which it packs into code words directly.  L: K + 4*(K/R) floats of LDS for this row
// (4 pad floats per R keep the transposes nearly bank-conflict free); red/ired: T/64
// floats/ints of LDS when T > 64.  With T == 64 the row belongs to one wave and nothing
// here waits on other waves.
template <int LOGK, int LOGT>
__device__ __forceinline__ void fwht_quant_row(float (&v)[1 << (LOGK - LOGT)], float* L, float* red,
                                               int* ired, int t, int64_t row, int32_t* __restrict__ q,
                                               float* __restrict__ sa, int32_t* __restrict__ qcorr,
                                               float inv_sqrt_k) {
  constexpr int K = 1 << LOGK;
  constexpr int T = 1 << LOGT;
  constexpr int r = LOGK - LOGT;
  constexpr int R = 1 << r;
  constexpr int PASSES = (LOGK + r - 1) / r;
  constexpr int LAST_W = LOGK - (PASSES - 1) * r;
  static_assert(r >= 3 && r - LAST_W >= 3, "the last pass must leave runs of >= 8 elements");
  auto addr = [](int e) { return e + 4 * (e >> r); };
  auto elem = [](int p, int tt, int j) {
    const int lo = p * r;
    const int w = (LOGK - lo) < r ? (LOGK - lo) : r;
    const int rest = (tt << (r - w)) | (j >> w);
    return (rest & ((1 << lo) - 1)) | ((j & ((1 << w) - 1)) << lo) | ((rest >> lo) << (lo + w));
  };
  auto sync = [&]() {
    if constexpr (T > 64) __syncthreads();
    else __builtin_amdgcn_wave_barrier();
  };

#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    if (p > 0) {
      // Transpose: scatter with the previous pass's mapping, gather with this one's.
      if (p == 1) {
#pragma unroll
        for (int c = 0; c < R / 4; ++c)
          *reinterpret_cast<float4*>(&L[addr(t * R + 4 * c)]) =
              make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
      } else {
#pragma unroll
        for (int j = 0; j < R; ++j) L[addr(elem(p - 1, t, j))] = v[j];
      }
      sync();
#pragma unroll
      for (int j = 0; j < R; ++j) v[j] = L[addr(elem(p, t, j))];
      sync();
    }
    const int w = (LOGK - p * r) < r ? (LOGK - p * r) : r;
#pragma unroll
    for (int b = 0; b < r; ++b) {
      if (b >= w) break;
#pragma unroll
      for (int j = 0; j < R; ++j) {
        if (j & (1 << b)) continue;
        const float a = v[j], c = v[j + (1 << b)];
        v[j] = __fadd_rn(a, c);
        v[j + (1 << b)] = __fsub_rn(a, c);
      }
    }
  }

  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < R; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = wave_max(amax);
  if constexpr (T > 64) {
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < T / 64; ++i) amax = fmaxf(amax, red[i]);
  }
  const float sdiv = __fadd_rn(__fdiv_rn(amax, 7.0f), 1e-12f);
  if (t == 0) sa[row] = __fmul_rn(sdiv, inv_sqrt_k);

  // Last pass: for each value g of the pass bits the registers j = g + 2^w * i,
  // i = 0 .. 2^(r-w) - 1, hold consecutive elements; pack them 8 at a time and store two
  // words (16 codes, 8 bytes: consecutive words of the row's slot in its fragment) at once.
  constexpr int RUN = R >> LAST_W;
  constexpr int NW = (1 << LAST_W) * (RUN / 8);  // code words per thread
  static_assert(RUN % 16 == 0, "runs of 16 codes per 8-byte store");
  auto gather8 = [&](int g, int u, float (&c8)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) c8[e] = v[g + (1 << LAST_W) * (8 * u + e)];
  };
  uint32_t words[NW];
  bool near_tie = false;
  const float rcp = __builtin_amdgcn_rcpf(sdiv);
#pragma unroll
  for (int g = 0; g < (1 << LAST_W); ++g)
#pragma unroll
    for (int u = 0; u < RUN / 8; ++u) {
      float c8[8];
      gather8(g, u, c8);
      words[g * (RUN / 8) + u] = static_cast<uint32_t>(quant_pack8_rcp(c8, rcp, near_tie));
    }
  if (__builtin_amdgcn_ballot_w64(near_tie) != 0) {  // rare: redo with exact division
#pragma unroll
    for (int g = 0; g < (1 << LAST_W); ++g)
#pragma unroll
      for (int u = 0; u < RUN / 8; ++u) {
        float c8[8];
        gather8(g, u, c8);
        words[g * (RUN / 8) + u] = static_cast<uint32_t>(quant_pack8(c8, sdiv));
      }
  }
#pragma unroll
  for (int g = 0; g < (1 << LAST_W); ++g)
#pragma unroll
    for (int u = 0; u < RUN / 8; u += 2) {
      const int e0 = elem(PASSES - 1, t, g + (1 << LAST_W) * 8 * u);
      const uint2 wd = make_uint2(words[g * (RUN / 8) + u] ^ kObFlipLo, words[g * (RUN / 8) + u + 1] ^ kObFlipLo);
      *reinterpret_cast<uint2*>(&q[frag_word_index(row, e0 >> 3, kblocks128(K))]) = wd;
    }
  int s16 = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) s16 += odd_code_sum16(words[i]);
  s16 = row_sum<T>(s16, ired);  // T == 64: one wave per row, no barrier
  if (t == 0) qcorr[row] = -8 * s16;
}

}  // namespace
}  // namespace w4a4
