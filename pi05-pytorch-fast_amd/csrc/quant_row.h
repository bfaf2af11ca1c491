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

constexpr int kDppXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRev4 = 0x1B;       // quad_perm [3,2,1,0]: lane i^3 within the quad
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i^7 within 8
constexpr int kDppRor8 = 0x128;      // row_ror:8: lane i^8 within the 16-lane row

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
// x of lane (this lane ^ (1 << K)), K = 0..3.
template <int K>
__device__ __forceinline__ float lane_xor_f(float x) {
  if constexpr (K == 0) return dpp_f<kDppXor1>(x);
  else if constexpr (K == 1) return dpp_f<kDppXor2>(x);
  else if constexpr (K == 2) return dpp_f<kDppHalfMirror>(dpp_f<kDppRev4>(x));
  else return dpp_f<kDppRor8>(x);
}
template <int K>
__device__ __forceinline__ int lane_xor_i(int x) {
  if constexpr (K == 0) return dpp_i<kDppXor1>(x);
  else if constexpr (K == 1) return dpp_i<kDppXor2>(x);
  else if constexpr (K == 2) return dpp_i<kDppHalfMirror>(dpp_i<kDppRev4>(x));
  else return dpp_i<kDppRor8>(x);
}
// Max / sum over the 64 lanes, the result in every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, lane_xor_f<0>(v));
  v = fmaxf(v, lane_xor_f<1>(v));
  v = fmaxf(v, lane_xor_f<2>(v));
  v = fmaxf(v, lane_xor_f<3>(v));
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ int wave_sum_dpp(int v) {
  v += lane_xor_i<0>(v);
  v += lane_xor_i<1>(v);
  v += lane_xor_i<2>(v);
  v += lane_xor_i<3>(v);
  auto r16 = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
  v = static_cast<int>(r16[0]) + static_cast<int>(r16[1]);
  auto r32 = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
  return static_cast<int>(r32[0]) + static_cast<int>(r32[1]);
}
// The same reductions under the names the quantizers use.  Max and integer sums do not
// depend on the order.  The fp32 sum keeps the xor butterfly 32, 16, 8, 4, 2, 1 (each
// step v + partner, and fp32 addition is commutative), so it equals the LDS-permute
// loop v += shfl_xor(v, o) for o = 32 .. 1 bit for bit, without its six LDS round trips.
__device__ __forceinline__ float wave_max(float v) { return wave_max_dpp(v); }
__device__ __forceinline__ int wave_sum(int v) { return wave_sum_dpp(v); }
__device__ __forceinline__ float wave_sum_f(float v) {
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __fadd_rn(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __fadd_rn(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  v = __fadd_rn(v, lane_xor_f<3>(v));
  v = __fadd_rn(v, lane_xor_f<2>(v));
  v = __fadd_rn(v, lane_xor_f<1>(v));
  return __fadd_rn(v, lane_xor_f<0>(v));
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

// Eight codes c = clamp(rint(v / sdiv), -7, 7) packed as nibbles 0..7 of one word in the
// stored form: low nibble of each byte c + 8 (offset binary), high nibble c & 0xF (two's
// complement).  Each code is computed as c + 8, in [1, 15], and placed with one
// shift-or; the final xor turns the high nibbles from offset binary to two's complement
// ((c + 8) ^ 8 == c & 0xF).  A NaN quotient gives -7 (the clamp keeps the non-NaN bound).
__device__ __forceinline__ uint32_t quant_pack8(const float (&v)[8], float sdiv) {
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = __builtin_rintf(__fdiv_rn(v[e], sdiv));
    r = fminf(fmaxf(r, -7.0f), 7.0f) + 8.0f;
    word |= static_cast<uint32_t>(r) << (4 * e);
  }
  return word ^ kObFlipHi;
}

// Same eight codes without a division per element.  qa = fl(v * rcp(sdiv) + 8) (one
// fused rounding) differs from the exact q + 8, q = v / sdiv, by less than 1.31e-6:
// |q| <= 7 and v_rcp_f32 is documented to 1 ulp, a relative error of at most 2^-23, so
// v * rcp is within 7 * 2^-23 (8.3e-7) of q; the fma adds 8 exactly and rounds once, at an
// ulp of at most 2^-20 for results below 16 (error <= 2^-21, 4.8e-7).
// rint(q + 8) == rint(q) + 8 (8 is even, so ties still go to even), so rint(qa) - 8 ==
// rint(q) unless q lies within 1.31e-6 of a half-integer.  Any lane that sees qa within
// 3e-6 of one (more than twice that bound) raises `near_tie` for this word; the caller then
// redoes that word's codes with quant_pack8 (exact division).  Both paths therefore
// produce the reference's round-half-even codes bit for bit.  One slow row sets a
// launch's end, so the redo is kept small: a 3e-6 window (1e-5 before) and only the
// flagged words redone (before: every word of the wave), which took the K=16384 quant at
// 776 rows from 18.4 to 16.9 us.
__device__ __forceinline__ uint32_t quant_pack8_rcp(const float (&v)[8], float rcp, bool& near_tie) {
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float qa = __builtin_fmaf(v[e], rcp, 8.0f);
    float r = __builtin_rintf(qa);
    near_tie |= fabsf(qa - r) > 0.499997f;
    r = fminf(fmaxf(r, 1.0f), 15.0f);
    word |= static_cast<uint32_t>(r) << (4 * e);
  }
  return word ^ kObFlipHi;
}

// The codes of quant_pack8 / quant_pack8_rcp as floats c + 8 in [1, 15] (same arithmetic,
// so the same codes), for the E3M2 operand form.
__device__ __forceinline__ void quant_codes8(const float (&v)[8], float sdiv, float* c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float r = __builtin_rintf(__fdiv_rn(v[e], sdiv));
    c[e] = fminf(fmaxf(r, -7.0f), 7.0f) + 8.0f;
  }
}
__device__ __forceinline__ void quant_codes8_rcp(const float (&v)[8], float rcp, bool& near_tie, float* c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float qa = __builtin_fmaf(v[e], rcp, 8.0f);
    const float r = __builtin_rintf(qa);
    near_tie |= fabsf(qa - r) > 0.499997f;
    c[e] = fminf(fmaxf(r, 1.0f), 15.0f);
  }
}

// One lane's 32 consecutive codes of row `row` (elements 32 t .. 32 t + 31, t the lane) as
// an E3M2 fragment slot (the q6 layout of w4a4_internal.h): c holds code + 8.
// v_cvt_scalef32_2xpk16_bf6_f32 converts two 16-value vectors, interleaving them (output
// value 2i from the first, 2i + 1 from the second), so the even and the odd codes go in
// separately; integers in [-7, 7] convert exactly.
__device__ __forceinline__ void store_e3m2_slot(const float (&c)[32], int t, int64_t row, int32_t kb128,
                                                uint8_t* __restrict__ q6) {
  typedef float v16f __attribute__((ext_vector_type(16)));
  v16f ev, od;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    ev[i] = c[2 * i] - 8.0f;
    od[i] = c[2 * i + 1] - 8.0f;
  }
  const auto d = __builtin_amdgcn_cvt_scalef32_2xpk16_bf6_f32(ev, od, 1.0f);
  uint8_t* const frag = q6 + ((row >> 4) * kb128 + (t >> 2)) * static_cast<int64_t>(kE3m2FragBytes);
  const int slot = static_cast<int>(row & 15) + 16 * (t & 3);
  *reinterpret_cast<uint4*>(frag + 16 * slot) = make_uint4(d[0], d[1], d[2], d[3]);
  *reinterpret_cast<uint2*>(frag + 1024 + 8 * slot) = make_uint2(d[4], d[5]);
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
        // elem(p, t, j) is the OR of disjoint thread bits elem(p, t, 0) and register bits
        // elem(p, 0, j), and the padded address is linear over such fields, so every
        // access is one per-thread base plus a compile-time offset (the LDS
        // instruction's immediate) instead of per-access index arithmetic.
        float* const wb = L + addr(elem(p - 1, t, 0));
#pragma unroll
        for (int j = 0; j < R; ++j) wb[addr(elem(p - 1, 0, j))] = v[j];
      }
      sync();
      const float* const rb = L + addr(elem(p, t, 0));
#pragma unroll
      for (int j = 0; j < R; ++j) v[j] = rb[addr(elem(p, 0, j))];
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
  bool tie[NW];
  bool near_tie = false;
  const float rcp = __builtin_amdgcn_rcpf(sdiv);
#pragma unroll
  for (int g = 0; g < (1 << LAST_W); ++g)
#pragma unroll
    for (int u = 0; u < RUN / 8; ++u) {
      float c8[8];
      gather8(g, u, c8);
      const int i = g * (RUN / 8) + u;
      tie[i] = false;
      words[i] = quant_pack8_rcp(c8, rcp, tie[i]);
      near_tie |= tie[i];
    }
  if (__builtin_amdgcn_ballot_w64(near_tie) != 0) {  // rare: redo the flagged words exactly
#pragma unroll
    for (int g = 0; g < (1 << LAST_W); ++g)
#pragma unroll
      for (int u = 0; u < RUN / 8; ++u) {
        const int i = g * (RUN / 8) + u;
        if (__builtin_amdgcn_ballot_w64(tie[i]) != 0) {
          float c8[8];
          gather8(g, u, c8);
          const uint32_t exact = quant_pack8(c8, sdiv);
          words[i] = tie[i] ? exact : words[i];
        }
      }
  }
#pragma unroll
  for (int g = 0; g < (1 << LAST_W); ++g)
#pragma unroll
    for (int u = 0; u < RUN / 8; u += 2) {
      const int e0 = elem(PASSES - 1, t, g + (1 << LAST_W) * 8 * u);
      const uint2 wd = make_uint2(words[g * (RUN / 8) + u], words[g * (RUN / 8) + u + 1]);
      *reinterpret_cast<uint2*>(&q[frag_word_index(row, e0 >> 3, kblocks128(K))]) = wd;
    }
  int s16 = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) s16 += odd_code_sum16(words[i]);
  s16 = row_sum<T>(s16, ired);  // T == 64: one wave per row, no barrier
  if (t == 0) qcorr[row] = -8 * s16;
}


// ---- One wave per row, registers only (T = 64).  Lane t holds R = K / 64 consecutive
// elements t*R .. t*R + R - 1 in v[0..R-1] (r = log2 R register bits, then 6 lane bits).
// The butterfly stages still run in increasing order of the stride, each writing
// (a + b, a - b) exactly, so the result is bit-identical to the CPU transform:
//   element bits 0 .. r-1     registers (pairs v[j], v[j ^ 2^b]);
//   element bits r .. r+3     lane bits 0-3: the partner's value comes through DPP
//                             (xor 1, 2: quad_perm; xor 4: quad_perm + row_half_mirror;
//                             xor 8: row_ror:8) straight into the add, and the upper lane
//                             adds its own value negated: partner + (-own) = a - b;
//   element bits r+4, r+5     lane bits 4 and 5: v_permlane16_swap / v_permlane32_swap on
//                             the register pairs of bit 0 / bit 1 (already transformed)
//                             exchange that register bit with the lane bit, the stage runs
//                             in registers, and the swaps are undone afterwards.
// No LDS and no barrier; the wave max and sum use the same DPP / swap exchanges.
// Register pairs (v[j], v[j | 2^B]) exchange register bit B with lane bit 4 (SW = 16) or
// lane bit 5 (SW = 32); applying it twice restores the layout.
template <int SW, int B, int R>
__device__ __forceinline__ void swap_lane_bit(float (&v)[R]) {
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if (j & (1 << B)) continue;
    auto r = (SW == 16) ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j | (1 << B)]), false, false)
                        : __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j | (1 << B)]), false, false);
    v[j] = __uint_as_float(r[0]);
    v[j | (1 << B)] = __uint_as_float(r[1]);
  }
}
template <int B, int R>
__device__ __forceinline__ void reg_stage(float (&v)[R]) {
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if (j & (1 << B)) continue;
    const float a = v[j], c = v[j + (1 << B)];
    v[j] = __fadd_rn(a, c);
    v[j + (1 << B)] = __fsub_rn(a, c);
  }
}
template <int K, int R>
__device__ __forceinline__ void lane_stage(float (&v)[R], int lane) {
  const uint32_t neg = static_cast<uint32_t>((lane >> K) & 1) << 31;  // upper lane: a - b
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const float partner = lane_xor_f<K>(v[j]);
    v[j] = __fadd_rn(partner, __uint_as_float(__float_as_uint(v[j]) ^ neg));
  }
}

// RMSNorm of one row held by one wave (transformers' GemmaRMSNorm, modeling_gemma.py:64-78,
// weight wv with the (1 + w) offset when unit_offset), in place:
//   h = fp16((x * r) * g),  r = 1 / sqrt(ss / K + eps) (correctly rounded sqrt and
//   division),  g = unit_offset + w,
// with ss summed per lane over its R consecutive elements in order, then over the 64 lanes
// by the xor butterfly 32, 16, .., 1; v then holds the fp16 h as fp32 values.
// r of the row (the sum of squares in the order above).
template <int K, int R>
__device__ __forceinline__ float rms_norm_rr_wave(const float (&v)[R], float eps) {
#pragma clang fp contract(off)
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < R; ++j) ss = ss + v[j] * v[j];
  ss = wave_sum_f(ss);
  return 1.0f / __builtin_sqrtf(ss * (1.0f / K) + eps);
}
// h = fp16((x * r) * g) of the N values in v, elementwise (any layout of the row).
template <int N>
__device__ __forceinline__ void rms_norm_apply(float (&v)[N], const half8 (&wv)[N / 8], float rr, int unit_offset) {
#pragma clang fp contract(off)
#pragma unroll
  for (int c = 0; c < N / 8; ++c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = unit_offset ? 1.0f + static_cast<float>(wv[c][e]) : static_cast<float>(wv[c][e]);
      float y = (v[8 * c + e] * rr) * g;
      asm volatile("" : "+v"(y));  // keep the fp32 product (no v_fma_mix into fp16)
      v[8 * c + e] = static_cast<float>(static_cast<_Float16>(y));
    }
  }
}
template <int K, int R>
__device__ __forceinline__ void rms_norm_row_wave(float (&v)[R], const half8 (&wv)[R / 8], float eps,
                                                  int unit_offset) {
  rms_norm_apply<R>(v, wv, rms_norm_rr_wave<K>(v, eps), unit_offset);
}

// E3M2: the codes go out as E3M2 fragment slots (q then points at the q6 buffer; no row
// corrections), else as INT4 words and qcorr.
template <int LOGK, bool E3M2 = false>
__device__ __forceinline__ void fwht_quant_row_wave(float (&v)[1 << (LOGK - 6)], int t, int64_t row,
                                                    int32_t* __restrict__ q, float* __restrict__ sa,
                                                    int32_t* __restrict__ qcorr, float inv_sqrt_k) {
  constexpr int K = 1 << LOGK;
  constexpr int r = LOGK - 6;
  constexpr int R = 1 << r;
  static_assert(r >= 4, "runs of >= 16 consecutive elements per lane");
#pragma unroll
  for (int b = 0; b < r; ++b) {
    if (b == 0) reg_stage<0>(v);
    else if (b == 1) reg_stage<1>(v);
    else if (b == 2) reg_stage<2>(v);
    else if (b == 3) reg_stage<3>(v);
    else if (b == 4) reg_stage<4>(v);
    else if (b == 5) reg_stage<5>(v);
    else if (b == 6) reg_stage<6>(v);
    else if (b == 7) reg_stage<7>(v);
  }
  lane_stage<0>(v, t);
  lane_stage<1>(v, t);
  lane_stage<2>(v, t);
  lane_stage<3>(v, t);
  swap_lane_bit<16, 0>(v);
  reg_stage<0>(v);  // element bit r + 4
  swap_lane_bit<32, 1>(v);
  reg_stage<1>(v);  // element bit r + 5
  swap_lane_bit<32, 1>(v);
  swap_lane_bit<16, 0>(v);

  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < R; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = wave_max_dpp(amax);
  const float sdiv = __fadd_rn(__fdiv_rn(amax, 7.0f), 1e-12f);
  if (t == 0) sa[row] = __fmul_rn(sdiv, inv_sqrt_k);
  if constexpr (E3M2) {
    static_assert(R == 32, "one E3M2 fragment slot (32 codes) per lane");
    float c[R];
    bool tie[R / 8];
    bool near_tie = false;
    const float rcp = __builtin_amdgcn_rcpf(sdiv);
#pragma unroll
    for (int u = 0; u < R / 8; ++u) {
      float c8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) c8[e] = v[8 * u + e];
      tie[u] = false;
      quant_codes8_rcp(c8, rcp, tie[u], c + 8 * u);
      near_tie |= tie[u];
    }
    if (__builtin_amdgcn_ballot_w64(near_tie) != 0) {  // rare: redo the flagged groups exactly
#pragma unroll
      for (int u = 0; u < R / 8; ++u) {
        if (__builtin_amdgcn_ballot_w64(tie[u]) != 0) {
          float c8[8], x8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) c8[e] = v[8 * u + e];
          quant_codes8(c8, sdiv, x8);
#pragma unroll
          for (int e = 0; e < 8; ++e) c[8 * u + e] = tie[u] ? x8[e] : c[8 * u + e];
        }
      }
    }
    store_e3m2_slot(c, t, row, kblocks128(K), reinterpret_cast<uint8_t*>(q));
    return;
  }
  // Codes of the lane's R consecutive elements: R / 8 words, word u = codes 8u .. 8u + 7.
  uint32_t words[R / 8];
  bool tie[R / 8];
  bool near_tie = false;
  const float rcp = __builtin_amdgcn_rcpf(sdiv);
#pragma unroll
  for (int u = 0; u < R / 8; ++u) {
    float c8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) c8[e] = v[8 * u + e];
    tie[u] = false;
    words[u] = quant_pack8_rcp(c8, rcp, tie[u]);
    near_tie |= tie[u];
  }
  if (__builtin_amdgcn_ballot_w64(near_tie) != 0) {  // rare: redo the flagged words exactly
#pragma unroll
    for (int u = 0; u < R / 8; ++u) {
      if (__builtin_amdgcn_ballot_w64(tie[u]) != 0) {
        float c8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) c8[e] = v[8 * u + e];
        const uint32_t exact = quant_pack8(c8, sdiv);
        words[u] = tie[u] ? exact : words[u];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < R / 8; u += 2) {
    const uint2 wd = make_uint2(words[u], words[u + 1]);
    *reinterpret_cast<uint2*>(&q[frag_word_index(row, (t * R) / 8 + u, kblocks128(K))]) = wd;
  }
  int s16 = 0;
#pragma unroll
  for (int u = 0; u < R / 8; ++u) s16 += odd_code_sum16(words[u]);
  s16 = wave_sum_dpp(s16);
  if (t == 0) qcorr[row] = -8 * s16;
}

// ---- Two waves per row (T = 128): thread t = 64 h + lane (h = the wave of the pair) holds
// R = K / 128 consecutive elements t*R .. t*R + R - 1.  Element bits 0 .. r+5 are the
// one-wave form's (registers, then lane bits 0-5); the last stage, over the wave bit h,
// exchanges the halves through LDS: lane L of the lower wave keeps a + b, of the upper
// wave a - b, with a the lower wave's value.  The row max and the odd-code sum combine the
// two waves' through LDS too.  xch: 2 * 64 * R floats of LDS for this row; redf / redi: 2
// words each.  Every wave of the workgroup calls it together (three workgroup barriers);
// with `store` false the pair computes but writes nothing (a row past the matrix).
template <int LOGK>
__device__ __forceinline__ void fwht_quant_row_2wave(float (&v)[1 << (LOGK - 7)], int t, float* xch, float* redf,
                                                     int* redi, bool store, int64_t row, int32_t* __restrict__ q,
                                                     float* __restrict__ sa, int32_t* __restrict__ qcorr,
                                                     float inv_sqrt_k) {
  constexpr int K = 1 << LOGK;
  constexpr int r = LOGK - 7;
  constexpr int R = 1 << r;
  static_assert(r >= 4 && R % 4 == 0, "runs of >= 16 consecutive elements per lane");
  const int lane = t & 63;
  const int h = t >> 6;
#pragma unroll
  for (int b = 0; b < r; ++b) {
    if (b == 0) reg_stage<0>(v);
    else if (b == 1) reg_stage<1>(v);
    else if (b == 2) reg_stage<2>(v);
    else if (b == 3) reg_stage<3>(v);
    else if (b == 4) reg_stage<4>(v);
    else if (b == 5) reg_stage<5>(v);
    else if (b == 6) reg_stage<6>(v);
  }
  lane_stage<0>(v, lane);
  lane_stage<1>(v, lane);
  lane_stage<2>(v, lane);
  lane_stage<3>(v, lane);
  swap_lane_bit<16, 0>(v);
  reg_stage<0>(v);  // element bit r + 4
  swap_lane_bit<32, 1>(v);
  reg_stage<1>(v);  // element bit r + 5
  swap_lane_bit<32, 1>(v);
  swap_lane_bit<16, 0>(v);
  // element bit r + 6: the other wave's value of the same register and lane
#pragma unroll
  for (int j = 0; j < R; j += 4)
    *reinterpret_cast<float4*>(xch + (h * 64 + lane) * R + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
  __syncthreads();
  const float* px = xch + ((h ^ 1) * 64 + lane) * R;
#pragma unroll
  for (int j = 0; j < R; j += 4) {
    const float4 o4 = *reinterpret_cast<const float4*>(px + j);
    const float o[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) v[j + e] = h == 0 ? __fadd_rn(v[j + e], o[e]) : __fsub_rn(o[e], v[j + e]);
  }

  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < R; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = wave_max_dpp(amax);
  if (lane == 0) redf[h] = amax;
  __syncthreads();
  amax = fmaxf(redf[0], redf[1]);
  const float sdiv = __fadd_rn(__fdiv_rn(amax, 7.0f), 1e-12f);
  if (store && t == 0) sa[row] = __fmul_rn(sdiv, inv_sqrt_k);
  uint32_t words[R / 8];
  bool tie[R / 8];
  bool near_tie = false;
  const float rcp = __builtin_amdgcn_rcpf(sdiv);
#pragma unroll
  for (int u = 0; u < R / 8; ++u) {
    float c8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) c8[e] = v[8 * u + e];
    tie[u] = false;
    words[u] = quant_pack8_rcp(c8, rcp, tie[u]);
    near_tie |= tie[u];
  }
  if (__builtin_amdgcn_ballot_w64(near_tie) != 0) {  // rare: redo the flagged words exactly
#pragma unroll
    for (int u = 0; u < R / 8; ++u) {
      if (__builtin_amdgcn_ballot_w64(tie[u]) != 0) {
        float c8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) c8[e] = v[8 * u + e];
        const uint32_t exact = quant_pack8(c8, sdiv);
        words[u] = tie[u] ? exact : words[u];
      }
    }
  }
  if (store) {
#pragma unroll
    for (int u = 0; u < R / 8; u += 2) {
      const uint2 wd = make_uint2(words[u], words[u + 1]);
      *reinterpret_cast<uint2*>(&q[frag_word_index(row, (t * R) / 8 + u, kblocks128(K))]) = wd;
    }
  }
  int s16 = 0;
#pragma unroll
  for (int u = 0; u < R / 8; ++u) s16 += odd_code_sum16(words[u]);
  s16 = wave_sum_dpp(s16);
  if (lane == 0) redi[h] = s16;
  __syncthreads();
  if (store && t == 0) qcorr[row] = -8 * (redi[0] + redi[1]);
}
}  // namespace
}  // namespace w4a4
