// Fused Walsh-Hadamard rotation + per-token symmetric INT4 quantization + nibble pack
// for gfx950 (wave64).
//
// Semantics follow the reference's CPU statement (pi05_fast/w4a4/pack.py:113-131) and
// its GPU kernels (pi05_fast/w4a4/csrc/int4_gemm.cu:396-477), with two deliberate
// differences from the GPU kernels: the butterflies are staged in fp32 (the reference
// GPU kernel rounds every stage to fp16) and the rotated scale uses the host-rounded
// fp32(1/sqrt(K)) (the reference GPU kernel uses rsqrtf).  Both follow the CPU
// statement, which is what the oracle checks bit for bit.
//
// Work decomposition: one workgroup of T threads per row.  Thread t owns J = K/(8T)
// chunks of 8 consecutive elements; element i = e + 8*(t + T*j), e in [0,8), j in [0,J).
// Every chunk is one 16-byte fp16 load (the row is read fully coalesced) and one packed
// int32 store into the fragment-major code layout that the GEMM reads (frag_word_index in
// w4a4_internal.h), with the low nibbles in offset binary (the activation encoding of that
// header).  Each row also gets its correction qcorr = -128 * (sum of its odd-k codes),
// stored after the code fragments.  The radix-2 stages of the
// unnormalised Sylvester transform run in increasing order of the stride h:
//   h = 1, 2, 4            inside a chunk (registers),
//   h = 8 .. 256           across lanes of the wave (lane xor 1..32),
//   h = 512 .. 4T/... wave across waves of the workgroup (through LDS),
//   h >= 8T                across the chunks of a thread (registers).
// Each stage writes (a + b, a - b) for the pair (i, i + h) exactly as the fp32 CPU
// transform does, so the rotated values are bit-identical to it.

#include "cache_warm.h"
#include "quant_row.h"

namespace w4a4 {
namespace {

template <int T>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < T / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}

template <int K, int T>
__global__ __launch_bounds__(T) void quant_rot_kernel(const _Float16* __restrict__ x, int64_t m,
                                                      int32_t* __restrict__ q,
                                                      float* __restrict__ sa,
                                                      int32_t* __restrict__ qcorr,
                                                      float inv_sqrt_k) {
  constexpr int J = K / (8 * T);
  static_assert(J >= 1 && K == 8 * T * J, "K must be 8*T*J");
  static_assert(T >= 64 && (T & (T - 1)) == 0, "T must be a power of two >= 64");
  // Cross-wave exchange in groups of JG chunks keeps the buffer at <= 32 KB.
  constexpr int JG = J < 4 ? J : 4;
  __shared__ __align__(16) float xch[(T > 64) ? 8 * T * JG : 1];
  __shared__ float red[T / 64];
  __shared__ int ired[T / 64];

  const int64_t row = blockIdx.x;
  if (row >= m) return;
  const int t = threadIdx.x;
  const _Float16* xr = x + row * K;

  float v[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const half8 h = *reinterpret_cast<const half8*>(xr + 8 * (t + T * j));
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = static_cast<float>(h[e]);
  }

  // h = 1, 2, 4: inside each chunk.
#pragma unroll
  for (int j = 0; j < J; ++j) {
#pragma unroll
    for (int len = 1; len < 8; len <<= 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (e & len) continue;
        const float a = v[j][e], b = v[j][e + len];
        v[j][e] = __fadd_rn(a, b);
        v[j][e + len] = __fsub_rn(a, b);
      }
    }
  }

  // h = 8 .. 256: lane xor 1 .. 32.  The lower partner keeps a + b, the upper a - b.
#pragma unroll
  for (int mask = 1; mask < 64; mask <<= 1) {
    const bool upper = (t & mask) != 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float mine = v[j][e];
        const float other = __shfl_xor(mine, mask, 64);
        v[j][e] = upper ? __fsub_rn(other, mine) : __fadd_rn(mine, other);
      }
    }
  }

  // h = 512 .. 4T: across waves, through LDS.
#pragma unroll
  for (int wb = 64; wb < T; wb <<= 1) {
    const bool upper = (t & wb) != 0;
#pragma unroll
    for (int j0 = 0; j0 < J; j0 += JG) {
#pragma unroll
      for (int jj = 0; jj < JG; ++jj) {
        float4* dst = reinterpret_cast<float4*>(&xch[8 * (t + T * jj)]);
        dst[0] = make_float4(v[j0 + jj][0], v[j0 + jj][1], v[j0 + jj][2], v[j0 + jj][3]);
        dst[1] = make_float4(v[j0 + jj][4], v[j0 + jj][5], v[j0 + jj][6], v[j0 + jj][7]);
      }
      __syncthreads();
#pragma unroll
      for (int jj = 0; jj < JG; ++jj) {
        const float4* src = reinterpret_cast<const float4*>(&xch[8 * ((t ^ wb) + T * jj)]);
        const float4 p0 = src[0], p1 = src[1];
        const float o[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[j0 + jj][e] = upper ? __fsub_rn(o[e], v[j0 + jj][e]) : __fadd_rn(v[j0 + jj][e], o[e]);
      }
      __syncthreads();
    }
  }

  // h = 8T .. K/2: across the chunks of this thread.
#pragma unroll
  for (int jb = 1; jb < J; jb <<= 1) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (j & jb) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = v[j][e], b = v[j + jb][e];
        v[j][e] = __fadd_rn(a, b);
        v[j + jb][e] = __fsub_rn(a, b);
      }
    }
  }

  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[j][e]));
  amax = block_max<T>(amax, red);

  const float sdiv = __fadd_rn(__fdiv_rn(amax, 7.0f), 1e-12f);
  if (t == 0) sa[row] = __fmul_rn(sdiv, inv_sqrt_k);
  int s16 = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t w = quant_pack8(v[j], sdiv);
    s16 += odd_code_sum16(w);
    q[frag_word_index(row, t + T * j, kblocks128(K))] = static_cast<int32_t>(w);
  }
  s16 = row_sum<T>(s16, ired);
  if (t == 0) qcorr[row] = -8 * s16;
}

// Register-FFT form of the same transform for K = 2^LOGK, T = 2^LOGT threads per row
// (fwht_quant_row in quant_row.h): each thread loads R = K/T consecutive values (one
// coalesced 2R-byte load) and the passes run in registers with LDS transposes between
// them.  ROWS rows per workgroup; with T = 64 every row belongs to one wave and the
// passes need no workgroup barrier.
// NORM: the row is first replaced by its RMSNorm (transformers' GemmaRMSNorm,
// modeling_gemma.py:64-78, with weight nw and the (1 + w) offset when unit_offset):
//   h = fp16((x * r) * g),  r = 1 / sqrt(ss / K + eps) (correctly rounded sqrt and
//   division),  g = unit_offset + w,
// with ss summed per lane over its R consecutive elements in order, then over the 64
// lanes by the xor butterfly 32, 16, .., 1 (the oracle restates this order exactly), and
// the fp16 h is what gets rotated and quantized, as if the norm's output had been stored.
// E3M2 (K = 2048): the codes are written as E3M2 fragments (q points at the q6 buffer).
template <int LOGK, int LOGT, int ROWS, bool NORM = false, bool E3M2 = false>
__global__ __launch_bounds__(ROWS << LOGT) void fwht_quant_kernel(
    const _Float16* __restrict__ x, int64_t m, int32_t* __restrict__ q, float* __restrict__ sa,
    int32_t* __restrict__ qcorr, float inv_sqrt_k, const _Float16* __restrict__ nw = nullptr,
    float eps = 0.0f, int unit_offset = 0, const CacheWarmParams warm = CacheWarmParams{}) {
  constexpr int K = 1 << LOGK;
  constexpr int T = 1 << LOGT;
  constexpr int R = 1 << (LOGK - LOGT);
  static_assert(T == 64 || ROWS == 1, "rows of more than one wave need a workgroup per row");
  // Workgroups past the rows (launched only with warm buffers) warm the cache and leave.
  {
    const int64_t row_blocks = (m + ROWS - 1) / ROWS;
    if (static_cast<int64_t>(blockIdx.x) >= row_blocks) {
      cache_warm_part<(ROWS << LOGT)>(warm, blockIdx.x - row_blocks, gridDim.x - row_blocks, threadIdx.x);
      return;
    }
  }
  constexpr int LROW = K + 4 * (K / R);  // LDS floats per row (4 pad floats per R)
  // One wave per row (T == 64) runs in registers only (fwht_quant_row_wave).
  __shared__ __align__(16) float lds[T == 64 ? 1 : ROWS * LROW];
  __shared__ float red[ROWS * (T / 64 > 0 ? T / 64 : 1)];
  __shared__ int ired[T / 64];

  const int sub = threadIdx.x >> LOGT;
  const int t = threadIdx.x & (T - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS + sub;
  if constexpr (T > 64) {
    if (row >= m) return;  // ROWS == 1: the whole workgroup leaves together
  } else {
    if (row >= m) return;  // the wave owns its row: no workgroup barrier below
  }
  float* L = lds + sub * LROW;

  float v[R];
  const _Float16* xr = x + row * K + t * R;
#pragma unroll
  for (int c = 0; c < R / 8; ++c) {
    const half8 h = *reinterpret_cast<const half8*>(xr + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[8 * c + e] = static_cast<float>(h[e]);
  }
  if constexpr (NORM) {
    static_assert(T == 64, "the fused RMSNorm reduces over one wave");
    // The norm weights are loaded with the row, before the sum of squares needs it.
    half8 wv[R / 8];
#pragma unroll
    for (int c = 0; c < R / 8; ++c) wv[c] = *reinterpret_cast<const half8*>(nw + t * R + 8 * c);
    __builtin_amdgcn_sched_barrier(0);
    rms_norm_row_wave<K>(v, wv, eps, unit_offset);
  }

  if constexpr (T == 64) {
    (void)L;
    fwht_quant_row_wave<LOGK, E3M2>(v, t, row, q, sa, qcorr, inv_sqrt_k);
  } else {
    static_assert(!E3M2, "E3M2 codes come from the one-wave rows");
    fwht_quant_row<LOGK, LOGT>(v, L, red, ired, t, row, q, sa, qcorr, inv_sqrt_k);
  }
}

// Unrotated quantization for every other K (K % 64 == 0): int4_gemm.cu:451-477.
// One workgroup of 256 threads per row, two passes over the row (amax, then codes).
__global__ __launch_bounds__(256) void quant_rows_kernel(const _Float16* __restrict__ x, int64_t m,
                                                         int32_t k, int32_t* __restrict__ q,
                                                         float* __restrict__ sa,
                                                         int32_t* __restrict__ qcorr) {
  __shared__ float red[4];
  __shared__ int ired[4];
  const int64_t row = blockIdx.x;
  if (row >= m) return;
  const int t = threadIdx.x;
  const int chunks = k / 8;
  const _Float16* xr = x + row * k;
  float amax = 0.0f;
  for (int c = t; c < chunks; c += 256) {
    const half8 h = *reinterpret_cast<const half8*>(xr + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(static_cast<float>(h[e])));
  }
  amax = block_max<256>(amax, red);
  const float sdiv = __fadd_rn(__fdiv_rn(amax, 7.0f), 1e-12f);
  if (t == 0) sa[row] = sdiv;
  int s16 = 0;
  for (int c = t; c < chunks; c += 256) {
    const half8 h = *reinterpret_cast<const half8*>(xr + 8 * c);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(h[e]);
    const uint32_t w = quant_pack8(v, sdiv);
    s16 += odd_code_sum16(w);
    q[frag_word_index(row, c, kblocks128(k))] = static_cast<int32_t>(w);
  }
  s16 = row_sum<256>(s16, ired);
  if (t == 0) qcorr[row] = -8 * s16;
}


// K = 2048 with two waves per row, for row counts that leave most SIMDs idle: waves 2i
// and 2i + 1 of a workgroup take row 2 blockIdx.x + i, 16 elements per lane
// (fwht_quant_row_2wave: thread t of the pair holds elements 16 t .. 16 t + 15).  With
// NORM both waves also load the row in the one-wave layout (lane l: elements 32 l ..
// 32 l + 31) and take its sum of squares in the one-wave order, so that the norm, and
// with it every code, equals fwht_quant_kernel<11, 6, 4, true>'s bit for bit.  A pair
// past M (odd M) computes a copy of row M - 1 and stores nothing.  Workgroups past the
// rows (launched only with warm buffers) warm the cache, as in fwht_quant_kernel.
// Measured with the RMSNorm (µs, two-wave rows / one-wave rows): M = 1: 3.46 / 3.73, 64:
// 3.8 / 4.2-4.3, 256: 3.9-4.0 / 4.4, 512: 4.2 / 4.45-4.5, but 640: 5.3-5.4 / 4.6 (more
// waves than SIMDs), so the two-wave rows run up to kTwoWaveRowsMax rows.
constexpr int64_t kTwoWaveRowsMax = 512;
template <bool NORM>
__global__ __launch_bounds__(256) void fwht_quant2_kernel(const _Float16* __restrict__ x, int64_t m,
                                                          int32_t* __restrict__ q, float* __restrict__ sa,
                                                          int32_t* __restrict__ qcorr, float inv_sqrt_k,
                                                          const _Float16* __restrict__ nw, float eps,
                                                          int unit_offset,
                                                          const CacheWarmParams warm = CacheWarmParams{}) {
  __shared__ __align__(16) float xch[2][2 * 64 * 16];
  __shared__ float redf[2][2];
  __shared__ int redi[2][2];
  const int tid = threadIdx.x;
  {
    const int64_t row_blocks = (m + 1) / 2;
    if (static_cast<int64_t>(blockIdx.x) >= row_blocks) {
      cache_warm_part<256>(warm, blockIdx.x - row_blocks, gridDim.x - row_blocks, tid);
      return;
    }
  }
  const int pr = tid >> 7;
  const int t = tid & 127;
  const int64_t row_raw = 2 * static_cast<int64_t>(blockIdx.x) + pr;
  const bool valid = row_raw < m;
  const int64_t row = valid ? row_raw : m - 1;
  const _Float16* xr = x + row * 2048;
  float v2[16];
  {
    const half8 a0 = *reinterpret_cast<const half8*>(xr + 16 * t);
    const half8 a1 = *reinterpret_cast<const half8*>(xr + 16 * t + 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v2[e] = static_cast<float>(a0[e]);
      v2[8 + e] = static_cast<float>(a1[e]);
    }
  }
  if constexpr (NORM) {
    const int lane = tid & 63;
    half8 xw[4], w2[2];
#pragma unroll
    for (int c = 0; c < 4; ++c) xw[c] = *reinterpret_cast<const half8*>(xr + 32 * lane + 8 * c);
#pragma unroll
    for (int c = 0; c < 2; ++c) w2[c] = *reinterpret_cast<const half8*>(nw + 16 * t + 8 * c);
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * c + e] = static_cast<float>(xw[c][e]);
    rms_norm_apply<16>(v2, w2, rms_norm_rr_wave<2048>(v, eps), unit_offset);
  }
  fwht_quant_row_2wave<11>(v2, t, xch[pr], redf[pr], redi[pr], valid, row, q, sa, qcorr, inv_sqrt_k);
}

}  // namespace

hipError_t launch_quantize(const void* x, int64_t m, int32_t k, int32_t* q, float* sa,
                           float inv_sqrt_k, hipStream_t stream, const CacheWarmParams* warm) {
  if (m <= 0) return hipSuccess;
  const _Float16* xh = static_cast<const _Float16*>(x);
  int32_t* qcorr = q + q_payload_words((m + 15) / 16, kblocks128(k));
  const dim3 grid(static_cast<unsigned>(m));
  switch (k) {
    case 16384: {
      // Cache warming fills the slots that the last round of rows leaves idle (68 KB of LDS
      // per row: two workgroups per CU).
      const int64_t kSlots = 2 * static_cast<int64_t>(device_cu_count());
      const int64_t tail = m % kSlots;
      const int64_t extra = (warm != nullptr && warm->nbuf > 0 && tail != 0) ? kSlots - tail : 0;
      fwht_quant_kernel<14, 8, 1><<<dim3(static_cast<unsigned>(m + extra)), 256, 0, stream>>>(
          xh, m, q, sa, qcorr, inv_sqrt_k, nullptr, 0.0f, 0, extra > 0 ? *warm : CacheWarmParams{});
      break;
    }
    case 2048:
      if (m <= kTwoWaveRowsMax) {
        fwht_quant2_kernel<false><<<dim3(static_cast<unsigned>((m + 1) / 2)), 256, 0, stream>>>(
            xh, m, q, sa, qcorr, inv_sqrt_k, nullptr, 0.0f, 0);
        break;
      }
      fwht_quant_kernel<11, 6, 4><<<dim3(static_cast<unsigned>((m + 3) / 4)), 256, 0, stream>>>(
          xh, m, q, sa, qcorr, inv_sqrt_k);
      break;
    case 1024:
      quant_rot_kernel<1024, 128><<<grid, 128, 0, stream>>>(xh, m, q, sa, qcorr, inv_sqrt_k);
      break;
    default:
      quant_rows_kernel<<<grid, 256, 0, stream>>>(xh, m, k, q, sa, qcorr);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm_quantize(const void* x, const void* w, float eps, int unit_offset,
                                  int64_t m, int32_t k, int32_t* q, float* sa, float inv_sqrt_k,
                                  hipStream_t stream, const CacheWarmParams* warm) {
  if (m <= 0) return hipSuccess;
  if (k != 2048) return hipErrorInvalidValue;
  int32_t* qcorr = q + q_payload_words((m + 15) / 16, kblocks128(k));
  // Cache warming: one workgroup for each CU that the row workgroups (4 rows each) leave
  // without one; none once the rows cover every CU.
  const int64_t row_blocks = (m + 3) / 4;
  const int64_t cus = device_cu_count();
  if (m <= kTwoWaveRowsMax) {  // two waves per row, two rows per workgroup; warming as below
    const int64_t pair_blocks = (m + 1) / 2;
    const int64_t extra2 = (warm != nullptr && warm->nbuf > 0 && pair_blocks < cus) ? cus - pair_blocks : 0;
    fwht_quant2_kernel<true><<<dim3(static_cast<unsigned>(pair_blocks + extra2)), 256, 0, stream>>>(
        static_cast<const _Float16*>(x), m, q, sa, qcorr, inv_sqrt_k, static_cast<const _Float16*>(w), eps,
        unit_offset, extra2 > 0 ? *warm : CacheWarmParams{});
    return hipGetLastError();
  }
  const int64_t extra = (warm != nullptr && warm->nbuf > 0 && row_blocks < cus) ? cus - row_blocks : 0;
  fwht_quant_kernel<11, 6, 4, true><<<dim3(static_cast<unsigned>(row_blocks + extra)), 256, 0, stream>>>(
      static_cast<const _Float16*>(x), m, q, sa, qcorr, inv_sqrt_k, static_cast<const _Float16*>(w),
      eps, unit_offset, extra > 0 ? *warm : CacheWarmParams{});
  return hipGetLastError();
}

hipError_t launch_quantize_e3m2(const void* x, const void* nw, float eps, int unit_offset, int64_t m,
                                int32_t k, void* q6, float* sa, float inv_sqrt_k, hipStream_t stream,
                                const CacheWarmParams* warm) {
  if (m <= 0) return hipSuccess;
  if (k != 2048) return hipErrorInvalidValue;
  // Cache warming as in launch_rmsnorm_quantize: one workgroup per CU the rows leave idle.
  const int64_t row_blocks = (m + 3) / 4;
  const int64_t cus = device_cu_count();
  const int64_t extra = (warm != nullptr && warm->nbuf > 0 && row_blocks < cus) ? cus - row_blocks : 0;
  const CacheWarmParams wp = extra > 0 ? *warm : CacheWarmParams{};
  const dim3 grid(static_cast<unsigned>(row_blocks + extra));
  const _Float16* xh = static_cast<const _Float16*>(x);
  int32_t* q = static_cast<int32_t*>(q6);
  if (nw != nullptr)
    fwht_quant_kernel<11, 6, 4, true, true><<<grid, 256, 0, stream>>>(
        xh, m, q, sa, nullptr, inv_sqrt_k, static_cast<const _Float16*>(nw), eps, unit_offset, wp);
  else
    fwht_quant_kernel<11, 6, 4, false, true><<<grid, 256, 0, stream>>>(xh, m, q, sa, nullptr, inv_sqrt_k, nullptr,
                                                                       0.0f, 0, wp);
  return hipGetLastError();
}

}  // namespace w4a4
