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
// w4a4_internal.h).  The radix-2 stages of the
// unnormalised Sylvester transform run in increasing order of the stride h:
//   h = 1, 2, 4            inside a chunk (registers),
//   h = 8 .. 256           across lanes of the wave (lane xor 1..32),
//   h = 512 .. 4T/... wave across waves of the workgroup (through LDS),
//   h >= 8T                across the chunks of a thread (registers).
// Each stage writes (a + b, a - b) for the pair (i, i + h) exactly as the fp32 CPU
// transform does, so the rotated values are bit-identical to it.

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Eight codes clamp(rint(v / sdiv), -7, 7) packed as nibbles 0..7 of one word.
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
                                                      float* __restrict__ sa, float inv_sqrt_k) {
  constexpr int J = K / (8 * T);
  static_assert(J >= 1 && K == 8 * T * J, "K must be 8*T*J");
  static_assert(T >= 64 && (T & (T - 1)) == 0, "T must be a power of two >= 64");
  // Cross-wave exchange in groups of JG chunks keeps the buffer at <= 32 KB.
  constexpr int JG = J < 4 ? J : 4;
  __shared__ __align__(16) float xch[(T > 64) ? 8 * T * JG : 1];
  __shared__ float red[T / 64];

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
#pragma unroll
  for (int j = 0; j < J; ++j) q[frag_word_index(row, t + T * j, kblocks128(K))] = quant_pack8(v[j], sdiv);
}

// Unrotated quantization for every other K (K % 64 == 0): int4_gemm.cu:451-477.
// One workgroup of 256 threads per row, two passes over the row (amax, then codes).
__global__ __launch_bounds__(256) void quant_rows_kernel(const _Float16* __restrict__ x, int64_t m,
                                                         int32_t k, int32_t* __restrict__ q,
                                                         float* __restrict__ sa) {
  __shared__ float red[4];
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
  for (int c = t; c < chunks; c += 256) {
    const half8 h = *reinterpret_cast<const half8*>(xr + 8 * c);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(h[e]);
    q[frag_word_index(row, c, kblocks128(k))] = quant_pack8(v, sdiv);
  }
}

}  // namespace

hipError_t launch_quantize(const void* x, int64_t m, int32_t k, int32_t* q, float* sa,
                           float inv_sqrt_k, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  const _Float16* xh = static_cast<const _Float16*>(x);
  const dim3 grid(static_cast<unsigned>(m));
  switch (k) {
    case 16384:
      quant_rot_kernel<16384, 256><<<grid, 256, 0, stream>>>(xh, m, q, sa, inv_sqrt_k);
      break;
    case 2048:
      quant_rot_kernel<2048, 256><<<grid, 256, 0, stream>>>(xh, m, q, sa, inv_sqrt_k);
      break;
    case 1024:
      quant_rot_kernel<1024, 128><<<grid, 128, 0, stream>>>(xh, m, q, sa, inv_sqrt_k);
      break;
    default:
      quant_rows_kernel<<<grid, 256, 0, stream>>>(xh, m, k, q, sa);
      break;
  }
  return hipGetLastError();
}

}  // namespace w4a4
