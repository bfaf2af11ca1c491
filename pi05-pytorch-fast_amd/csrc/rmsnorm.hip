// One-pass RMSNorm of fp16 rows for the decoder around the W4A4 projections: the input
// norms of every attention and MLP block feed the QKV and gate/up activation quant.
//
// Semantics of transformers' GemmaRMSNorm (modeling_gemma.py:64-78) in fp32:
//   r = 1 / sqrt(sum(float(x)^2) * fp32(1/K) + eps)       (correctly rounded sqrt, division)
//   y = fp16((float(x) * r) * (1 + float(w)))           (unit_offset = 1, Gemma)
//   y = fp16((float(x) * r) * float(w))                 (unit_offset = 0)
// One wave owns a row, keeps it in registers and writes the fp16 result once (the eager
// module runs seven kernels with fp32 intermediates in HBM).  The sum of squares has one
// fixed order, shared with the RMSNorm fused into the K = 2048 activation quant
// (quant_rot.hip): lane l sums its R = 8 * ceil(K / 512) consecutive elements
// l*R .. min((l+1)*R, K) - 1 in order, then the 64 lane sums are combined by the xor
// butterfly 32, 16, .., 1.  Both kernels therefore give the same fp16 rows, bit for bit,
// and the oracle restates that order (rms_norm_lanes).  torch's reduction sums in another
// order and its rsqrt is not correctly rounded, so an output can differ from the eager
// module's by one fp16 ulp on rare elements.

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// y = fp16(a * b) with the fp32 product rounded first (the empty asm keeps the backend
// from folding the multiply and the conversion into one v_fma_mix).
__device__ __forceinline__ _Float16 mul_to_f16(float a, float b) {
  float y = a * b;
  asm volatile("" : "+v"(y));
  return static_cast<_Float16>(y);
}

// One wave per row; lane l holds chunks (8 consecutive elements) l*cpl .. l*cpl + cpl - 1
// of the row's K/8 chunks, cpl = ceil(K/512) <= CPL.
template <int CPL>  // chunks per lane held in registers (K <= 512 * CPL)
__global__ __launch_bounds__(256) void rmsnorm_kernel(const _Float16* __restrict__ x,
                                                      const _Float16* __restrict__ w, float eps,
                                                      float inv_k, int unit_offset, int64_t m,
                                                      int32_t k, _Float16* __restrict__ y) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= m) return;  // the wave owns its row: no barrier below
  const int chunks = k / 8;
  const int cpl = (chunks + 63) / 64;
  const _Float16* xr = x + row * k;
  half8 v[CPL];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane * cpl + j;
    const bool valid = j < cpl && c < chunks;
    v[j] = valid ? *reinterpret_cast<const half8*>(xr + 8 * c) : half8{};
    if (valid) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = static_cast<float>(v[j][e]);
        ss = ss + f * f;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss = ss + __shfl_xor(ss, o, 64);
  const float r = 1.0f / __builtin_sqrtf(ss * inv_k + eps);
  _Float16* yr = y + row * k;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane * cpl + j;
    if (j >= cpl || c >= chunks) continue;
    const half8 wv = *reinterpret_cast<const half8*>(w + 8 * c);
    half8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = unit_offset ? (1.0f + static_cast<float>(wv[e])) : static_cast<float>(wv[e]);
      o[e] = mul_to_f16(static_cast<float>(v[j][e]) * r, g);
    }
    *reinterpret_cast<half8*>(yr + 8 * c) = o;
  }
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, const void* w, float eps, int unit_offset, int64_t m,
                          int32_t k, void* y, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((m + 3) / 4));
  const float inv_k = static_cast<float>(1.0 / static_cast<double>(k));  // as the fused kernel
  const auto* xh = static_cast<const _Float16*>(x);
  const auto* wh = static_cast<const _Float16*>(w);
  auto* yh = static_cast<_Float16*>(y);
  if (k <= 512 * 4)
    rmsnorm_kernel<4><<<grid, 256, 0, stream>>>(xh, wh, eps, inv_k, unit_offset, m, k, yh);
  else if (k <= 512 * 16)
    rmsnorm_kernel<16><<<grid, 256, 0, stream>>>(xh, wh, eps, inv_k, unit_offset, m, k, yh);
  else
    rmsnorm_kernel<32><<<grid, 256, 0, stream>>>(xh, wh, eps, inv_k, unit_offset, m, k, yh);
  return hipGetLastError();
}

}  // namespace w4a4
