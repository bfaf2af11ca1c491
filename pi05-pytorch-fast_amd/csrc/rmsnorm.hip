// One-pass RMSNorm of fp16 rows for the decoder around the W4A4 projections: the input
// norms of every attention and MLP block feed the QKV and gate/up activation quant.
//
// Semantics of transformers' GemmaRMSNorm (modeling_gemma.py:64-78), evaluated in the
// same fp32 operation order:
//   r = rsqrt(mean(float(x)^2) + eps)
//   y = fp16((float(x) * r) * (1 + float(w)))        (unit_offset = 1, Gemma)
//   y = fp16((float(x) * r) * float(w))              (unit_offset = 0)
// The eager module runs this as seven elementwise/reduction kernels with fp32
// intermediates in HBM; here one wave owns a row, keeps it in registers and writes the
// fp16 result once.  The sum of squares is reduced in a different order than torch's
// reduction kernel, so r can differ from the eager value in its last bit; the outputs
// then differ by one fp16 ulp on a small fraction of elements.

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

// One wave per row, CH = K/8 16-byte chunks per row spread over the 64 lanes.
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
  const _Float16* xr = x + row * k;
  half8 v[CPL];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = j * 64 + lane;
    v[j] = (c < chunks) ? *reinterpret_cast<const half8*>(xr + 8 * c) : half8{};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = static_cast<float>(v[j][e]);
      ss += f * f;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float r = rsqrtf(ss * inv_k + eps);
  _Float16* yr = y + row * k;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = j * 64 + lane;
    if (c >= chunks) continue;
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
  const float inv_k = 1.0f / static_cast<float>(k);
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
