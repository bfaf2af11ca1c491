// GELU-tanh of fp16 values as torch.nn.functional.gelu(x, approximate="tanh") computes
// it on the GPU (fp32: x^3 = (x*x)*x, inner = kBeta * fma(kKappa, x^3, x),
// y = (0.5*x) * (1 + tanhf(inner)), rounded to fp16), shared by the gate/up GEMM epilogue,
// its split-K reduction, the elementwise entry point and the correction-table generator.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a4 {

// The exact expression.  Contraction is off so that only the one FMA is formed, and the
// empty asm keeps the fp32 result in a register: otherwise the backend folds the last
// multiply and the fp16 conversion into one v_fma_mix, which rounds once and differs from
// the fp32-then-fp16 rounding on about a fifth of all fp16 inputs.
__device__ __forceinline__ float gelu_tanh_exact(float x) {
#pragma clang fp contract(off)
  const float x3 = (x * x) * x;
  const float inner = 0.7978845608028654f * __builtin_fmaf(0.044715f, x3, x);
  float y = (0.5f * x) * (1.0f + tanhf(inner));
  asm volatile("" : "+v"(y));
  return y;
}

// fp16 bits of the fast evaluation: tanh(u) = 1 - 2 / (1 + 2^(2u log2 e)) from the
// hardware exp2 and reciprocal, a third of the instructions of tanhf.  Every operation is
// a single IEEE fp32 operation or one hardware instruction, so the result is the same in
// every kernel that inlines this.  It differs from the exact expression's fp16 result on
// 428 of the 65536 fp16 inputs: 426 with x in [-8, -1) (mostly x in [-5.2, -3], where
// 1 + tanh cancels to a few ulps) and 2 single-ulp roundings elsewhere.
__device__ __forceinline__ uint16_t gelu_tanh_fast_bits(float x) {
#pragma clang fp contract(off)
  const float x3 = (x * x) * x;
  const float inner = 0.7978845608028654f * __builtin_fmaf(0.044715f, x3, x);
  const float e = __builtin_amdgcn_exp2f(inner * 2.8853900817779268f);  // exp(2 inner)
  const float t = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f);
  float y = (0.5f * x) * (1.0f + t);
  asm volatile("" : "+v"(y));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(y));
}

// Corrections: the exact result's fp16 bit pattern minus the fast one's, for the inputs
// where they differ (gelu_tanh_fix.inc, generated on the GPU from these two functions by
// gelu_fix_gen.hip; the exhaustive test compares every fp16 input with torch).  Those in
// the window of negative x with |x| in [1, 8) (bit patterns 0xbc00 .. 0xc7ff: 426 of
// the 428) go to a 3 KB int8 table indexed by bits - kGeluFixBase; the others (2) are
// compared one by one.
constexpr uint32_t kGeluFixBase = 0xbc00u;
constexpr uint32_t kGeluFixSpan = 3u << 10;
constexpr int kGeluFixEntries = kGeluFixSpan;

// Index of fp16 bit pattern xb in the table (0 outside the window, where *in is false).
__device__ __forceinline__ uint32_t gelu_fix_index(uint32_t xb, bool& in) {
  const uint32_t off = xb - kGeluFixBase;
  in = off < kGeluFixSpan;
  return in ? off : 0u;
}

}  // namespace w4a4
