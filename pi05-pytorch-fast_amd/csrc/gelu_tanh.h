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

// fp16 bits of the fast evaluation: y = x (1 - r), r = 1 / (1 + 2^q), from the hardware
// exp2 and reciprocal, with q = 2u log2 e = x * (K0 + K1 x^2) (K0 = 2 log2(e) sqrt(2/pi),
// K1 = K0 * 0.044715): (0.5 x)(1 + tanh(u)) = x (1 - 1 / (1 + e^(2u))).  The products with
// x read the fp16 input directly (v_fma_mix), so x is never converted to fp32:
//   s = x * x + 0           exact (an fp16 square fits fp32 and is never -0),
//   q = x * (K0 + K1 s) + 0 the sign of a zero product is lost, and 2^(+-0) = 1 either way,
//   y = x * (1 - r) - 0     one fp32 rounding, as a plain fp32 multiply; the -0 addend
//                           keeps the sign of a zero product (gelu(-0) = -0),
// then y is rounded to fp16.  Every step is a single IEEE fp32 operation or one hardware
// instruction, so the result is the same in every kernel that inlines this.  It differs
// from the exact expression's fp16 result on a few hundred of the 65536 fp16 inputs, all
// with |x| in [2^-4, 5.3) (mostly negative x in [-5.2, -2], where 1 - r cancels to a few
// ulps), by at most a few ulps: gelu_tanh_fix.inc lists them.  (The form with y = x r and
// r = 1 / (1 + 2^-q), one instruction fewer, is closer to the exact values but gives 2^-24
// for the input 2^-24, whose exact result is a tie rounded to 0, outside the table.)
constexpr float kGeluK0 = 2.3022081983184814f;   // 2 log2(e) sqrt(2/pi)
constexpr float kGeluK1 = 0.10294324159622192f;  // K0 * 0.044715
__device__ __forceinline__ uint16_t gelu_tanh_fast_bits(_Float16 xh) {
#pragma clang fp contract(off)
  const float x = static_cast<float>(xh);
  const float s = __builtin_fmaf(x, x, 0.0f);
  const float q = __builtin_fmaf(x, __builtin_fmaf(s, kGeluK1, kGeluK0), 0.0f);
  const float c = 1.0f - __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(q));
  // fma(x, c, -0.0f) would be folded into a multiply that converts x to fp32 first.
  float y;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(y) : "v"(xh), "v"(c), "s"(-0.0f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(y));
}

// Corrections: the exact result's fp16 bit pattern minus the fast one's, for the inputs
// where they differ (gelu_tanh_fix.inc, generated on the GPU from these two functions by
// gelu_fix_gen.hip; the exhaustive test compares every fp16 input with torch).  They all
// lie in the window |x| bits in [kGeluFixAbsBase, kGeluFixAbsBase + kGeluFixHalf - 1).
// The int8 table is indexed by the fp16 bits minus the base, clamped: positive inputs of
// the window land in [0, kGeluFixHalf - 1), negative ones in [kGeluFixNeg,
// kGeluFixNeg + kGeluFixHalf - 1) (kGeluFixNeg = 0x8000, the sign bit), and every input
// outside the window reads a zero entry: positive ones above it land in the zero run
// [kGeluFixHalf - 1, kGeluFixNeg), negative ones below it too (their bits minus the base
// lie in [0x8000 - base, 0x8000)), and the others wrap or run past the negative half and
// are clamped to its last (zero) entry.  The index is two ALU instructions; the zero run
// between the halves is filled, not copied, where the table is staged in LDS.
constexpr uint32_t kGeluFixAbsBase = 0x2c00u;
constexpr uint32_t kGeluFixHalf = 6656u;
constexpr uint32_t kGeluFixNeg = 0x8000u;
constexpr uint32_t kGeluFixLast = kGeluFixNeg + kGeluFixHalf - 1;  // zero entry
constexpr int kGeluFixEntries = 39 * 1024;                          // > kGeluFixLast, 1 KB pieces
static_assert(kGeluFixLast < static_cast<uint32_t>(kGeluFixEntries), "the clamp stays in the table");

// Table slot of fp16 bit pattern xb (zero-extended).
__host__ __device__ constexpr uint32_t gelu_fix_index(uint32_t xb) {
  const uint32_t off = xb - kGeluFixAbsBase;
  return off < kGeluFixLast ? off : kGeluFixLast;
}
__host__ __device__ constexpr bool gelu_fix_in_window(uint32_t xb) {
  return ((xb & 0x7fffu) - kGeluFixAbsBase) < kGeluFixHalf - 1;
}
// The 1 KB pieces of the table that can hold nonzero entries: [0, kGeluFixPosPieces) and
// [kGeluFixNeg / 1024, kGeluFixEntries / 1024); the pieces between are all zero.
constexpr int kGeluFixPosPieces = (kGeluFixHalf + 1023) / 1024;
constexpr int kGeluFixNegPiece0 = kGeluFixNeg / 1024;
static_assert(kGeluFixNegPiece0 * 1024 + kGeluFixHalf <= static_cast<uint32_t>(kGeluFixEntries),
              "the negative half fits the table");

}  // namespace w4a4
