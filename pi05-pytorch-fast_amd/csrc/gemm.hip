// W4A4 GEMM for gfx950: int4 codes unpacked to int8, CDNA4 int8 MFMA
// (v_mfma_i32_16x16x64_i8), int32 accumulation, dequant epilogue.
//
// Reference semantics (pi05_fast/w4a4/csrc/int4_gemm.cu:63-204, 206-394; pack.py:134-145):
//   acc[m, n] = sum_k qa[m, k] * qw[n, k]            (int32, exact)
//   y[m, n]   = fp16((float(acc) * sa[m]) * sw[n])   (two fp32 products, RNE to fp16)
//
// INT4 -> INT8.  Packed words hold two codes per byte in the nibble encodings of
// w4a4_internal.h (activations: offset-binary low nibble, two's complement high nibble;
// weights: the reverse).  One AND per int8 word unpacks either operand into exact signed
// bytes (c + 8 or 16 c), and the MFMA pairs every activation byte with the weight byte of
// the same k, so its int32 sum is
//   S = 16 * acc + 128 * sum_{k odd} a + 128 * sum_{k even} b.
// The row and column terms are precomputed (qcorr after the activation codes, wcorr after
// the weight scales) and the accumulators start at qcorr[m] + wcorr[n], so they end at
// 16 * acc exactly; |S| <= 2048 K < 2^31 for any K the host accepts.  This costs 2 ALU ops per packed word
// instead of the 3 of a shift-and-mask unpack, which matters: the unpack is the largest
// non-MFMA cost of the loop.
//
// Tiling.  A wave owns a (16*MI) x (16*NI) tile = MI x NI accumulators of 16x16.  The
// NWAVES waves of a workgroup are arranged NW along N times KW along K: with KW > 1 the
// waves of one column block split the workgroup's k range into KW contiguous parts and
// sum their accumulators through LDS at the end (a reduce-scatter, after which each wave
// finishes its share of the row blocks), which gives narrow GEMMs (QKV, o, down) enough
// waves without a global split-K workspace.
// Both operands live in HBM in the same MFMA-fragment-major layout (frag_word_index: one
// 1 KB fragment per 16 rows/columns x 128 k; lane L loads slot L = 32 codes of row/
// column L%16, the operands of the block's two MFMAs), so every operand fetch is one
// fully coalesced 16-byte-per-lane load straight into registers.  (The vector memory
// pipeline issues about one wave-wide load per ~20 clocks per CU whatever its width, so
// 16-byte loads double the operand bandwidth of 8-byte ones.)  The K loop walks 128-deep
// k blocks through a RING-deep register ring (2 at two waves per SIMD): the loads of
// block kb + RING - 1 are issued before block kb is multiplied.  There is no LDS
// traffic and no barrier in the loop: the waves of a workgroup share their A fragments
// through the L1/L2 caches only.  (Measured alternatives that lost: A staged through a
// double-buffered LDS tile, whose per-stage barrier stalls the MFMA pipe more than the
// shared loads save; L2 warm-up touches of the weights a few blocks ahead, whose extra
// load instructions cost more than the misses they avoid; and deeper rings at one wave
// per SIMD, which lose the second wave's latency hiding.)
// Every global load in the loop is unconditional (out-of-range rows, columns and k
// blocks are clamped to valid addresses and their results are discarded), so the
// compiler's vmcnt bookkeeping stays exact and the prefetches overlap the MFMAs.
//
// Work order.  The grid is one-dimensional over the (m-tile, n-tile) pairs (y = K slice).
// Workgroups are dealt round-robin to the 8 XCDs, so block b runs on XCD b % 8; the tile
// index is remapped so that every XCD owns a contiguous run of tiles in n-major,
// m-minor order.  The m-tiles that share one weight column block therefore run side by
// side on one XCD and read those weights from its L2.
//
// Epilogue.  The weights are MFMA operand A, so each lane ends with four consecutive
// output columns of one row.  The tile's row and column scales were fetched under the
// main loop and staged in LDS; each 16-row block of a wave's fp16 output is staged in LDS
// (one 8-byte write per lane and fragment) and written back as whole rows with 16-byte
// non-temporal stores.  Modes: fp16 with scales, int32 split-K partials, int32
// accumulators, and paired gate/up tiles finished exactly as the eager
// `gelu(gate, approximate="tanh") * up` on the fp16 gate and up (apply.py:135-138).

#include <type_traits>

#include "cache_warm.h"
#include "gelu_tanh.h"
#include "quant_row.h"
#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v12i __attribute__((ext_vector_type(12)));
typedef float v4f __attribute__((ext_vector_type(4)));

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Activation operand bytes: (a[2j] + 8, 16 a[2j+1]) for the 8 codes of word x, then y.
__device__ __forceinline__ v4i unpack_a(uint32_t x, uint32_t y) {
  return v4i{static_cast<int>(x & kLoNib), static_cast<int>(x & kHiNib),
             static_cast<int>(y & kLoNib), static_cast<int>(y & kHiNib)};
}
// Weight operand bytes: (16 b[2j], b[2j+1] + 8), aligned with unpack_a's k order.
__device__ __forceinline__ v4i unpack_w(uint32_t x, uint32_t y) {
  return v4i{static_cast<int>(x & kHiNib), static_cast<int>(x & kLoNib),
             static_cast<int>(y & kHiNib), static_cast<int>(y & kLoNib)};
}

// GELU-tanh correction table (gelu_tanh.h), built at compile time from the generated
// list of {fp16 bits, exact - fast} pairs.
struct GeluFixEntry {
  uint16_t bits;
  int8_t d;
};
constexpr GeluFixEntry kGeluFixList[] = {
#include "gelu_tanh_fix.inc"
};
struct alignas(16) GeluFixTable {
  int8_t v[kGeluFixEntries];
};
constexpr GeluFixTable make_gelu_fix() {
  GeluFixTable t{};
  for (const GeluFixEntry& e : kGeluFixList) t.v[gelu_fix_index(e.bits)] = e.d;
  return t;
}
__device__ const GeluFixTable kGeluFix = make_gelu_fix();
constexpr bool gelu_fixes_in_window() {
  for (const GeluFixEntry& e : kGeluFixList)
    if (!gelu_fix_in_window(e.bits)) return false;
  return true;
}
static_assert(gelu_fixes_in_window(), "every GELU correction lies in the table window");

// torch.nn.functional.gelu(x, approximate="tanh") of an fp16 value, bit for bit: the fast
// evaluation plus the table's correction (`fix` is the table in global memory or LDS).
// Over every fp16 input, inf and NaN included, the result is identical to torch's eager
// GELU on the same GPU: the input domain is exactly the 2^16 fp16 values, so that
// exhaustive comparison covers all cases.
__device__ __forceinline__ _Float16 gelu_tanh_f16(_Float16 xh, const int8_t* fix) {
  const uint32_t xb = __builtin_bit_cast(uint16_t, xh);
  const int d = fix[gelu_fix_index(xb)];
  const uint32_t fb = gelu_tanh_fast_bits(xh);
  return __builtin_bit_cast(_Float16, static_cast<uint16_t>(fb + d));
}

// fp16 * fp16 as torch's eager mul: one fp32 product rounded to fp16.
__device__ __forceinline__ _Float16 mul_f16(_Float16 a, _Float16 b) {
  float y = static_cast<float>(a) * static_cast<float>(b);
  asm volatile("" : "+v"(y));
  return static_cast<_Float16>(y);
}

// fp16((float(acc) * sa) * sw) with both products rounded to fp32 first.  The empty asm
// keeps the fp32 product in a register: without it the backend folds the second multiply
// and the fp16 conversion into one v_fma_mixlo_f16, which rounds only once and differs
// from the reference's fp32-then-fp16 rounding on rare ties.
__device__ __forceinline__ _Float16 dequant(int32_t acc, float sa, float sw) {
  float y = __fmul_rn(__fmul_rn(static_cast<float>(acc), sa), sw);
  asm volatile("" : "+v"(y));
  return static_cast<_Float16>(y);
}

// The same from an fp32 accumulator that already holds acc exactly (the E3M2 MFMA's
// integer-valued fp32 sums): the identical two products and conversion.
__device__ __forceinline__ _Float16 dequant(float acc, float sa, float sw) {
  float y = __fmul_rn(__fmul_rn(acc, sa), sw);
  asm volatile("" : "+v"(y));
  return static_cast<_Float16>(y);
}

// E3M2 operand of one fragment from six consecutive dwords (the upper two are unused).
__device__ __forceinline__ v8i e3m2_op(v4i lo, int d4, int d5) { return v8i{lo.x, lo.y, lo.z, lo.w, d4, d5, 0, 0}; }

// RoPE of four dimension pairs (d, d + 128), each product and sum rounded to fp16 as
// torch's (x * cos) + (rotate_half(x) * sin) on fp16 tensors (attention.hip's rope_pair).
__device__ __forceinline__ void rope4(half4& lo, half4& hi, half4 clo, half4 chi, half4 slo, half4 shi) {
#pragma clang fp contract(off)
  const half4 a = lo * clo;
  const half4 b = hi * slo;
  const half4 c = hi * chi;
  const half4 e = lo * shi;
  lo = a - b;
  hi = c + e;
}

// Slot (16-byte, 8 halves) of key token t, dimensions dd .. dd + 7 (dd % 8 == 0) in the
// fragment-major K of one batch (kv_prep_kernel's layout).
__device__ __forceinline__ int kfrag_slot(int t, int dd) {
  return ((t >> 4) * 8 + (dd >> 5)) * 64 + (t & 15) + 16 * ((dd & 31) >> 3);
}
// Slot of dimension d, keys t0 .. t0 + 7 (t0 % 8 == 0) in the fragment-major V^T of one
// batch with nst 32-key steps.
__device__ __forceinline__ int64_t vfrag_slot(int d, int t0, int nst) {
  return (static_cast<int64_t>((d >> 4) * nst + (t0 >> 5))) * 64 + 16 * ((t0 & 31) >> 3) + (d & 15);
}

// ---- Down-projection quant in the gate/up launch (QFUSE).  The MLP's down projection
// quantizes h = gelu(gate) * up (K = 16384) right after the gate/up GEMM writes it
// (apply.py:138-141 -> int4_gemm.cu:496-531).  Rows of h can be rotated only once all of
// their 16384 columns are stored, i.e. once every n-tile of their m-tile is done, so the
// launch appends quant workgroups to the GEMM tiles: a GEMM workgroup counts its m-tile's
// completion after its stores (release at agent scope: the workgroups of one row block run
// on all eight XCDs), and a quant workgroup takes rows in increasing order from a shared
// counter, waits (bounded) for the row's m-tile, acquires, and runs the row through the
// K = 16384 quantizer of the standalone kernel (fwht_quant_row, 256 threads, one 68 KB LDS
// row), so the codes are those of pi05w4a4_quantize bit for bit.  The tiles are dealt
// m-tile-major within each XCD, so the first round of tiles completes whole row blocks and
// the quant workgroups that fill the slots left idle by the partial last round of tiles
// have rows to work on while it runs.
// No deadlock: a GEMM workgroup never waits, and each XCD dispatches its workgroups in
// index order, so a quant workgroup (index >= every GEMM tile's) only takes a slot on an
// XCD whose GEMM tiles have all been dispatched; those finish, so every counter reaches its
// target.  The wait is bounded anyway (spin_limit rounds of s_sleep): one that runs out
// leaves the row unquantized, sets *qstatus for the host and the workgroup leaves.
constexpr int kQuantLogK = 14;
constexpr int kQuantLogT = 8;
constexpr int kQuantR = 1 << (kQuantLogK - kQuantLogT);                             // 64 values per thread
constexpr int kQuantLrow = (1 << kQuantLogK) + 4 * ((1 << kQuantLogK) / kQuantR);   // LDS floats per row
constexpr int kQuantLdsBytes = kQuantLrow * 4 + 64;                                 // + reductions, broadcast

template <int TILE_ROWS>
__device__ __forceinline__ void down_quant_role(const GemmParams& p, char* lds) {
  float* const L = reinterpret_cast<float*>(lds);
  float* const red = L + kQuantLrow;
  int* const ired = reinterpret_cast<int*>(red + 4);
  int* const bcast = ired + 4;
  const int t = threadIdx.x;
  const int64_t M = p.m;
  const int nquant = static_cast<int>(gridDim.x) - p.ntiles * p.mtiles;
  int32_t* const next_row = p.qctl;
  int32_t* const exited = p.qctl + kMlpCtlExited;
  int32_t* const done = p.qctl + kMlpCtlHeader;  // m-tile i at done[kMlpCtlStride * i]
  const int target = p.ntiles + p.wait_extra;
  const _Float16* const h = static_cast<const _Float16*>(p.g[0].y);
  int32_t* const qcorr = p.dq + q_payload_words((M + 15) / 16, kblocks128(1 << kQuantLogK));
  for (;;) {
    if (t == 0) *bcast = __hip_atomic_fetch_add(next_row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int row = *bcast;
    __syncthreads();
    if (row >= M) {
      // No row left: the grab past the end is this workgroup's own warming slice.
      if (p.warm.nbuf > 0 && row - M < nquant) cache_warm_part<256>(p.warm, row - M, nquant, t);
      break;
    }
    const int mt = row / TILE_ROWS;
    if (t == 0) {
      int ready = 1;
      int spins = 0;
      // Long sleeps between polls: the polls bypass the caches, and at a round trip every
      // 0.25 us the waiting workgroups slowed the GEMM tiles beside them by 2x.
      while (__hip_atomic_load(done + kMlpCtlStride * mt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        if (++spins > p.spin_limit) {
          ready = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(127);
      }
      *bcast = ready;
    }
    __syncthreads();
    if (*bcast == 0) {
      if (t == 0 && p.qstatus != nullptr)
        __hip_atomic_store(p.qstatus, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      break;
    }
    // The row block's stores happen-before the counts this thread saw: acquire them.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    float v[kQuantR];
    const _Float16* xr = h + static_cast<int64_t>(row) * (1 << kQuantLogK) + t * kQuantR;
#pragma unroll
    for (int c = 0; c < kQuantR / 8; ++c) {
      const half8 hv = *reinterpret_cast<const half8*>(xr + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * c + e] = static_cast<float>(hv[e]);
    }
    fwht_quant_row<kQuantLogK, kQuantLogT>(v, L, red, ired, t, row, p.dq, p.dsa, qcorr, p.dinv_sqrt_k);
    __syncthreads();  // the next row reuses L, red and bcast
  }
  // The last quant workgroup to leave returns the control block to zero for the next launch
  // (every GEMM tile has counted by then, unless a wait ran out: the host then clears it).
  if (t == 0) {
    const int before = __hip_atomic_fetch_add(exited, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (before == nquant - 1) {
      for (int i = 0; i < p.mtiles; ++i)
        __hip_atomic_store(done + kMlpCtlStride * i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(next_row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(exited, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// E3M2: both operands in the E3M2 layouts of w4a4_internal.h (q6 fragments, w6 column
// pairs) and v_mfma_f32_16x16x128_f8f6f4: one MFMA per fragment pair and 128-deep k block
// (half the int8 MFMA issue time for the same work) and no unpack.  Its operands take
// 1.5x the bytes of INT4 codes, and a CU's vector-memory path delivers about one 64-lane
// 16-byte load per ~28 clocks, so the A fragments, which the four waves of the workgroup
// share, are staged once per workgroup in a double-buffered LDS tile by direct
// global-to-LDS loads (11 1 KB chunks per k block, dealt over the waves), and only the B
// column pairs stream per wave (three 16-byte loads per pair).  Step kb: wait for this
// wave's loads, workgroup barrier (every wave's A(kb) chunks are in LDS; every wave has
// read slot kb + 1 in step kb - 1), read A(kb) from LDS, issue A(kb + 1) and B(kb + 1),
// then the 28 MFMAs.  All LDS reads of a step precede its LDS-bound loads, so the
// compiler's conservative wait on those loads never lands before a read.  The fp32
// accumulators start at zero and end at acc exactly (no 16x factor, no corrections).
template <int MI, int NI, int NWAVES, int KW, bool GELU, int RING, int WPE, bool QKV_PREP = false, bool QFUSE = false,
          bool E3M2 = false, bool QPRO = false, int NKB = 0>
__global__ __launch_bounds__(64 * NWAVES) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm_w4a4_kernel(const GemmParams p) {
  static_assert(!(GELU && QKV_PREP), "the attention prep is a fp16 epilogue");
  static_assert(!QPRO || (MI == 1 && NWAVES == 4 && KW == 4 && RING >= 3 && !GELU && !QFUSE && !E3M2),
                "the quant prologue runs in the four K-split waves of one 16-row block");
  static_assert(!E3M2 || (NI % 2 == 0 && NWAVES == 4 && KW == 1 && !QFUSE && (!GELU || NI == 4)),
                "E3M2 operands: four waves along N, whole column pairs per wave");
  static_assert(!GELU || (NI % 2 == 0), "GELU pairing needs an even NI");
  static_assert(NWAVES % KW == 0 && (KW & (KW - 1)) == 0, "waves split as NW x KW");
  constexpr int NW = NWAVES / KW;
  // K split over the waves (one column block, KW k parts): the k parts are summed by a
  // reduce-scatter, after which wave w finishes the row blocks mi = w (mod KW), so that the
  // waves share the epilogue.
  static_assert(KW == 1 || NW == 1, "a K split covers one column block");
  constexpr bool kSpread = KW > 1;

  // ---- LDS: one pool carved at fixed offsets (the correction table, the tile's scales,
  // the k-reduction buffer, the output staging rows).  With QFUSE the down-projection
  // quant workgroups of the same launch reuse the pool for their row transposes.
  constexpr bool kFixWide = KW == 1;
  constexpr int kFixPieces = kGeluFixPosPieces + (kGeluFixEntries / 1024 - kGeluFixNegPiece0);
  constexpr int kFixCompact = kFixPieces * 1024;
  constexpr int TROWS = 16 * MI;
  constexpr int NCOL = 16 * NI * NW;  // GELU: the gate and the up columns of the tile
  // k reduction: row blocks per phase.  The 8-part tiles (one workgroup per CU) take half
  // the tile at a time; the 4-part ones keep the buffer at 32 KB (two workgroups per CU).
  constexpr int PM0 = KW == 8 ? (MI + 1) / 2 : (32 / (KW * NI) > 0 ? 32 / (KW * NI) : 1);
  constexpr int PM = PM0 < MI ? PM0 : MI;
  constexpr int OCW = GELU ? 8 * NI : 16 * NI;  // output columns of a wave
  constexpr int LSR = OCW + 8;                  // staged row stride in halves (pad)
  constexpr int kLdsFix = 0;
  constexpr int kLdsSa = kLdsFix + ((GELU ? (kFixWide ? kGeluFixEntries : kFixCompact) : 16) + 15) / 16 * 16;
  constexpr int kLdsSw = kLdsSa + TROWS * 4;
  constexpr int kLdsRed = kLdsSw + NCOL * 4;
  constexpr int kLdsStage = kLdsRed + (kSpread ? KW * PM * NI * 64 * 16 : 0);
  constexpr int kLdsA6 = (kLdsStage + (kSpread ? KW : NW) * 16 * LSR * 2 + 15) / 16 * 16;
  // E3M2 A stage: MI 1 KB chunks of d0-3 parts, then ceil(MI / 2) 1 KB chunks of the
  // concatenated 512-byte d4-5 parts (the last one half used when MI is odd).
  constexpr int kA6Chunks = MI + (MI + 1) / 2;
  constexpr int kA6Stage = kA6Chunks * 1024;
  // QPRO: the block's 16 rows of codes (K = 2048: 16 fragments of 1 KB), 16 row scales, 16
  // row corrections, then the two-wave rows' exchange (2 rows x 2 x 64 x 16 floats) and
  // reductions (2 rows x 2 floats, 2 x 2 ints).
  constexpr int kLdsPro = kLdsA6 + (E3M2 ? 2 * kA6Stage : 0);
  constexpr int kProXch = 16 * 1024 + 2 * 16 * 4;
  constexpr int kProRed = kProXch + 2 * 2 * 64 * 16 * 4;
  constexpr int kLdsGemm = kLdsPro + (QPRO ? kProRed + 8 * 4 : 0);
  constexpr int kLdsPool = (QFUSE && kQuantLdsBytes > kLdsGemm) ? kQuantLdsBytes : kLdsGemm;
  __shared__ __align__(16) char lds_pool[kLdsPool];
  int8_t* const fix_lds = reinterpret_cast<int8_t*>(lds_pool + kLdsFix);
  float* const epi_sa = reinterpret_cast<float*>(lds_pool + kLdsSa);  // row scales / 16 of the tile
  float* const epi_sw = reinterpret_cast<float*>(lds_pool + kLdsSw);  // column scales of the tile

  if constexpr (QFUSE) {
    static_assert(GELU && KW == 1, "the down-projection quant rides on the paired gate/up tiles");
    // Workgroups past the GEMM tiles quantize rows of h as their row blocks complete.
    if (static_cast<int>(blockIdx.x) >= p.ntiles * p.mtiles) {
      down_quant_role<16 * MI>(p, lds_pool);
      return;
    }
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform values are kept in scalar registers: fragment base addresses are scalar
  // and every load of a k block shares one 32-bit lane offset.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // QPRO: the M <= 4 rows are quantized here, by every workgroup for itself.  M <= 2: waves
  // 2r and 2r + 1 take row min(r, M - 1), 16 elements per lane (thread 64 (w & 1) + lane:
  // elements 16 t .. 16 t + 15, the two-wave quantizer), and each also holds the whole row
  // in the one-wave layout (lane l: elements 32 l .. 32 l + 31) for the norm's sum of squares
  // in the one-wave order; M = 3, 4: wave w takes row min(w, M - 1) in the one-wave layout.
  // The loads (and the norm weights') are issued first, so that the weight prefetches below
  // queue behind them and their wait covers these loads only.  Without a norm the weight
  // loads read the row again.
  half8 pro_x[QPRO ? 4 : 1], pro_w[QPRO ? 4 : 1], pro_x2[QPRO ? 2 : 1], pro_w2[QPRO ? 2 : 1];
  const int pro_t2 = 64 * (wave & 1) + lane;
  if constexpr (QPRO) {
    const int64_t prow = min(static_cast<int64_t>(p.m <= 2 ? (wave >> 1) : wave), p.m - 1);
    const _Float16* xrow = p.xpro + prow * 2048;
    const _Float16* wrow = p.nwpro != nullptr ? p.nwpro : xrow;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pro_x[c] = *reinterpret_cast<const half8*>(xrow + lane * 32 + 8 * c);
      pro_w[c] = *reinterpret_cast<const half8*>(wrow + lane * 32 + 8 * c);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      pro_x2[c] = *reinterpret_cast<const half8*>(xrow + pro_t2 * 16 + 8 * c);
      pro_w2[c] = *reinterpret_cast<const half8*>(wrow + pro_t2 * 16 + 8 * c);
    }
  }
  const int wn = wave % NW;  // column block of the wave
  const int wk = wave / NW;  // k part of the wave

  // ---- tile of this workgroup (XCD-aware order, see the header)
  int tile = blockIdx.x;
  {
    // XCD x = b % 8 owns the contiguous tiles [x*q + min(x, r), ..) with q = total / 8,
    // r = total % 8 (one more tile for the first r XCDs): a bijection for any total.
    const int total = p.ntiles * p.mtiles;
    const int x = tile & 7, q = total >> 3, r = total & 7;
    tile = x * q + min(x, r) + (tile >> 3);
  }
  int mt = tile % p.mtiles;
  int nt = tile / p.mtiles;
  if constexpr (QFUSE) {
    // Row blocks complete early: XCD x owns the n-tiles [x*per, (x+1)*per) and runs them
    // m-tile-major (a bijection whenever 8 divides the n-tile count).
    if ((p.ntiles & 7) == 0) {
      const int per = p.ntiles >> 3, i = static_cast<int>(blockIdx.x) >> 3;
      mt = i / per;
      nt = (static_cast<int>(blockIdx.x) & 7) * per + i % per;
    }
  }
  if constexpr (QKV_PREP) {
    // The K and V n-tiles (the groups after Q) carry the attention prep and so the longer
    // epilogue; they are spread evenly through the n order (one in every s positions), so
    // that no XCD's contiguous run of tiles is made of them only.  A bijection on the
    // n-tiles whenever their count divides the total.
    const int light = p.g[1].tile_begin, heavy = p.ntiles - light;
    if (p.rope_group > 0 && heavy > 0 && p.ntiles % heavy == 0) {
      const int s = p.ntiles / heavy, pos = nt;
      nt = (pos % s == s / 2) ? light + pos / s : pos - pos / s - (pos % s > s / 2 ? 1 : 0);
    }
  }
  const int ks = blockIdx.y;

  // GELU: the correction table goes to LDS for the epilogue's per-lane lookups.  Its two
  // halves are copied by direct global-to-LDS loads (no registers; lane L of a wave writes
  // bytes 16L..16L+15 of the wave's 1 KB piece).  Without a k split (KW == 1) the table
  // keeps its global layout, the zero run between the halves filled in place, so that a
  // lookup is gelu_fix_index's two instructions; with one, whose reduction buffer leaves
  // no room for 39 KB in the 8-part tiles, the halves are packed back to back
  // (kFixCompact) and the lookup adds the sign's half offset.  The copies complete under
  // the main loop; a vmcnt(0) wait and the barrier ahead of the epilogue order them (and
  // the fill) before the reads.
  if constexpr (GELU) {
    static_assert(kGeluFixEntries % 1024 == 0, "the table is copied in 1 KB pieces");
    for (int c = wave; c < kFixPieces; c += NWAVES) {
      const int piece = c < kGeluFixPosPieces ? c : kGeluFixNegPiece0 + (c - kGeluFixPosPieces);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(kGeluFix.v + piece * 1024 + lane * 16),
          (__attribute__((address_space(3))) void*)(fix_lds + (kFixWide ? piece : c) * 1024), 16, 0, 0);
    }
    if constexpr (kFixWide) {
      constexpr int kZero0 = kGeluFixPosPieces * 1024, kZero1 = kGeluFixNegPiece0 * 1024;
      for (int i = kZero0 + tid * 16; i < kZero1; i += 64 * NWAVES * 16)
        *reinterpret_cast<int4*>(fix_lds + i) = int4{0, 0, 0, 0};
    }
  }
  // LDS slot of the correction of fp16 bits xb.
  auto fix_slot = [](uint32_t xb) -> uint32_t {
    if constexpr (kFixWide) {
      return gelu_fix_index(xb);
    } else {
      const uint32_t off = (xb & 0x7fffu) - kGeluFixAbsBase;
      return (off < kGeluFixHalf - 1 ? off : kGeluFixHalf - 1) + (xb >> 15) * (kGeluFixPosPieces * 1024);
    }
  };

  // Group selection with scalar selects (no dynamic indexing of the argument struct).
  const int32_t* W = p.g[0].w;
  void* Y = p.g[0].y;
  int N = p.g[0].n;
  int tile_begin = 0;
  int col_off = 0;
  int gsel = 0;
  const int32_t* W2 = p.g[1].w;  // GELU: the up weight
  {
    int acc_off = p.g[0].n;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i) {
      if (!GELU && i < p.ngroups && nt >= p.g[i].tile_begin) {
        W = p.g[i].w;
        Y = p.g[i].y;
        N = p.g[i].n;
        tile_begin = p.g[i].tile_begin;
        col_off = acc_off;
        gsel = i;
      }
      if (i < p.ngroups) acc_off += p.g[i].n;
    }
  }

  const int K = p.k;
  const int KB128 = kblocks128(K);
  // Words per weight column before the scales: 16 per k block (INT4), 24 (E3M2).
  const int64_t scale_off = static_cast<int64_t>(KB128) * (E3M2 ? 24 : 16);
  const int64_t M = p.m;
  const int64_t m0 = static_cast<int64_t>(mt) * (16 * MI);
  // First output column of this wave (within the group).  In GELU mode a wave covers
  // 8*NI gate columns and the same up columns.
  const int wcol = GELU ? (nt * (8 * NI * NW) + wn * (8 * NI))
                        : ((nt - tile_begin) * (16 * NI * NW) + wn * (16 * NI));

  // Fragment base addresses.  Row blocks past M and column blocks past N are clamped to
  // the last valid block; their accumulators are never stored.
  const int nb_last = (N >> 4) - 1;
  const char* bbase[NI];
  bool bvalid[NI];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    int col;
    const int32_t* base;
    if (GELU) {
      col = wcol + (ni % (NI / 2)) * 16;
      base = (ni < NI / 2) ? W : W2;
    } else {
      col = wcol + ni * 16;
      base = W;
    }
    bvalid[ni] = col < N;
    const int nb = min(col >> 4, nb_last);
    bbase[ni] = reinterpret_cast<const char*>(base + static_cast<int64_t>(nb) * KB128 * 256);
  }
  const char* abase[MI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int mb = min(mt * MI + mi, p.mblocks - 1);
    abase[mi] = reinterpret_cast<const char*>(p.q + static_cast<int64_t>(mb) * KB128 * 256);
  }

  // k blocks of this wave: part wk of the workgroup's slice.
  int kb_begin, kb_end;
  {
    const int s0 = ks * p.kblocks_per_split;
    const int s1 = min(s0 + p.kblocks_per_split, KB128);
    const int per = (s1 - s0 + KW - 1) / KW;
    kb_begin = min(s0 + wk * per, s1);
    kb_end = min(kb_begin + per, s1);
  }
  const int nkb = kb_end - kb_begin;

  using AccV = std::conditional_t<E3M2, v4f, v4i>;
  AccV acc[MI][NI];

  // ---- main loop: A and B straight from global memory into a 2-deep register ring.
  // Each load is a scalar fragment base plus one shared unsigned 32-bit lane offset
  // (global_load_dwordx4 with an SGPR base): no per-load address arithmetic.
  uint4 ra[RING][MI];
  uint4 rb[RING][NI];
  auto load = [&](int kb, uint4 (&a)[MI], uint4 (&b)[NI]) {
    const uint32_t off = static_cast<uint32_t>(min(kb, kb_end - 1)) * 1024u + static_cast<uint32_t>(lane) * 16u;
    if constexpr (!QPRO) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) a[mi] = *reinterpret_cast<const uint4*>(abase[mi] + off);
    }
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) b[ni] = *reinterpret_cast<const uint4*>(bbase[ni] + off);
  };
  // QPRO: the activation fragment of block kb from the workgroup's LDS codes.
  const char* const pro_q = lds_pool + kLdsPro;
  auto load_a_lds = [&](int kb, uint4 (&a)[MI]) {
    const int kc = max(min(kb, kb_end - 1), 0);
    a[0] = *reinterpret_cast<const uint4*>(pro_q + static_cast<uint32_t>(kc) * 1024u + static_cast<uint32_t>(lane) * 16u);
  };
  // The two MFMAs of a 128-deep block (codes 0-15 and 16-31 of each lane's 32).  The
  // weights are operand A of the MFMA and the activations operand B, so accumulator
  // element r of lane L is output row 16*mi + L%16, column 16*ni + 4*(L/16) + r: four
  // consecutive columns of one row per lane.  Pad codes of a K that is not a multiple
  // of 128 multiply zero weight words: no guard.
  // The operands of a block's first MFMAs (all weight fragments of half 0 and activation
  // fragment 0) are unpacked at the end of the previous block, among its last MFMAs, so
  // that a block starts multiplying at once (nb0 / na0 carry them across blocks).
  v4i nb0[NI];
  v4i na0;
  auto unpack_first = [&](const uint4 (&a)[MI], const uint4 (&b)[NI]) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) nb0[ni] = unpack_w(b[ni].x, b[ni].y);
    na0 = unpack_a(a[0].x, a[0].y);
  };
  auto compute = [&](const uint4 (&a)[MI], const uint4 (&b)[NI], const uint4 (&an)[MI],
                     const uint4 (&bn)[NI]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i bop[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) bop[ni] = h ? unpack_w(b[ni].z, b[ni].w) : nb0[ni];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const v4i aop = h ? unpack_a(a[mi].z, a[mi].w) : (mi == 0 ? na0 : unpack_a(a[mi].x, a[mi].y));
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bop[ni], aop, acc[mi][ni], 0, 0, 0);
      }
    }
    unpack_first(an, bn);  // the next block (loaded one step ago)
  };
  // The first ring load is unconditional: with nkb == 0 it reads the clamped block
  // kb_end - 1 >= 0 and is never used.
  if constexpr (!E3M2) load(kb_begin, ra[0], rb[0]);
  if constexpr (QPRO) {
    // The rest of the weight prefetch goes out before the prologue's arithmetic.
#pragma unroll
    for (int d = 1; d < RING - 1; ++d) load(kb_begin + d, ra[d], rb[d]);
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * c + e] = static_cast<float>(pro_x[c][e]);
    // Codes, scales and corrections of the block's rows (rows past M hold a copy of row
    // M - 1; the rows after are never written: their outputs are never stored).
    int32_t* const lq = reinterpret_cast<int32_t*>(lds_pool + kLdsPro);
    float* const lsa = reinterpret_cast<float*>(lds_pool + kLdsPro + 16 * 1024);
    int32_t* const lqc = reinterpret_cast<int32_t*>(lds_pool + kLdsPro + 16 * 1024 + 16 * 4);
    if (p.m <= 2) {  // uniform over the workgroup: every wave joins the pair quantizer's barriers
      float v2[16];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) v2[8 * c + e] = static_cast<float>(pro_x2[c][e]);
      if (p.nwpro != nullptr) rms_norm_apply<16>(v2, pro_w2, rms_norm_rr_wave<2048>(v, p.eps_pro), p.unit_offset_pro);
      const int pr = wave >> 1;
      float* const xch = reinterpret_cast<float*>(lds_pool + kLdsPro + kProXch) + pr * 2 * 64 * 16;
      float* const redf = reinterpret_cast<float*>(lds_pool + kLdsPro + kProRed) + 2 * pr;
      int* const redi = reinterpret_cast<int*>(lds_pool + kLdsPro + kProRed + 4 * 4) + 2 * pr;
      fwht_quant_row_2wave<11>(v2, pro_t2, xch, redf, redi, true, pr, lq, lsa, lqc, p.inv_sqrt_k_pro);
    } else {
      if (p.nwpro != nullptr) rms_norm_row_wave<2048>(v, pro_w, p.eps_pro, p.unit_offset_pro);
      fwht_quant_row_wave<11>(v, lane, wave, lq, lsa, lqc, p.inv_sqrt_k_pro);
    }
    __syncthreads();
    load_a_lds(kb_begin, ra[0]);
  }

  // Accumulators start at the correction terms, qcorr[row] + wcorr[col], so that they end
  // at 16 * acc exactly (S + qcorr + wcorr).  Only the first k part of the first K slice
  // carries them: the other parts' sums are added to it.  Lane L owns rows 16*mi + L%16
  // and columns 16*ni + 4*(L/16) + 0..3 of its wave tile (see the epilogue).  Rows and
  // columns past the matrix read clamped, in-bounds words and are never stored.
  if constexpr (E3M2) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = AccV{0, 0, 0, 0};
  } else {
    const bool first_part = (ks == 0) && (wk == 0);
    int32_t qc[MI];
    if constexpr (QPRO) {
      qc[0] = reinterpret_cast<const int32_t*>(lds_pool + kLdsPro + 16 * 1024 + 16 * 4)[lane & 15];
    } else {
      const int32_t* qcorr = p.q + q_payload_words(p.mblocks, KB128);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) qc[mi] = qcorr[min(mt * MI + mi, p.mblocks - 1) * 16 + (lane & 15)];
    }
    v4i wc[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = GELU ? (wcol + (ni % (NI / 2)) * 16) : (wcol + ni * 16);
      const int32_t* wcorr = ((GELU && ni >= NI / 2) ? W2 : W) + N * scale_off + N;
      wc[ni] = *reinterpret_cast<const v4i*>(wcorr + min(col, N - 16) + (lane >> 4) * 4);
    }
    // The selection is applied to the MI + NI correction vectors, not to the MI x NI sums.
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) qc[mi] = first_part ? qc[mi] : 0;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) wc[ni] = first_part ? wc[ni] : v4i{0, 0, 0, 0};
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = wc[ni] + qc[mi];
  }

  // QKV attention prep, small tiles (2 x 2 fragments per wave): the K group's rotary
  // values are fetched now so that their latency hides under the main loop.  The loads
  // are unconditional (other waves read a fixed in-bounds word of the codes) to keep the
  // vmcnt bookkeeping exact.
  constexpr bool kRopePre = QKV_PREP && MI * (NI / 2) <= 2;
  half4 rpre[kRopePre ? MI : 1][kRopePre ? NI / 2 : 1][4];
  if constexpr (kRopePre) {
    const bool rope_wave = p.rope_group == gsel + 1;
    const _Float16* dummy = reinterpret_cast<const _Float16*>(p.q);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int j = 0; j < NI / 2; ++j) {
        const int64_t rl = min(m0 + mi * 16 + (lane & 15), M - 1);
        const int64_t off = rl * kAttnHeadDim + ((wcol >> 5) + j) * 16 + (lane >> 4) * 4;
        const _Float16* c = rope_wave ? p.cosb + off : dummy;
        const _Float16* sn = rope_wave ? p.sinb + off : dummy;
        const int hi = rope_wave ? 128 : 0;
        rpre[mi][j][0] = *reinterpret_cast<const half4*>(c);
        rpre[mi][j][1] = *reinterpret_cast<const half4*>(c + hi);
        rpre[mi][j][2] = *reinterpret_cast<const half4*>(sn);
        rpre[mi][j][3] = *reinterpret_cast<const half4*>(sn + hi);
      }
  }

  // Epilogue scales of the whole workgroup tile, fetched now so that their latency hides
  // under the main loop: thread t holds the row scale of tile row t % (16*MI) and the
  // column scale of tile column t % NCOL.  All indices are clamped, so every thread loads
  // unconditionally; columns past N get zero scales when staged to LDS after the loop.
  float e_sa;
  float e_sw;
  bool e_colvalid;
  {
    const int r = tid % TROWS;
    // The accumulator readout (kEpiAcc) has no row scales (p.sa may be null): it reads
    // the first M words of q instead, which always exist, and never uses the values.
    const float* sa_src = (p.sa != nullptr) ? p.sa : reinterpret_cast<const float*>(p.q);
    if constexpr (QPRO)
      e_sa = reinterpret_cast<const float*>(lds_pool + kLdsPro + 16 * 1024)[r & 15];
    else
      e_sa = sa_src[min(m0 + r, M - 1)];
    const int f = (tid / 16) % (NI * NW);  // fragment of the tile: wave f / NI, ni = f % NI
    const int fn = f % NI, fw = f / NI;
    const int fcol0 = GELU ? (nt * (8 * NI * NW) + fw * (8 * NI) + (fn % (NI / 2)) * 16)
                           : ((nt - tile_begin) * (16 * NI * NW) + fw * (16 * NI) + fn * 16);
    const int col = fcol0 + (tid & 15);
    e_colvalid = col < N;
    e_sw = __int_as_float((((GELU && fn >= NI / 2) ? W2 : W) + N * scale_off)[min(col, N - 1)]);
  }

  // Step s multiplies block kb_begin + s from ring slot s % RING and first prefetches
  // block s + RING - 1 into the slot freed by step s - 1.  The loop runs whole
  // iterations of RING steps; steps past nkb only load (clamped, in bounds) and skip
  // their multiply, so no memory instruction is conditional and the compiler's vmcnt
  // bookkeeping stays exact.
  if constexpr (E3M2) {
    // A: chunk c of a stage (c < MI: the d0-3 part of row block c of the tile; c >= MI:
    // bytes 1024 (c - MI) .. of the concatenated d4-5 parts; for odd MI the last chunk is
    // half used and its upper lanes re-read in-bounds bytes into an unread LDS area).  Wave
    // w issues chunks w, w + 4, ... below kA6Chunks.  Row blocks past M are clamped.
    constexpr int kAPerWave = (kA6Chunks + NWAVES - 1) / NWAVES;
    char* const a6 = lds_pool + kLdsA6;
    const char* agp[kAPerWave];
    int aoff[kAPerWave];
#pragma unroll
    for (int j = 0; j < kAPerWave; ++j) {
      const int c = min(wave + NWAVES * j, kA6Chunks - 1);
      int blk, off;
      if (c < MI) {
        blk = c;
        off = lane * 16;
      } else {
        const int t = (c - MI) * 1024 + lane * 16;
        blk = min(t >> 9, MI - 1);
        off = 1024 + (t & 511);
      }
      const int mb = min(mt * MI + blk, p.mblocks - 1);
      agp[j] = reinterpret_cast<const char*>(p.q) + static_cast<int64_t>(mb) * KB128 * kE3m2FragBytes + off;
      aoff[j] = c * 1024;
    }
    const int nachunks = (kA6Chunks - wave + NWAVES - 1) / NWAVES;
    auto load_a6 = [&](int kb, int slot) {
      const int64_t o = static_cast<int64_t>(min(kb, kb_end - 1)) * kE3m2FragBytes;
#pragma unroll
      for (int j = 0; j < kAPerWave; ++j) {
        if (j >= nachunks) break;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(agp[j] + o),
                                         (__attribute__((address_space(3))) void*)(a6 + slot * kA6Stage + aoff[j]),
                                         16, 0, 0);
      }
    };
    // B: the wave's NI / 2 column pairs (GELU: its gate pair and its up pair; else
    // consecutive pairs), pairs past N clamped.
    constexpr int NP = NI / 2;
    const char* bp6[NP];
#pragma unroll
    for (int qd = 0; qd < NP; ++qd) {
      const int pair = min((GELU ? wcol : wcol + 32 * qd) >> 5, (N >> 5) - 1);
      const int32_t* base = (GELU && qd == 1) ? W2 : W;
      bp6[qd] = reinterpret_cast<const char*>(base) + static_cast<int64_t>(pair) * KB128 * kE3m2PairBytes + lane * 16;
    }
    // A pair's three loads land in one 12-dword value, so that both fragments are
    // consecutive register runs of it (no copies to assemble the MFMA operands).
    v12i b6[2][NP];
    auto load_b6 = [&](int kb, v12i (&b)[NP]) {
      const int64_t o = static_cast<int64_t>(min(kb, kb_end - 1)) * kE3m2PairBytes;
#pragma unroll
      for (int qd = 0; qd < NP; ++qd) {
        const v4i c0 = *reinterpret_cast<const v4i*>(bp6[qd] + o);
        const v4i c1 = *reinterpret_cast<const v4i*>(bp6[qd] + o + 1024);
        const v4i c2 = *reinterpret_cast<const v4i*>(bp6[qd] + o + 2048);
        const v8i c01 = __builtin_shufflevector(c0, c1, 0, 1, 2, 3, 4, 5, 6, 7);
        const v8i c2x = __builtin_shufflevector(c2, c2, 0, 1, 2, 3, 4, 5, 6, 7);
        b[qd] = __builtin_shufflevector(c01, c2x, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11);
      }
    };
    load_a6(kb_begin, 0);
    load_b6(kb_begin, b6[0]);
    for (int i = 0; i < nkb; i += 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (i + j >= nkb) break;  // uniform over the workgroup: every wave has the same k range
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        const char* st = a6 + j * kA6Stage;
        v8i aop[MI];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const v4i lo = *reinterpret_cast<const v4i*>(st + mi * 1024 + lane * 16);
          const int2 hi = *reinterpret_cast<const int2*>(st + MI * 1024 + mi * 512 + lane * 8);
          aop[mi] = e3m2_op(lo, hi.x, hi.y);
        }
        __builtin_amdgcn_sched_barrier(0);
        // The last step requests nothing (uniform branch): every step starts with a full
        // vmcnt(0) wait, so no wait count depends on it.
        if (i + j + 1 < nkb) {
          load_a6(kb_begin + i + j + 1, j ^ 1);
          load_b6(kb_begin + i + j + 1, b6[j ^ 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) {
            // fragment ni: pair ni / 2, column half ni % 2 (dwords 0-5 or 6-11 of the record)
            const v12i r = b6[j][ni >> 1];
            const v8i bop = (ni & 1) ? __builtin_shufflevector(r, r, 6, 7, 8, 9, 10, 11, 6, 7)
                                     : __builtin_shufflevector(r, r, 0, 1, 2, 3, 4, 5, 0, 1);
            acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bop, aop[mi], acc[mi][ni], 3, 3, 0, 0, 0, 0);
          }
        }
      }
    }
    // The clamped prefetches of the last step land before the LDS is reused or the wave ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else if constexpr (NKB > 0) {
    // Every wave's slice is exactly NKB blocks (the host launches this form only then): a
    // straight-line loop whose loads are all known at compile time, so that no clamped
    // load is issued past the last block and the compiler's waits are exact.  Block s
    // goes to ring slot s % RING, requested RING - 1 steps ahead.
    static_assert(!QPRO && !GELU, "fixed-length K slices: plain and attention-prep tiles");
#pragma unroll
    for (int d = 1; d < RING - 1 && d < NKB; ++d) load(kb_begin + d, ra[d], rb[d]);
    unpack_first(ra[0], rb[0]);
#pragma unroll
    for (int s = 0; s < NKB; ++s) {
      if (s + RING - 1 < NKB) load(kb_begin + s + RING - 1, ra[(s + RING - 1) % RING], rb[(s + RING - 1) % RING]);
      __builtin_amdgcn_sched_barrier(0);
      compute(ra[s % RING], rb[s % RING], ra[(s + 1) % RING], rb[(s + 1) % RING]);
    }
  } else {
  if constexpr (!QPRO) {
#pragma unroll
    for (int d = 1; d < RING - 1; ++d) load(kb_begin + d, ra[d], rb[d]);
  }
  if constexpr (QPRO) load_a_lds(kb_begin + 1, ra[1 % RING]);
  unpack_first(ra[0], rb[0]);
  for (int i = 0; i < nkb; i += RING) {
#pragma unroll
    for (int j = 0; j < RING; ++j) {
      load(kb_begin + i + j + RING - 1, ra[(j + RING - 1) % RING], rb[(j + RING - 1) % RING]);
      // Keep each prefetch at the top of its step: under register pressure the
      // scheduler would otherwise sink the loads next to their use.
      __builtin_amdgcn_sched_barrier(0);
      // GELU, first step: vector loads complete in issue order, so once at most the
      // MI + NI loads just issued are outstanding, the correction table's direct loads
      // (issued first) have landed; the first block's operands, issued after them, are
      // awaited here anyway.
      if constexpr (GELU) {
        if (i == 0 && j == 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(MI + NI) : "memory");
      }
      // QPRO: the activation fragment two blocks ahead, from LDS (slots j, j + 1 hold this
      // block's and the next one's).
      if constexpr (QPRO) load_a_lds(kb_begin + i + j + 2, ra[(j + 2) % RING]);
      if (j == 0 || i + j < nkb) compute(ra[j], rb[j], ra[(j + 1) % RING], rb[(j + 1) % RING]);
    }
  }
  }

  // A wave without k blocks never waited for its correction-table loads (see the first
  // step above): it waits now, before the barrier below (or the k reduction's) publishes
  // the table to the other waves.
  if constexpr (GELU) {
    if (nkb == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  if (tid < TROWS) epi_sa[tid] = E3M2 ? e_sa : e_sa * 0.0625f;  // INT4: the accumulators hold 16 acc
  if (tid < NCOL) epi_sw[tid] = e_colvalid ? e_sw : 0.0f;
  if constexpr (KW == 1) __syncthreads();  // KW > 1: the k reduction below synchronises

  // Residual (fp16 mode, one group): the 16-byte row pieces this wave's epilogue stores
  // (see the store loop below) are loaded now, so that their latency hides under the k
  // reduction and the staging instead of stalling every store.  Addresses are clamped into
  // the matrix; pieces outside it are never stored.
  constexpr int ROCW = 16 * NI;
  constexpr int RLPR = ROCW / 8;
  constexpr int RRPI = 64 / RLPR;
  constexpr int RJ = (16 + RRPI - 1) / RRPI;
  uint4 resv[GELU ? 1 : MI][GELU ? 1 : RJ];
  const bool has_res = !GELU && p.res != nullptr && p.mode == kEpiFp16;
  if constexpr (!GELU) {
    if (has_res && (kSpread || wk == 0)) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int j = 0; j < RJ; ++j) {
          if (kSpread && mi % KW != wk) continue;
          const int rr = min(j * RRPI + lane / RLPR, 15);
          const int64_t row = min(m0 + mi * 16 + rr, M - 1);
          const int col = min(wcol + (lane % RLPR) * 8, N - 8);
          resv[mi][j] = *reinterpret_cast<const uint4*>(p.res + row * N + col);
        }
    }
  }

  // ---- k-part reduction through LDS (KW > 1): in phases of PM row blocks, every wave
  // stores its parts of the phase's row blocks and the owner of each row block (wave
  // mi mod KW) sums the KW parts of its fragments (int32: any order gives the same sum).
  if constexpr (kSpread) {
    v4i* const red = reinterpret_cast<v4i*>(lds_pool + kLdsRed);  // KW * PM * NI * 64
#pragma unroll
    for (int ph = 0; ph * PM < MI; ++ph) {
#pragma unroll
      for (int i = 0; i < PM; ++i) {
        if (ph * PM + i >= MI) continue;
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) red[((wk * PM + i) * NI + ni) * 64 + lane] = acc[ph * PM + i][ni];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < PM; ++i) {
        const int mi = ph * PM + i;
        if (mi >= MI || mi % KW != wk) continue;
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          v4i sum = red[(i * NI + ni) * 64 + lane];
#pragma unroll
          for (int w = 1; w < KW; ++w) sum += red[((w * PM + i) * NI + ni) * 64 + lane];
          acc[mi][ni] = sum;
        }
      }
      if ((ph + 1) * PM < MI) __syncthreads();
    }
    if (wk >= MI) return;  // no row block to finish
  }

  // ---- epilogue.  Lane L holds rows 16*mi + L%16 and columns 16*ni + 4*(L/16) + 0..3.
  const int lrow = lane & 15;
  const int lcol = (lane >> 4) * 4;
  auto out_col = [&](int ni) {  // first of the lane's four columns of fragment ni
    return GELU ? (wcol + (ni % (NI / 2)) * 16 + lcol) : (wcol + ni * 16 + lcol);
  };
  // The accumulators hold 16 * acc.  Row scales come from LDS pre-divided by 16, which
  // folds that factor into the scale: float(16 t) * (sa / 16) rounds exactly like
  // float(t) * sa (both rescalings are exact powers of two).
  if (p.mode == kEpiFp16 || p.mode == kEpiGeluUp) {
    float sv[MI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) sv[mi] = epi_sa[mi * 16 + lrow];
    float4 sw[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) sw[ni] = *reinterpret_cast<const float4*>(&epi_sw[(wn * NI + ni) * 16 + lcol]);
    // Each 16-row block of the wave's output is staged in LDS (8-byte writes of a lane's
    // four columns) and written back as whole rows with 16-byte stores: a wave row of
    // 64 (GELU: 32) fp16 columns is 128 (64) contiguous bytes.  The staging area is
    // private to the wave.
    constexpr int LPR = OCW / 8;                  // lanes per row, 16 bytes each
    constexpr int RPI = 64 / LPR;                 // rows per store instruction
    static_assert(16 % RPI == 0 || RPI % 16 == 0, "store rows must tile the 16-row block");
    _Float16* const stage = reinterpret_cast<_Float16*>(lds_pool + kLdsStage) + (kSpread ? wk : wn) * (16 * LSR);
    // Stores address the wave's output block through a scalar base and a 32-bit lane
    // offset (the block spans at most 16*MI rows of N columns).
    char* yw = reinterpret_cast<char*>(static_cast<_Float16*>(Y) + m0 * N + wcol);
    // Residual (one-group fp16 mode): y = fp16(y + res), the rounding of torch's fp16 add.
    static_assert(GELU || (LPR == RLPR && RPI == RRPI), "residual pieces follow the store layout");
    // Attention prep (QKV): this wave's group is K in RoPE-pair order, or V.
    const bool rope = QKV_PREP && p.rope_group == gsel + 1;
    const bool vtr = QKV_PREP && p.vt_group == gsel + 1;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      if (kSpread && mi % KW != wk) continue;  // another wave's row block
      half4 ob[GELU ? 1 : NI];
#pragma unroll
      for (int ni = 0; ni < (GELU ? NI / 2 : NI); ++ni) {
        const AccV s = acc[mi][ni];
        const float swv[4] = {sw[ni].x, sw[ni].y, sw[ni].z, sw[ni].w};
        half4 o;
        if (GELU) {
          const AccV su = acc[mi][ni + NI / 2];
          const float swu[4] = {sw[ni + NI / 2].x, sw[ni + NI / 2].y, sw[ni + NI / 2].z, sw[ni + NI / 2].w};
          // The four table lookups are issued ahead of the GELU arithmetic, which hides
          // their LDS latency.  The product with up is a packed fp16 multiply: the product
          // of two fp16 values is exact in fp32, so one fp16 rounding of it is the eager
          // fp16 mul's result (fp32 product, rounded to fp16).
          _Float16 g16[4];
          half4 u16;
          int fix[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            g16[r] = dequant(s[r], sv[mi], swv[r]);
            u16[r] = dequant(su[r], sv[mi], swu[r]);
            fix[r] = fix_lds[fix_slot(__builtin_bit_cast(uint16_t, g16[r]))];
          }
          half4 gl;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            gl[r] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(gelu_tanh_fast_bits(g16[r]) + fix[r]));
          o = gl * u16;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = dequant(s[r], sv[mi], swv[r]);
        }
        if constexpr (GELU)
          *reinterpret_cast<half4*>(stage + lrow * LSR + ni * 16 + lcol) = o;
        else
          ob[ni] = o;
      }
      if constexpr (!GELU) {
        if (rope) {
          // Fragment pair (2j, 2j + 1) holds key dimensions d .. d + 3 and d + 128 .. d + 131
          // of the lane's row: RoPE, then the fragment-major K copy; the staged key states
          // are stored in dimension order below.
          const int64_t r = m0 + mi * 16 + lrow;
          const int64_t rl = min(r, M - 1);
          const int rb = static_cast<int>(rl / p.seq);
          const int t = static_cast<int>(rl) - rb * p.seq;
          _Float16* kf = p.kv + static_cast<int64_t>(rb) * 2 * p.s_pad * kAttnHeadDim;
#pragma unroll
          for (int j = 0; j < NI / 2; ++j) {
            const int d = ((wcol >> 5) + j) * 16 + lcol;
            if constexpr (kRopePre) {
              rope4(ob[2 * j], ob[2 * j + 1], rpre[mi][j][0], rpre[mi][j][1], rpre[mi][j][2], rpre[mi][j][3]);
            } else {
              const _Float16* cr = p.cosb + rl * kAttnHeadDim + d;
              const _Float16* sr = p.sinb + rl * kAttnHeadDim + d;
              rope4(ob[2 * j], ob[2 * j + 1], *reinterpret_cast<const half4*>(cr),
                    *reinterpret_cast<const half4*>(cr + 128), *reinterpret_cast<const half4*>(sr),
                    *reinterpret_cast<const half4*>(sr + 128));
            }
            if (r < M) {
              *reinterpret_cast<half4*>(kf + kfrag_slot(t, d & ~7) * 8 + (d & 7)) = ob[2 * j];
              *reinterpret_cast<half4*>(kf + kfrag_slot(t, (d + 128) & ~7) * 8 + (d & 7)) = ob[2 * j + 1];
            }
          }
        }
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) *reinterpret_cast<half4*>(stage + lrow * LSR + ni * 16 + lcol) = ob[ni];
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < (16 + RPI - 1) / RPI; ++j) {
        const int rr = j * RPI + lane / LPR;
        const int trow = mi * 16 + rr;  // row within the tile
        const int tcol = (lane % LPR) * 8;
        uint4 v = *reinterpret_cast<const uint4*>(stage + min(rr, 15) * LSR + tcol);
        // Non-temporal: the outputs are not re-read by this kernel, so they should not
        // displace the weights streaming through L2 (measured 1-3% faster).
        if (rr < 16 && m0 + trow < M && wcol + tcol < N) {
          const uint32_t off = static_cast<uint32_t>(trow * N + tcol) * 2u;
          char* dst = yw + off;
          if constexpr (!GELU) {
            if (has_res) {
              half8 o8 = __builtin_bit_cast(half8, v);
              o8 += __builtin_bit_cast(half8, resv[mi][j]);
              v = __builtin_bit_cast(uint4, o8);
            }
            if (rope) {
              // GEMM column gc = 32P + 16h + c is key dimension 16P + 128h + c
              const int gc = wcol + tcol;
              const int kd = ((gc >> 5) + 8 * ((gc >> 4) & 1)) * 16 + (gc & 15);
              dst = reinterpret_cast<char*>(static_cast<_Float16*>(Y) + (m0 + trow) * N + kd);
            }
          }
          __builtin_nontemporal_store(v4i{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)},
                                      reinterpret_cast<v4i*>(dst));
        }
      }
      if constexpr (!GELU) {
        if (vtr) {
          // V^T fragments: lane pairs (dimension, 8-key group) of the staged 16 rows.  A row
          // group never straddles two batches (seq and the tile rows are multiples of 8).
          const int nst = p.s_pad / 32;
#pragma unroll
          for (int it = 0; it < NI / 2; ++it) {
            const int idx = lane + 64 * it;
            const int dim = idx % OCW;
            const int kg = idx / OCW;
            const int64_t row0 = m0 + mi * 16 + kg * 8;
            half8 x;
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = stage[(kg * 8 + e) * LSR + dim];
            if (row0 < M && wcol + dim < N) {
              const int rb = static_cast<int>(row0 / p.seq);
              const int t0 = static_cast<int>(row0) - rb * p.seq;
              _Float16* vf = p.kv + (static_cast<int64_t>(rb) * 2 + 1) * p.s_pad * kAttnHeadDim;
              *reinterpret_cast<half8*>(vf + vfrag_slot(wcol + dim, t0, nst) * 8) = x;
            }
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    if constexpr (!GELU) {
      if ((rope || vtr) && (!kSpread || wk == 0)) {
        // Keys seq .. s_pad - 1 of every batch whose last token lies in this tile: zeros.
        const int npad = p.s_pad - p.seq;
        const int64_t mend = min(m0 + 16 * MI, M);
        for (int64_t b = m0 / p.seq; b * p.seq < mend; ++b) {
          const int64_t last = b * p.seq + p.seq - 1;
          if (last < m0 || last >= mend) continue;
          _Float16* kf = p.kv + b * 2 * p.s_pad * kAttnHeadDim;
          if (rope) {
            constexpr int NG = NI * 2;  // 8-dimension groups of the wave's key dimensions
            for (int idx = lane; idx < npad * NG; idx += 64) {
              const int t = p.seq + idx / NG;
              const int g = idx % NG;
              const int dd = ((wcol >> 5) + (g >> 2) + 8 * ((g >> 1) & 1)) * 16 + 8 * (g & 1);
              *reinterpret_cast<half8*>(kf + kfrag_slot(t, dd) * 8) = half8{};
            }
          } else {
            _Float16* vf = kf + static_cast<int64_t>(p.s_pad) * kAttnHeadDim;
            const int nst = p.s_pad / 32;
            for (int idx = lane; idx < (npad / 8) * OCW; idx += 64) {
              const int d = wcol + idx % OCW;
              const int t0 = p.seq + 8 * (idx / OCW);
              if (d < N) *reinterpret_cast<half8*>(vf + vfrag_slot(d, t0, nst) * 8) = half8{};
            }
          }
        }
      }
    }
    if constexpr (QFUSE) {
      // This tile's part of h is stored: count it for its row block.  Each wave waits for
      // its own stores to be acknowledged, the barrier gathers the waves, and one release
      // at agent scope (the consumers run on any XCD) precedes the count.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_fetch_add(p.qctl + kMlpCtlHeader + kMlpCtlStride * mt, 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  } else if constexpr (!E3M2) {
    // kEpiPartial: partial sums of 16 * acc, int32 [ksplit, M, n_total] at column
    // col_off + col (slice 0 carries the corrections);
    // kEpiAcc:     int32 [M, N] accumulators of the group, (16 * acc) / 16.
    int32_t* out;
    int64_t ld;
    if (p.mode == kEpiPartial) {
      out = p.partial + static_cast<int64_t>(ks) * M * p.n_total + col_off;
      ld = p.n_total;
    } else {
      out = static_cast<int32_t*>(Y);
      ld = N;
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int64_t row = m0 + mi * 16 + lrow;
      if ((kSpread && mi % KW != wk) || row >= M) continue;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        if (!bvalid[ni]) continue;
        // partial columns in GELU mode: gate block [0, N), up block [N, 2N)
        const int col = out_col(ni) + ((GELU && ni >= NI / 2) ? N : 0);
        v4i v = acc[mi][ni];
        if (p.mode == kEpiAcc) v = v >> 4;  // exact: a multiple of 16
        *reinterpret_cast<v4i*>(out + row * ld + col) = v;
      }
    }
  }
}

// Sum the split-K partials and apply the epilogue.  Each thread owns 4 consecutive
// output columns of one row.
template <bool GELU>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmParams p) {
  const int64_t M = p.m;
  const int ncols = GELU ? p.gelu_pair_n : p.n_total;
  const int64_t quads = static_cast<int64_t>(ncols) / 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= M * quads) return;
  const int64_t row = idx / quads;
  const int c = static_cast<int>(idx % quads) * 4;
  const int64_t scale_off = static_cast<int64_t>(kblocks128(p.k)) * 16;
  const int64_t plane = M * p.n_total;
  const float sav = p.sa[row] * 0.0625f;  // the sums below are 16 * acc
  // Partials are read four slices at a time (clamped slice indices, masked sums), so that
  // four loads are in flight per thread instead of one dependent load per slice.
  auto sum_slices = [&](int col) {
    v4i s = v4i{0, 0, 0, 0};
    const int32_t* base = p.partial + row * p.n_total + col;
    for (int k0 = 0; k0 < p.ksplit; k0 += 4) {
      v4i a[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        a[j] = *reinterpret_cast<const v4i*>(base + min(k0 + j, p.ksplit - 1) * plane);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (k0 + j < p.ksplit) s += a[j];
    }
    return s;
  };
  if (GELU) {
    const int N = p.gelu_pair_n;
    const v4i g = sum_slices(c);
    const v4i u = sum_slices(N + c);
    const float* swg = reinterpret_cast<const float*>(p.g[0].w + N * scale_off);
    const float* swu = reinterpret_cast<const float*>(p.g[1].w + N * scale_off);
    const int gv[4] = {g[0], g[1], g[2], g[3]};
    const int uv[4] = {u[0], u[1], u[2], u[3]};
    _Float16* y = static_cast<_Float16*>(p.g[0].y) + row * N + c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y[e] = mul_f16(gelu_tanh_f16(dequant(gv[e], sav, swg[c + e]), kGeluFix.v), dequant(uv[e], sav, swu[c + e]));
    }
    return;
  }
  const v4i s = sum_slices(c);
  // locate the group of column c (groups are consecutive in the partial columns)
  const int32_t* W = p.g[0].w;
  void* Y = p.g[0].y;
  int N = p.g[0].n;
  int off = 0;
  int acc_off = p.g[0].n;
#pragma unroll
  for (int i = 1; i < kMaxGroups; ++i) {
    if (i < p.ngroups && c >= acc_off) {
      W = p.g[i].w;
      Y = p.g[i].y;
      N = p.g[i].n;
      off = acc_off;
    }
    if (i < p.ngroups) acc_off += p.g[i].n;
  }
  const int col = c - off;
  const float* sw = reinterpret_cast<const float*>(W + N * scale_off);
  _Float16* y = static_cast<_Float16*>(Y) + row * N + col;
  const int sv[4] = {s[0], s[1], s[2], s[3]};
  const _Float16* res = p.res != nullptr ? p.res + row * N + col : nullptr;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const _Float16 o = dequant(sv[e], sav, sw[col + e]);
    y[e] = res != nullptr ? static_cast<_Float16>(o + res[e]) : o;
  }
}

// Elementwise y = fp16(gelu_tanh(g) * u) on fp16 inputs: the gate/up epilogue's arithmetic
// on given values (grid-stride loop).
__global__ __launch_bounds__(256) void gelu_up_kernel(const _Float16* g, const _Float16* u, int64_t n,
                                                      _Float16* y) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
    y[i] = mul_f16(gelu_tanh_f16(g[i], kGeluFix.v), u[i]);
}

template <int MI, int NI, int NWAVES, int KW, int RING = 2, int WPE = 2>
hipError_t launch_cfg(const GemmParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.ntiles) * static_cast<unsigned>(p.mtiles),
                  static_cast<unsigned>(p.ksplit));
  if (p.mode == kEpiGeluUp || (p.mode == kEpiPartial && p.gelu_pair_n > 0))
    gemm_w4a4_kernel<MI, NI, NWAVES, KW, true, RING, WPE><<<grid, 64 * NWAVES, 0, stream>>>(p);
  else if (p.rope_group > 0)
    gemm_w4a4_kernel<MI, NI, NWAVES, KW, false, RING, WPE, true><<<grid, 64 * NWAVES, 0, stream>>>(p);
  else
    gemm_w4a4_kernel<MI, NI, NWAVES, KW, false, RING, WPE><<<grid, 64 * NWAVES, 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(GemmParams p, int tile_cfg, hipStream_t stream) {
  switch (tile_cfg) {
    case kCfg7x4: return launch_cfg<7, 4, 4, 1>(p, stream);
    case kCfg7x4K4: return launch_cfg<7, 4, 4, 4>(p, stream);
    case kCfg7x4K8: {
      // K = 16384 in one slice: 16 blocks per wave, the straight-line form (down + residual
      // at 776 rows 22.1-22.2 -> 21.7 us).
      if (p.k == 16384 && p.ksplit == 1 && p.kblocks_per_split == 128 && p.mode == kEpiFp16 && p.rope_group == 0) {
        const dim3 grid(static_cast<unsigned>(p.ntiles) * static_cast<unsigned>(p.mtiles));
        gemm_w4a4_kernel<7, 4, 8, 8, false, 2, 2, false, false, false, false, 16><<<grid, 512, 0, stream>>>(p);
        return hipGetLastError();
      }
      return launch_cfg<7, 4, 8, 8>(p, stream);
    }
    case kCfg7x2: return launch_cfg<7, 2, 4, 1>(p, stream);
    case kCfg4x2: return launch_cfg<4, 2, 4, 1>(p, stream);
    // 32 x 128 tiles stream the whole K per wave: a 3-deep ring hides more of the load
    // latency (the QKV and o GEMMs of the forward: 11.0 -> 10.1 us each).
    case kCfg2x2: return launch_cfg<2, 2, 4, 1, 3, 2>(p, stream);
    case kCfg1x2: return launch_cfg<1, 2, 4, 1>(p, stream);
    // Small M: four waves split K with a 4-deep ring (one workgroup streams 32 columns of
    // weights; at M = 1 the QKV GEMM takes 3.0 us against 5.8 us for 16 x 128 tiles with
    // a global K split and its reduce launch).
    case kCfg1x2K4: return launch_cfg<1, 2, 4, 4, 4, 2>(p, stream);
    case kCfg2x2K4: return launch_cfg<2, 2, 4, 4, 4, 2>(p, stream);
    case kCfg4x2K4: return launch_cfg<4, 2, 4, 4, 4, 2>(p, stream);
    // Mid-size M: 64 x 64 tiles whose four waves split K, with a 2-deep ring (deeper rings
    // measured slower: o 6.9 us at ring 2, 7.5 at ring 4).
    case kCfg4x4K4: {
      // K = 2048 in one slice: every wave's part is exactly 4 blocks, so the straight-line
      // form runs (no clamped load past the last block; QKV + RoPE at 776 rows 8.55 ->
      // 8.27 us, o unchanged; 3- or 4-deep rings measured slower for o: 6.90 / 7.00 us).
      if (p.k == 2048 && p.ksplit == 1 && p.kblocks_per_split == 16 && p.mode == kEpiFp16) {
        const dim3 grid(static_cast<unsigned>(p.ntiles) * static_cast<unsigned>(p.mtiles));
        if (p.rope_group > 0)
          gemm_w4a4_kernel<4, 4, 4, 4, false, 2, 2, true, false, false, false, 4><<<grid, 256, 0, stream>>>(p);
        else
          gemm_w4a4_kernel<4, 4, 4, 4, false, 2, 2, false, false, false, false, 4><<<grid, 256, 0, stream>>>(p);
        return hipGetLastError();
      }
      return launch_cfg<4, 4, 4, 4, 2, 2>(p, stream);
    }
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_qpro(const GemmParams& p, hipStream_t stream) {
  if (p.m < 1 || p.m > kQproMaxRows || p.k != 2048 || p.mtiles != 1 || p.ksplit != 1 || p.mode != kEpiFp16 ||
      p.rope_group != 0 || p.xpro == nullptr)
    return hipErrorInvalidValue;
  // A 5-deep ring: all four k blocks of a wave's weights are requested before the prologue,
  // so that no weight fetch waits behind the quant arithmetic.
  gemm_w4a4_kernel<1, 2, 4, 4, false, 5, 2, false, false, false, true>
      <<<dim3(static_cast<unsigned>(p.ntiles)), 256, 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_gemm_gelu_quant(const GemmParams& p, int nquant, hipStream_t stream) {
  if (p.mode != kEpiGeluUp || p.ksplit != 1 || p.gelu_pair_n != (1 << kQuantLogK) || nquant < 1)
    return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(p.ntiles) * static_cast<unsigned>(p.mtiles) + static_cast<unsigned>(nquant));
  gemm_w4a4_kernel<7, 4, 4, 1, true, 2, 2, false, true><<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_gemm_e3m2(const GemmParams& p, int tile_cfg, hipStream_t stream) {
  if (p.ksplit != 1 || (p.mode != kEpiFp16 && p.mode != kEpiGeluUp)) return hipErrorInvalidValue;
  const bool gelu = p.mode == kEpiGeluUp;
  const bool prep = p.rope_group > 0;
  if ((gelu && (prep || p.res != nullptr || tile_cfg != kCfg7x4)) || (tile_cfg != kCfg7x4 && tile_cfg != kCfg2x2))
    return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(p.ntiles) * static_cast<unsigned>(p.mtiles));
  if (gelu)
    gemm_w4a4_kernel<7, 4, 4, 1, true, 2, 2, false, false, true><<<grid, 256, 0, stream>>>(p);
  else if (tile_cfg == kCfg7x4 && !prep)
    gemm_w4a4_kernel<7, 4, 4, 1, false, 2, 2, false, false, true><<<grid, 256, 0, stream>>>(p);
  else if (tile_cfg == kCfg7x4)
    gemm_w4a4_kernel<7, 4, 4, 1, false, 2, 2, true, false, true><<<grid, 256, 0, stream>>>(p);
  else if (!prep)
    gemm_w4a4_kernel<2, 2, 4, 1, false, 2, 2, false, false, true><<<grid, 256, 0, stream>>>(p);
  else
    gemm_w4a4_kernel<2, 2, 4, 1, false, 2, 2, true, false, true><<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_gelu_up(const void* g, const void* u, int64_t n, void* y, hipStream_t stream) {
  const int64_t blocks = (n + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks < 16384 ? blocks : 16384));
  gelu_up_kernel<<<grid, 256, 0, stream>>>(static_cast<const _Float16*>(g), static_cast<const _Float16*>(u), n,
                                           static_cast<_Float16*>(y));
  return hipGetLastError();
}

hipError_t launch_splitk_reduce(const GemmParams& p, hipStream_t stream) {
  const int ncols = p.gelu_pair_n > 0 ? p.gelu_pair_n : p.n_total;
  const int64_t threads = p.m * (ncols / 4);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (p.gelu_pair_n > 0)
    splitk_reduce_kernel<true><<<grid, 256, 0, stream>>>(p);
  else
    splitk_reduce_kernel<false><<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace w4a4
