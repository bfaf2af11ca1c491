// W4A4 GEMM for gfx950: int4 codes unpacked to int8, CDNA4 int8 MFMA
// (v_mfma_i32_16x16x64_i8), int32 accumulation, dequant epilogue.
//
// Reference semantics (pi05_fast/w4a4/csrc/int4_gemm.cu:63-204, 206-394; pack.py:134-145):
//   acc[m, n] = sum_k qa[m, k] * qw[n, k]            (int32, exact)
//   y[m, n]   = fp16((float(acc) * sa[m]) * sw[n])   (two fp32 products, RNE to fp16)
//
// INT4 -> INT8.  A packed word holds codes k0..k7 as nibbles 0..7.  Two ALU ops per
// int8 word produce the codes scaled by 16 with their sign intact:
//   w & 0xF0F0F0F0        -> bytes 16*k1, 16*k3, 16*k5, 16*k7
//   (w << 4) & 0xF0F0F0F0 -> bytes 16*k0, 16*k2, 16*k4, 16*k6
// A and B are unpacked identically, so byte position p of an MFMA operand holds the same
// k for both (the dot product is invariant under a common permutation of k), and the
// int32 accumulator equals 256 * acc exactly: |256 * acc| <= 256 * 64 * K < 2^31 for
// K <= 65536 per K slice (the host splits larger K).  The epilogue shifts it back.
//
// Tiling.  A wave owns a (16*MI) x (16*NI) tile = MI x NI accumulators of 16x16.  The 4
// waves of a workgroup are arranged NW along N times KW along K (NW * KW = 4): with
// KW > 1 the waves of one column block split the workgroup's k range into KW contiguous
// parts and add their accumulators through LDS at the end, which gives narrow GEMMs
// (QKV, o, down) enough workgroups without a global split-K workspace.
// Both operands live in HBM in the same MFMA-fragment-major layout (frag_word_index: one
// 1 KB fragment per 16 rows/columns x 128 k; lane L loads slot L = 32 codes of row/
// column L%16, the operands of the block's two MFMAs), so every operand fetch is one
// fully coalesced 16-byte-per-lane load straight into registers.  (The vector memory pipeline issues about one wave-wide load
// per ~20 clocks per CU whatever its width, so 16-byte loads double the operand bandwidth
// of 8-byte ones.)  The K loop walks 128-deep k blocks through a 2-deep register ring:
// the loads of block kb + 1 are issued before block kb is multiplied, and a 4-byte-per-
// lane touch warms the L2 with the weights PF blocks ahead.  There is no LDS traffic and
// no barrier in the loop: the waves of a workgroup share their A fragments through the
// L1/L2 caches only.  (A variant staging A through a double-buffered LDS tile measured
// slower: the per-stage barrier stalls the MFMA pipe more than the shared loads save.)
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
// Epilogue modes: fp16 with scales, int32 split-K partials, raw int32 accumulators, and
// paired gate/up tiles finished as fp16(gelu_tanh(gate) * up).

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kHiNib = 0xF0F0F0F0u;

__device__ __forceinline__ v4i unpack16(uint2 w) {
  v4i r;
  r[0] = static_cast<int>((w.x << 4) & kHiNib);
  r[1] = static_cast<int>(w.x & kHiNib);
  r[2] = static_cast<int>((w.y << 4) & kHiNib);
  r[3] = static_cast<int>(w.y & kHiNib);
  return r;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3)))
  const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
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

template <int MI, int NI, int KW, bool GELU, int PF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_w4a4_kernel(const GemmParams p) {
  static_assert(!GELU || (NI % 2 == 0), "GELU pairing needs an even NI");
  static_assert(KW == 1 || KW == 2 || KW == 4, "4 waves split as NW x KW");
  constexpr int NW = 4 / KW;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform values are kept in scalar registers: fragment base addresses are scalar
  // and every load of a k block shares one 32-bit lane offset.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % NW;  // column block of the wave
  const int wk = wave / NW;  // k part of the wave

  // ---- tile of this workgroup (XCD-aware order, see the header)
  int tile = blockIdx.x;
  {
    const int total = p.ntiles * p.mtiles;
    if ((total & 7) == 0) tile = (tile & 7) * (total >> 3) + (tile >> 3);
  }
  const int mt = tile % p.mtiles;
  const int nt = tile / p.mtiles;
  const int ks = blockIdx.y;

  // Group selection with scalar selects (no dynamic indexing of the argument struct).
  const int32_t* W = p.g[0].w;
  void* Y = p.g[0].y;
  int N = p.g[0].n;
  int tile_begin = 0;
  int col_off = 0;
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
      }
      if (i < p.ngroups) acc_off += p.g[i].n;
    }
  }

  const int K = p.k;
  const int KB128 = kblocks128(K);
  const int64_t scale_off = static_cast<int64_t>(KB128) * 16;  // words per weight column
  const int64_t M = p.m;
  const int64_t m0 = static_cast<int64_t>(mt) * (16 * MI);
  // First output column of this wave (within the group).  In GELU mode a wave covers
  // 8*NI gate columns and the same up columns.
  const int wcol = GELU ? (nt * (8 * NI * NW) + wn * (8 * NI))
                        : ((nt - tile_begin) * (16 * NI * NW) + wn * (16 * NI));

  // Fragment base pointers.  Row blocks past M and column blocks past N are clamped to
  // the last valid block; their accumulators are never stored.
  const int nb_last = (N >> 4) - 1;
  const int32_t* bptr[NI];
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
    bptr[ni] = base + static_cast<int64_t>(nb) * KB128 * 256;
  }
  const int32_t* aptr[MI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int mb = min(mt * MI + mi, p.mblocks - 1);
    aptr[mi] = p.q + static_cast<int64_t>(mb) * KB128 * 256;
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

  v4i acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4i{0, 0, 0, 0};

  // ---- main loop: A and B straight from global memory into a 2-deep register ring.
  constexpr int RING = 2;
  uint4 ra[RING][MI];
  uint4 rb[RING][NI];
  auto load = [&](int kb, uint4 (&a)[MI], uint4 (&b)[NI]) {
    const int off = min(kb, kb_end - 1) * 256 + lane * 4;  // < 2^31: one fragment column
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) a[mi] = *reinterpret_cast<const uint4*>(aptr[mi] + off);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) b[ni] = *reinterpret_cast<const uint4*>(bptr[ni] + off);
  };
  // The two MFMAs of a 128-deep block (codes 0-15 and 16-31 of each lane's 32).  Pad
  // codes of a K that is not a multiple of 128 are zero in the weights: no guard.
  auto compute = [&](const uint4 (&a)[MI], const uint4 (&b)[NI]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i bop[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bop[ni] = unpack16(h ? make_uint2(b[ni].z, b[ni].w) : make_uint2(b[ni].x, b[ni].y));
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const v4i aop = unpack16(h ? make_uint2(a[mi].z, a[mi].w) : make_uint2(a[mi].x, a[mi].y));
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop[ni], acc[mi][ni], 0, 0, 0);
      }
    }
  };
  // L2 warm-up of the weights PF blocks ahead.  The register ring holds only one block
  // in flight, which hides an L2 hit but not an HBM miss; the m-tiles that share a column
  // block all wait on the same miss.  One 4-byte load per lane and block touches every
  // 128-byte line of the wave's NI weight fragments PF blocks ahead (lane l: fragment
  // (l/8) % NI, line l % 8), so the ring's own loads find the lines in L2.  The touched
  // words are folded into a sink that is only read after the loop.
  const int32_t* tptr = bptr[0];
#pragma unroll
  for (int ni = 1; ni < NI; ++ni)
    if (((lane >> 3) % NI) == ni) tptr = bptr[ni];
  tptr += (lane & 7) * 32;
  int tring[PF > 0 ? PF : 1];
  int tsink = 0;
  constexpr int UNROLL = (PF == 3) ? 6 : ((PF == 4) ? 4 : 2);  // lcm(RING, PF)
  if (nkb > 0) {
    if constexpr (PF > 0) {
#pragma unroll
      for (int j = 0; j < PF; ++j) tring[j] = tptr[min(kb_begin + j, kb_end - 1) * 256];
    }
    load(kb_begin, ra[0], rb[0]);
    int i = 0;
    for (; i + UNROLL <= nkb; i += UNROLL) {
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const int cur = j % RING;
        const int nxt = (j + 1) % RING;
        load(kb_begin + i + j + 1, ra[nxt], rb[nxt]);
        if constexpr (PF > 0) {
          tsink ^= tring[j % PF];
          tring[j % PF] = tptr[min(kb_begin + i + j + PF, kb_end - 1) * 256];
        }
        // Keep the prefetch at the top of the step: under register pressure the
        // scheduler would otherwise sink the loads next to their use.
        __builtin_amdgcn_sched_barrier(0);
        compute(ra[cur], rb[cur]);
      }
    }
    // Remainder (< UNROLL blocks): the ring position continues at slot 0.
#pragma unroll
    for (int j = 0; j < UNROLL - 1; ++j) {
      if (i + j < nkb) {
        const int cur = j % RING;
        const int nxt = (j + 1) % RING;
        load(kb_begin + i + j + 1, ra[nxt], rb[nxt]);
        compute(ra[cur], rb[cur]);
      }
    }
  }
  if constexpr (PF > 0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) tsink ^= tring[j];
    if (tsink == 0x5f3759df && p.m < 0) static_cast<int32_t*>(Y)[0] = tsink;  // never true: m >= 0
  }

  // ---- k-part reduction through LDS (KW > 1): pairs of k parts are folded until part 0
  // of every column block holds the full sum; the other waves are done after that.
  if constexpr (KW > 1) {
    constexpr int FR = MI * NI * 64;  // v4i per wave
    __shared__ __align__(16) v4i red[(KW / 2) * NW * FR];
    auto put = [&](int slot) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) red[(slot * NW + wn) * FR + (mi * NI + ni) * 64 + lane] = acc[mi][ni];
    };
    auto add = [&](int slot) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] += red[(slot * NW + wn) * FR + (mi * NI + ni) * 64 + lane];
    };
    if constexpr (KW == 4) {
      if (wk >= 2) put(wk - 2);
      __syncthreads();
      if (wk < 2) add(wk);
      __syncthreads();
    }
    if (wk == 1) put(0);
    __syncthreads();
    if (wk == 0) add(0);
    if (wk != 0) return;
  }

  // ---- epilogue.  Accumulator element r of fragment (mi, ni) in lane L is
  // C[16*mi + 4*(L/16) + r][16*ni + L%16] of the wave tile.
  const int lcol = lane & 15;
  const int lrow = (lane >> 4) * 4;
  if (p.mode == kEpiFp16 || p.mode == kEpiGeluUp) {
    // fp16 outputs are staged per wave through LDS so that global stores are 16 bytes
    // per lane and every group of lanes writes whole rows of the wave's tile: 128-byte
    // lines for a 64-column tile.  The staging area is private to the wave (no barrier).
    constexpr int OC = GELU ? 8 * NI : 16 * NI;  // output columns of a wave
    constexpr int RB = 2 * OC;                   // bytes of one output row of a wave
    constexpr int LS = RB + 8;                   // LDS row stride (conflict-free b16 writes)
    constexpr int LPR = RB / 16;                 // lanes per row in the write-out
    constexpr int RPI = 64 / LPR;                // rows per write-out instruction
    static_assert(RB % 16 == 0, "a wave's output row must be a multiple of 16 bytes");
    __shared__ __align__(16) unsigned char stage_all[NW * 16 * LS];
    unsigned char* stage = stage_all + wn * (16 * LS);
    float sw[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = GELU ? (wcol + (ni % (NI / 2)) * 16 + lcol) : (wcol + ni * 16 + lcol);
      const int32_t* scales = ((GELU && ni >= NI / 2) ? W2 : W) + N * scale_off;
      sw[ni] = bvalid[ni] ? __int_as_float(scales[col]) : 0.0f;
    }
    // All row scales of the lane are fetched before the first store (the compiler cannot
    // hoist them across the output stores itself).  They are pre-multiplied by 1/256,
    // which folds the accumulator's 2^8 factor into the scale: float(256 t) * (sa / 256)
    // rounds exactly like float(t) * sa (both rescalings are exact powers of two and t
    // is below 2^24), so the fp16 results are unchanged.
    float sav[MI][4];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sav[mi][r] = p.sa[min(m0 + mi * 16 + lrow + r, M - 1)] * 0.00390625f;
    _Float16* y = static_cast<_Float16*>(Y);
    const int out_lane_col = (lane % LPR) * 8;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        _Float16* srow = reinterpret_cast<_Float16*>(stage + (lrow + r) * LS) + lcol;
        if (GELU) {
#pragma unroll
          for (int ni = 0; ni < NI / 2; ++ni) {
            const float g = static_cast<float>(dequant(acc[mi][ni][r], sav[mi][r], sw[ni]));
            const float u = static_cast<float>(dequant(acc[mi][ni + NI / 2][r], sav[mi][r], sw[ni + NI / 2]));
            srow[ni * 16] = static_cast<_Float16>(gelu_tanh(g) * u);
          }
        } else {
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) srow[ni * 16] = dequant(acc[mi][ni][r], sav[mi][r], sw[ni]);
        }
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < (16 + RPI - 1) / RPI; ++j) {
        const int rr = j * RPI + lane / LPR;
        const int64_t grow = m0 + mi * 16 + rr;
        const int gcol = wcol + out_lane_col;
        if (rr < 16 && grow < M && gcol < N) {
          const uint4 v = *reinterpret_cast<const uint4*>(stage + rr * LS + (lane % LPR) * 16);
          *reinterpret_cast<uint4*>(y + grow * N + gcol) = v;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else {
    // kEpiPartial: int32 [ksplit, M, n_total] at column col_off + col;
    // kEpiAcc:     int32 [M, N] in the group's output.
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
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + mi * 16 + lrow + r;
        if (row >= M) continue;
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          if (!bvalid[ni]) continue;
          int col;
          if (GELU) {
            // partial columns: gate block [0, N), up block [N, 2N)
            col = wcol + (ni % (NI / 2)) * 16 + lcol + ((ni >= NI / 2) ? N : 0);
          } else {
            col = wcol + ni * 16 + lcol;
          }
          out[row * ld + col] = acc[mi][ni][r] >> 8;
        }
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
  const float sav = p.sa[row];
  if (GELU) {
    const int N = p.gelu_pair_n;
    int4 g = make_int4(0, 0, 0, 0), u = make_int4(0, 0, 0, 0);
    for (int ks = 0; ks < p.ksplit; ++ks) {
      const int32_t* base = p.partial + ks * plane + row * p.n_total;
      const int4 a = *reinterpret_cast<const int4*>(base + c);
      const int4 b = *reinterpret_cast<const int4*>(base + N + c);
      g.x += a.x; g.y += a.y; g.z += a.z; g.w += a.w;
      u.x += b.x; u.y += b.y; u.z += b.z; u.w += b.w;
    }
    const float* swg = reinterpret_cast<const float*>(p.g[0].w + N * scale_off);
    const float* swu = reinterpret_cast<const float*>(p.g[1].w + N * scale_off);
    const int gv[4] = {g.x, g.y, g.z, g.w};
    const int uv[4] = {u.x, u.y, u.z, u.w};
    _Float16* y = static_cast<_Float16*>(p.g[0].y) + row * N + c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float gf = static_cast<float>(dequant(gv[e], sav, swg[c + e]));
      const float uf = static_cast<float>(dequant(uv[e], sav, swu[c + e]));
      y[e] = static_cast<_Float16>(gelu_tanh(gf) * uf);
    }
    return;
  }
  int4 s = make_int4(0, 0, 0, 0);
  for (int ks = 0; ks < p.ksplit; ++ks) {
    const int4 a = *reinterpret_cast<const int4*>(p.partial + ks * plane + row * p.n_total + c);
    s.x += a.x; s.y += a.y; s.z += a.z; s.w += a.w;
  }
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
  const int sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = dequant(sv[e], sav, sw[col + e]);
}

template <int MI, int NI, int KW, int PF = 3>
hipError_t launch_cfg(const GemmParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.ntiles) * static_cast<unsigned>(p.mtiles),
                  static_cast<unsigned>(p.ksplit));
  if (p.mode == kEpiGeluUp || (p.mode == kEpiPartial && p.gelu_pair_n > 0))
    gemm_w4a4_kernel<MI, NI, KW, true, PF><<<grid, 256, 0, stream>>>(p);
  else
    gemm_w4a4_kernel<MI, NI, KW, false, PF><<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(GemmParams p, int tile_cfg, hipStream_t stream) {
  switch (tile_cfg) {
    case kCfg7x4: return launch_cfg<7, 4, 1>(p, stream);
    case kCfg7x4K4: return launch_cfg<7, 4, 4>(p, stream);
    case kCfg7x2: return launch_cfg<7, 2, 1>(p, stream);
    case kCfg4x2: return launch_cfg<4, 2, 1>(p, stream);
    case kCfg2x2: return launch_cfg<2, 2, 1>(p, stream);
    case kCfg1x2: return launch_cfg<1, 2, 1>(p, stream);
    default: return hipErrorInvalidValue;
  }
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
