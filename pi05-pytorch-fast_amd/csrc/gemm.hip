// W4A4 GEMM for gfx950: int4 codes unpacked to int8 in registers, CDNA4 int8 MFMA
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
// Tiling.  A workgroup is 4 waves side by side along N.  A wave owns a (16*MI) x (16*NI)
// tile = MI x NI accumulators of 16x16.  Per 128-deep K stage:
//   A tile (16*MI rows x 64 bytes of codes) goes global -> registers -> LDS (double
//   buffered, one barrier per stage); every wave reads all MI row fragments from LDS;
//   B fragments are private to a wave and are loaded straight from the fragment-major
//   layout into registers one stage ahead.
// Epilogue modes: fp16 with scales, int32 split-K partials, raw int32 accumulators, and
// paired gate/up tiles finished as fp16(gelu_tanh(gate) * up).

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kLdsStride = 20;  // words per A row in LDS (16 + 4 pad: conflict-free b64 reads)
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

template <int MI, int NI, bool GELU>
__global__ __launch_bounds__(256) void gemm_w4a4_kernel(const GemmParams p) {
  constexpr int BM = 16 * MI;
  constexpr int WN = 16 * NI;                 // columns per wave (GELU: 8*NI gate + 8*NI up)
  constexpr int A_CHUNKS = BM * 4;            // 16-byte chunks per stage
  constexpr int A_PASSES = (A_CHUNKS + 255) / 256;
  static_assert(!GELU || (NI % 2 == 0), "GELU pairing needs an even NI");
  __shared__ __align__(16) int32_t As[2][BM * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nt = blockIdx.x;
  const int mt = blockIdx.y;
  const int ks = blockIdx.z;

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
  const int KW = K >> 3;
  const int KB64 = K >> 6;
  const int64_t M = p.m;
  const int64_t m0 = static_cast<int64_t>(mt) * BM;
  // First output column of this wave (within the group).  In GELU mode a tile covers
  // 32*NI gate columns and the same up columns; each wave owns 8*NI of them.
  const int wcol = GELU ? (nt * (32 * NI) + wave * (8 * NI)) : ((nt - tile_begin) * (64 * NI) + wave * WN);

  // Per-fragment B base pointers (fragment (nb, kb) is 128 words).
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
    const int nb = bvalid[ni] ? (col >> 4) : 0;
    bptr[ni] = base + static_cast<int64_t>(nb) * KB64 * 128 + lane * 2;
  }

  const int nstages = (K + 127) >> 7;
  const int s_begin = ks * p.kstages_per_split;
  const int s_end = min(s_begin + p.kstages_per_split, nstages);

  v4i acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4i{0, 0, 0, 0};

  int4 ra[A_PASSES];
  uint2 rb[NI][2], rbn[NI][2];

  auto load_a = [&](int s) {
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) {
      const int c = tid + 256 * i;
      const int r = c >> 2;
      const int kw = s * 16 + (c & 3) * 4;
      const int64_t grow = m0 + r;
      int4 v = make_int4(0, 0, 0, 0);
      if (c < A_CHUNKS && grow < M && kw < KW)
        v = *reinterpret_cast<const int4*>(p.q + grow * KW + kw);
      ra[i] = v;
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) {
      const int c = tid + 256 * i;
      if (c < A_CHUNKS)
        *reinterpret_cast<int4*>(&As[buf][(c >> 2) * kLdsStride + (c & 3) * 4]) = ra[i];
    }
  };
  auto load_b = [&](int s, uint2 (&dst)[NI][2]) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kb = 2 * s + h;
        uint2 v = make_uint2(0u, 0u);
        if (bvalid[ni] && kb < KB64)
          v = *reinterpret_cast<const uint2*>(bptr[ni] + static_cast<int64_t>(kb) * 128);
        dst[ni][h] = v;
      }
  };

  if (s_begin < s_end) {
    load_a(s_begin);
    load_b(s_begin, rb);
    store_a(0);
  }
  __syncthreads();

  for (int s = s_begin; s < s_end; ++s) {
    const int buf = (s - s_begin) & 1;
    const bool has_next = (s + 1) < s_end;
    if (has_next) {
      load_a(s + 1);
      load_b(s + 1, rbn);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (2 * s + h < KB64) {
        v4i bop[NI];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) bop[ni] = unpack16(rb[ni][h]);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const uint2 aw = *reinterpret_cast<const uint2*>(
              &As[buf][(mi * 16 + (lane & 15)) * kLdsStride + h * 8 + (lane >> 4) * 2]);
          const v4i aop = unpack16(aw);
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop[ni], acc[mi][ni], 0, 0, 0);
        }
      }
    }
    if (has_next) store_a(buf ^ 1);
    __syncthreads();
    if (has_next) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        rb[ni][0] = rbn[ni][0];
        rb[ni][1] = rbn[ni][1];
      }
    }
  }

  // ---- epilogue.  Accumulator element r of fragment (mi, ni) in lane L is
  // C[16*mi + 4*(L/16) + r][16*ni + L%16] of the wave tile.
  const int lcol = lane & 15;
  const int lrow = (lane >> 4) * 4;
  if (p.mode == kEpiFp16 || p.mode == kEpiGeluUp) {
    float sw[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = GELU ? (wcol + (ni % (NI / 2)) * 16 + lcol) : (wcol + ni * 16 + lcol);
      const int32_t* scales = (GELU && ni >= NI / 2) ? (W2 + static_cast<int64_t>(N) * KW)
                                                       : (W + static_cast<int64_t>(N) * KW);
      sw[ni] = bvalid[ni] ? __int_as_float(scales[col]) : 0.0f;
    }
    _Float16* y = static_cast<_Float16*>(Y);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + mi * 16 + lrow + r;
        if (row >= M) continue;
        const float sav = p.sa[row];
        if (GELU) {
#pragma unroll
          for (int ni = 0; ni < NI / 2; ++ni) {
            if (!bvalid[ni]) continue;
            const float g = static_cast<float>(dequant(acc[mi][ni][r] >> 8, sav, sw[ni]));
            const float u = static_cast<float>(dequant(acc[mi][ni + NI / 2][r] >> 8, sav, sw[ni + NI / 2]));
            y[row * N + wcol + ni * 16 + lcol] = static_cast<_Float16>(gelu_tanh(g) * u);
          }
        } else {
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) {
            if (!bvalid[ni]) continue;
            y[row * N + wcol + ni * 16 + lcol] = dequant(acc[mi][ni][r] >> 8, sav, sw[ni]);
          }
        }
      }
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
  const int KW = p.k >> 3;
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
    const float* swg = reinterpret_cast<const float*>(p.g[0].w + static_cast<int64_t>(N) * KW);
    const float* swu = reinterpret_cast<const float*>(p.g[1].w + static_cast<int64_t>(N) * KW);
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
  const float* sw = reinterpret_cast<const float*>(W + static_cast<int64_t>(N) * KW);
  _Float16* y = static_cast<_Float16*>(Y) + row * N + col;
  const int sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = dequant(sv[e], sav, sw[col + e]);
}

template <int MI, int NI>
hipError_t launch_cfg(const GemmParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.ntiles), static_cast<unsigned>(p.mtiles),
                  static_cast<unsigned>(p.ksplit));
  if (p.mode == kEpiGeluUp || (p.mode == kEpiPartial && p.gelu_pair_n > 0))
    gemm_w4a4_kernel<MI, NI, true><<<grid, 256, 0, stream>>>(p);
  else
    gemm_w4a4_kernel<MI, NI, false><<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(GemmParams p, int tile_cfg, hipStream_t stream) {
  switch (tile_cfg) {
    case 0: return launch_cfg<7, 4>(p, stream);
    case 1: return launch_cfg<7, 2>(p, stream);
    case 2: return launch_cfg<4, 2>(p, stream);
    case 3: return launch_cfg<2, 2>(p, stream);
    case 4: return launch_cfg<1, 2>(p, stream);
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
