// Prefix attention of the W4A4 prefix LM on gfx950: RoPE + scaled QK^T + additive mask +
// fp32 softmax + PV for grouped-query attention with head_dim 256 (PaliGemma-2B: 8 query
// heads sharing 1 KV head), fp16 in and out.
//
// Reference semantics: the attention between the QKV and o projections of the reference's
// fused attention forward (apply.py:167-188): transformers' apply_rotary_pos_emb
// (modeling_gemma.py) and eager_attention_forward, all in fp16 tensors:
//   q' = fp16(fp16(q * cos) + fp16(rotate_half(q) * sin))       (k' likewise)
//   s  = fp16(fp16(fp16(q' . k') * scaling) + mask)              (fp32 dot, fp16 result)
//   p  = fp16(exp(s - max_row s) / sum_row exp(s - max_row s))   (fp32 softmax)
//   o  = fp16(sum_k p * v)                                        (fp32 sum)
// The RoPE products and sums are computed in fp16 arithmetic, which rounds exactly like
// torch's fp32-opmath fp16 ops (an fp16 x fp16 product is exact in fp32, and the fp32 sum
// of two fp16 values rounds to the same fp16 as the exact sum), so q' and k' are
// bit-identical to the eager ones.  The softmax follows the eager order (the row's exact
// max and sum before the probabilities are rounded to fp16).  Only the order of the fp32
// sums inside the two products and the row sum differs from torch's.
//
// Layout.  With n_rep = H / KVH, the queries of KV head g are viewed as rows
// r = token * n_rep + j (head g * n_rep + j), which is the row-major [tokens, H, 256]
// output of the QKV GEMM read in place.  One workgroup owns 32 consecutive rows (4 tokens
// x 8 heads for PaliGemma) and every key of its KV head:
//   phase 0  each wave loads the 32 query rows as MFMA operands and applies RoPE in
//            registers (the partner of dimension d < 128 is d + 128, held by the same lane);
//   phase 1  S^T = K Q^T with v_mfma_f32_16x16x32_f16, the waves taking 16-key blocks in
//            turn; the fp16 scores (scaled, masked) go to LDS as [32 rows][keys] and each
//            wave keeps its running row maxima;
//   phase 2  the softmax: 8 threads per row take the row max, exp and sum the row in fp32
//            and write the fp16 probabilities back in place;
//   phase 3  O^T = V^T P^T, each wave owning 64 of the 256 output dimensions over all
//            keys: V^T comes from HBM (16-byte loads of 8 keys of one dimension), P^T from
//            LDS.  Each lane ends with 4 consecutive dimensions of one query row.
// K with RoPE applied and V transposed to [256][keys] (zero-padded to a multiple of 64
// keys) are produced once per call by kv_prep_kernel, so that every operand fetch of the
// attention kernel is one 16-byte load per lane.
//
// Bound: each workgroup streams all of K and V (2 x keys x 512 B) through its CU's vector
// memory path, about 64 B per clock, so the kernel is load-bound at roughly
// (keys x 1 KB) / 64 B per clock per workgroup, ~12k clocks at 776 keys.

#include "w4a4_internal.h"

namespace w4a4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kD = kAttnHeadDim;  // 256
constexpr int kRows = 32;         // query rows per workgroup
constexpr int kWaves = 4;

__device__ __forceinline__ half8 ld8(const _Float16* p) { return *reinterpret_cast<const half8*>(p); }
__device__ __forceinline__ void st8(_Float16* p, half8 v) { *reinterpret_cast<half8*>(p) = v; }

// RoPE of the element pairs (d, d + 128), d in [c, c + 8):
//   lo' = lo * cos_lo - hi * sin_lo,  hi' = hi * cos_hi + lo * sin_hi
// each product and the sum rounded to fp16, as torch's
// (x * cos) + (rotate_half(x) * sin) on fp16 tensors.
__device__ __forceinline__ void rope_pair(half8& lo, half8& hi, half8 clo, half8 chi, half8 slo,
                                          half8 shi) {
#pragma clang fp contract(off)
  const half8 a = lo * clo;
  const half8 b = hi * slo;
  const half8 c = hi * chi;
  const half8 e = lo * shi;
  lo = a - b;
  hi = c + e;
}

// ---- K RoPE + V transpose.  Grid (s_pad / 64, KVH, B), 256 threads; tile = 64 tokens.
__global__ __launch_bounds__(256) void kv_prep_kernel(const AttnParams p) {
  const int t0 = blockIdx.x * 64;
  const int g = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x;
  const int S = p.s;
  // K: 64 tokens x 16 chunk pairs (d in [8c, 8c + 8) and d + 128).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int it = tid + 256 * i;
    const int tok = t0 + (it >> 4);
    const int c = (it & 15) * 8;
    if (tok < S) {
      const _Float16* kr = p.k + (b * S + tok) * p.ld_kv + g * kD;
      const _Float16* cr = p.cosb + (b * S + tok) * kD;
      const _Float16* sr = p.sinb + (b * S + tok) * kD;
      half8 lo = ld8(kr + c), hi = ld8(kr + 128 + c);
      rope_pair(lo, hi, ld8(cr + c), ld8(cr + 128 + c), ld8(sr + c), ld8(sr + 128 + c));
      _Float16* o = p.k_rope + ((b * p.kvh + g) * S + tok) * kD;
      st8(o + c, lo);
      st8(o + 128 + c, hi);
    }
  }
  // V: [64 tokens][256] through LDS into v_t[d][t0 .. t0 + 63]; tokens past S are zero.
  __shared__ _Float16 tile[64][kD + 8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int it = tid + 256 * i;
    const int tok = it >> 5;
    const int c = (it & 31) * 8;
    half8 x = {};
    if (t0 + tok < S) x = ld8(p.v + (b * S + t0 + tok) * p.ld_kv + g * kD + c);
    st8(&tile[tok][c], x);
  }
  __syncthreads();
  _Float16* vt = p.v_t + (b * p.kvh + g) * static_cast<int64_t>(kD) * p.s_pad + t0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int it = tid + 256 * i;
    const int d = it >> 3;
    const int c = (it & 7) * 8;
    half8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = tile[c + e][d];
    st8(vt + static_cast<int64_t>(d) * p.s_pad + c, x);
  }
}

// ---- attention.  Grid (ceil(S * n_rep / 32), KVH, B), 256 threads.
// SCH = 8-key chunks per thread in the softmax phase (s_pad <= 64 * SCH).
template <int SCH>
__global__ __launch_bounds__(256) void prefix_attention_kernel(const AttnParams p) {
  extern __shared__ __align__(16) _Float16 sc[];  // [kRows][sld]: scores, then probabilities
  __shared__ float rowmax[kWaves][kRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int g = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int S = p.s;
  const int s_pad = p.s_pad;
  const int sld = s_pad + 8;
  const int n_rep = p.h / p.kvh;
  const int rows = S * n_rep;
  const int row0 = blockIdx.x * kRows;

  // Token and head of this lane's two query rows (row blocks qb = 0, 1); rows past the
  // group are clamped for loading and never stored.
  int tok[2], head[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int r = min(row0 + 16 * qb + lr, rows - 1);
    tok[qb] = r / n_rep;
    head[qb] = g * n_rep + r % n_rep;
  }

  // ---- phase 0: query operands with RoPE.  MFMA operand B of S^T = K Q^T: lane L holds
  // Q[row 16*qb + L%16][32*t + 8*(L/16) + 0..7] for the 8 steps t of the 256-deep dot.
  half8 qop[2][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const _Float16* qr = p.q + (b * S + tok[qb]) * p.ld_q + head[qb] * kD + 8 * lg;
    const _Float16* cr = p.cosb + (b * S + tok[qb]) * kD + 8 * lg;
    const _Float16* sr = p.sinb + (b * S + tok[qb]) * kD + 8 * lg;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      half8 lo = ld8(qr + 32 * t), hi = ld8(qr + 128 + 32 * t);
      rope_pair(lo, hi, ld8(cr + 32 * t), ld8(cr + 128 + 32 * t), ld8(sr + 32 * t),
                ld8(sr + 128 + 32 * t));
      qop[qb][t] = lo;
      qop[qb][t + 4] = hi;
    }
  }

  // ---- phase 1: scores.  Wave w takes the 16-key blocks w, w + 4, ...  MFMA operand A is
  // K[key 16*j + L%16][32*t + 8*(L/16) + 0..7]; the result lane L holds
  // S^T[key 16*j + 4*(L/16) + i][row 16*qb + L%16], i = 0..3.
  const _Float16* kbase = p.k_rope + (b * p.kvh + g) * static_cast<int64_t>(S) * kD + 8 * lg;
  const bool has_mask = p.mask != nullptr;
  // Mask rows (the rows' tokens); without a mask any valid address is read and ignored.
  const _Float16* mrow[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
    mrow[qb] = has_mask ? p.mask + b * p.mask_bs + static_cast<int64_t>(tok[qb]) * p.mask_rs : p.cosb;
  const int mlast = has_mask ? p.mask_len - 4 : 0;  // last 4-aligned mask group

  const int nblk = s_pad / 16;
  const int jlast = w + ((nblk - 1 - w) / kWaves) * kWaves;  // this wave's last block (w < nblk)
  float mx[2] = {-__builtin_inff(), -__builtin_inff()};

  auto load_k = [&](int j, half8 (&kk)[8]) {
    const int key = min(16 * j + lr, S - 1);
    const _Float16* kr = kbase + static_cast<int64_t>(key) * kD;
#pragma unroll
    for (int t = 0; t < 8; ++t) kk[t] = ld8(kr + 32 * t);
  };
  auto scores = [&](const half8 (&kk)[8], int j) {
#pragma clang fp contract(off)
    f4 acc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
    const int k0 = 16 * j + 4 * lg;
    half4 mv[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) mv[qb] = *reinterpret_cast<const half4*>(mrow[qb] + min(k0, mlast));
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        acc[qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[t], qop[qb][t], acc[qb], 0, 0, 0);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      half4 sv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        _Float16 s16 = static_cast<_Float16>(acc[qb][i]);
        s16 = static_cast<_Float16>(static_cast<float>(s16) * p.scaling);
        if (has_mask) s16 = static_cast<_Float16>(static_cast<float>(s16) + static_cast<float>(mv[qb][i]));
        if (k0 + i >= S) s16 = static_cast<_Float16>(-__builtin_inff());
        sv[i] = s16;
        mx[qb] = fmaxf(mx[qb], static_cast<float>(s16));
      }
      *reinterpret_cast<half4*>(&sc[(16 * qb + lr) * sld + k0]) = sv;
    }
  };

  if (w < nblk) {
    half8 ka[8], kb[8];
    load_k(w, ka);
    for (int j = w;; j += 2 * kWaves) {
      load_k(min(j + kWaves, jlast), kb);  // clamped prefetch: always in bounds
      scores(ka, j);
      if (j + kWaves > jlast) break;
      load_k(min(j + 2 * kWaves, jlast), ka);
      scores(kb, j + kWaves);
      if (j + 2 * kWaves > jlast) break;
    }
  }
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    mx[qb] = fmaxf(mx[qb], __shfl_xor(mx[qb], 16, 64));
    mx[qb] = fmaxf(mx[qb], __shfl_xor(mx[qb], 32, 64));
    if (lg == 0) rowmax[w][16 * qb + lr] = mx[qb];
  }
  __syncthreads();

  // ---- phase 2: softmax of row r = tid / 8 by its 8 threads (keys 8*(c + 8*ch) + 0..7).
  {
#pragma clang fp contract(off)
    const int r = tid >> 3;
    const int c = tid & 7;
    float m = rowmax[0][r];
#pragma unroll
    for (int v = 1; v < kWaves; ++v) m = fmaxf(m, rowmax[v][r]);
    const int nch = s_pad / 64;
    float e[SCH][8];
    float l = 0.0f;
#pragma unroll
    for (int ch = 0; ch < SCH; ++ch) {
      if (ch < nch) {
        const half8 sv = *reinterpret_cast<const half8*>(&sc[r * sld + 8 * (c + 8 * ch)]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          e[ch][i] = expf(static_cast<float>(sv[i]) - m);
          l += e[ch][i];
        }
      }
    }
    l += __shfl_xor(l, 1, 64);
    l += __shfl_xor(l, 2, 64);
    l += __shfl_xor(l, 4, 64);
#pragma unroll
    for (int ch = 0; ch < SCH; ++ch) {
      if (ch < nch) {
        half8 pv;
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = static_cast<_Float16>(e[ch][i] / l);
        *reinterpret_cast<half8*>(&sc[r * sld + 8 * (c + 8 * ch)]) = pv;
      }
    }
  }
  __syncthreads();

  // ---- phase 3: O^T = V^T P^T for dimensions 64*w .. 64*w + 63.  Operand A lane L:
  // V^T[d 64*w + 16*db + L%16][keys 32*t + 8*(L/16) + 0..7]; operand B lane L:
  // P[row 16*qb + L%16][the same keys].  Result lane L: O[row 16*qb + L%16][d + 4*(L/16) + i].
  const _Float16* vbase = p.v_t + (b * p.kvh + g) * static_cast<int64_t>(kD) * s_pad +
                          static_cast<int64_t>(64 * w + lr) * s_pad + 8 * lg;
  f4 o[4][2];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db][0] = o[db][1] = f4{0, 0, 0, 0};
  const int nst = s_pad / 32;
  auto load_v = [&](int t, half8 (&va)[4]) {
#pragma unroll
    for (int db = 0; db < 4; ++db) va[db] = ld8(vbase + static_cast<int64_t>(16 * db) * s_pad + 32 * t);
  };
  auto pv_step = [&](const half8 (&va)[4], int t) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const half8 pb = *reinterpret_cast<const half8*>(&sc[(16 * qb + lr) * sld + 32 * t + 8 * lg]);
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[db], pb, o[db][qb], 0, 0, 0);
    }
  };
  {
    half8 va[4], vb[4];
    load_v(0, va);
    for (int t = 0;; t += 2) {
      load_v(min(t + 1, nst - 1), vb);
      pv_step(va, t);
      if (t + 1 >= nst) break;
      load_v(min(t + 2, nst - 1), va);
      pv_step(vb, t + 1);
      if (t + 2 >= nst) break;
    }
  }

#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    if (row0 + 16 * qb + lr >= rows) continue;
    _Float16* orow = p.out + (b * S + tok[qb]) * p.ld_out + head[qb] * kD + 64 * w + 4 * lg;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      half4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = static_cast<_Float16>(o[db][qb][i]);
      *reinterpret_cast<half4*>(orow + 16 * db) = v;
    }
  }
}

}  // namespace

int64_t attn_s_pad(int32_t s) { return (static_cast<int64_t>(s) + 63) / 64 * 64; }

hipError_t launch_attn_kv_prep(const AttnParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.s_pad / 64), static_cast<unsigned>(p.kvh),
                  static_cast<unsigned>(p.b));
  kv_prep_kernel<<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_prefix_attention(const AttnParams& p, hipStream_t stream) {
  const int64_t rows = static_cast<int64_t>(p.s) * (p.h / p.kvh);
  const dim3 grid(static_cast<unsigned>((rows + kRows - 1) / kRows), static_cast<unsigned>(p.kvh),
                  static_cast<unsigned>(p.b));
  const size_t lds = static_cast<size_t>(kRows) * (p.s_pad + 8) * sizeof(_Float16);
  if (p.s_pad <= 256)
    prefix_attention_kernel<4><<<grid, 256, lds, stream>>>(p);
  else if (p.s_pad <= 512)
    prefix_attention_kernel<8><<<grid, 256, lds, stream>>>(p);
  else
    prefix_attention_kernel<16><<<grid, 256, lds, stream>>>(p);
  return hipGetLastError();
}

}  // namespace w4a4
