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
// max and sum before the probabilities are rounded to fp16); it evaluates exp with the
// hardware exp2 and divides through one reciprocal per row, and the fp32 sums inside the
// two products and the row sum run in another order than torch's, so the output agrees
// with the eager one to fp16 rounding, not bit for bit.
//
// Layout.  With n_rep = H / KVH, the queries of KV head g are viewed as rows
// r = token * n_rep + j (head g * n_rep + j), which is the row-major [tokens, H, 256]
// output of the QKV GEMM read in place.  kv_prep_kernel writes, once per call, K with
// RoPE (the key states, [B, KVH, S, 256]) and an MFMA-fragment-major copy of K and of V^T
// (keys zero-padded to s_pad, a multiple of 64): a 1 KB fragment holds the 64 lanes'
// 16-byte operands of one MFMA, so every operand fetch below is one contiguous 1 KB
// wave load.  K fragment (j, t): lane L = K[16j + L%16][32t + 8(L/16) + 0..7];
// V^T fragment (db, t): lane L = V[32t + 8(L/16) + 0..7][16db + L%16].
// One workgroup (8 waves) owns 32 consecutive rows (4 tokens x 8 heads for PaliGemma)
// and every key of its KV head:
//   phase 0  the 32 query rows are loaded once, RoPE'd and stored to LDS; each wave then
//            reads them as MFMA operands;
//   phase 1  S^T = K Q^T with v_mfma_f32_16x16x32_f16, the waves taking 16-key blocks in
//            turn; fp16(fp16(q.k) * scaling) goes to LDS as [32 rows][keys];
//   phase 2  16 threads per row add the mask in fp16, take the row max, exp and sum in
//            fp32 and write the fp16 probabilities back in place;
//   phase 3  O^T = V^T P^T, each wave owning 32 of the 256 output dimensions over all
//            keys (V^T fragments from HBM, P from LDS).  Each lane ends with 4
//            consecutive dimensions of one query row.
// The memory phases are kept fed ahead of time: the first two K blocks of every wave are
// requested in phase 0, and the first 8 V^T steps of its 8-deep ring during the softmax.
//
// Bound: each workgroup streams all of K and V (2 x keys x 512 B) through its CU's vector
// memory path, about 64 B per clock, ~13k clocks at 776 keys; the softmax is VALU work
// (a wave64 VALU instruction occupies its SIMD for 4 clocks).  Measured inside the
// 776-token forward (per-workgroup timestamps, medians): query load + RoPE 3.8 us,
// scores 4.4, softmax 3.0, PV 3.9, o-proj quant 3.5 (mostly the codes' store latency).

#include "cache_warm.h"
#include "quant_row.h"

namespace w4a4 {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kD = kAttnHeadDim;  // 256
constexpr int kRows = 32;           // query rows per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kQld = kD + 8;        // LDS row stride of the query tile (halves)
constexpr int kOld = 2048 + 8;      // LDS row stride of the output rows quantized in phase 4

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

// ---- K RoPE + V transpose.  Grid (s_pad / 16, KVH, B), 256 threads; tile = 16 tokens.
__global__ __launch_bounds__(256) void kv_prep_kernel(const AttnParams p) {
  const int t0 = blockIdx.x * 16;
  const int g = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x;
  const int S = p.s;
  _Float16* kf = p.kv_mfma + (b * p.kvh + g) * 2 * static_cast<int64_t>(p.s_pad) * kD;
  _Float16* vf = kf + static_cast<int64_t>(p.s_pad) * kD;
  // The V tile's loads are issued first, so that their latency overlaps the K part's
  // (the compiler cannot move them above the K stores, which might alias).
  half8 vx[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int it = tid + 256 * i;
    const int tok = it >> 5;
    const int c = (it & 31) * 8;
    vx[i] = half8{};
    if (t0 + tok < S) vx[i] = ld8(p.v + (b * S + t0 + tok) * p.ld_kv + g * kD + c);
  }
  // K: 16 tokens x 16 chunk pairs (d in [c, c + 8) and d + 128), one per thread.  The
  // RoPE'd row goes to k_rope and, as the 16-key block u of the fragment-major copy, to
  // lane (token % 16) + 16 * ((d % 32) / 8) of fragment (u, d / 32).  Tokens past S are zero.
  {
    const int tl = tid >> 4;
    const int tok = t0 + tl;
    const int c = (tid & 15) * 8;
    half8 lo = {}, hi = {};
    if (tok < S) {
      const _Float16* kr = p.k + (b * S + tok) * p.ld_kv + g * kD;
      const _Float16* cr = p.cosb + (b * S + tok) * kD;
      const _Float16* sr = p.sinb + (b * S + tok) * kD;
      lo = ld8(kr + c);
      hi = ld8(kr + 128 + c);
      rope_pair(lo, hi, ld8(cr + c), ld8(cr + 128 + c), ld8(sr + c), ld8(sr + 128 + c));
      _Float16* o = p.k_rope + ((b * p.kvh + g) * S + tok) * kD;
      st8(o + c, lo);
      st8(o + 128 + c, hi);
    }
    const int lane = tl + 16 * ((c & 31) >> 3);
    const int t = c >> 5;
    st8(kf + ((blockIdx.x * 8 + t) * 64 + lane) * 8, lo);
    st8(kf + ((blockIdx.x * 8 + t + 4) * 64 + lane) * 8, hi);
  }
  // V: [16 tokens][256] through LDS into the fragment-major V^T: the tile is half h of the
  // 32-key step u / 2, i.e. lanes 32h .. 32h + 31 of each of its 16 dimension-block
  // fragments.  Tokens past S are zero.
  __shared__ _Float16 tile[16][kD + 8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int it = tid + 256 * i;
    st8(&tile[it >> 5][(it & 31) * 8], vx[i]);
  }
  __syncthreads();
  const int nst = p.s_pad / 32;
  const int step = blockIdx.x >> 1;
  const int h = blockIdx.x & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int it = tid + 256 * i;
    const int db = it >> 5;
    const int l32 = it & 31;
    const int lane = 32 * h + l32;
    const int d = 16 * db + (lane & 15);
    const int k0 = 8 * (l32 >> 4);
    half8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = tile[k0 + e][d];
    st8(vf + ((db * nst + step) * 64 + lane) * 8, x);
  }
}

// ---- attention.  Grid (ceil(S * n_rep / 32) + warm, KVH, B), 512 threads (8 waves).
// SCH = 8-key chunks per thread in the softmax phase (s_pad <= 128 * SCH).
template <int SCH>
__global__ __launch_bounds__(kThreads) void prefix_attention_kernel(const AttnParams p) {
  extern __shared__ __align__(16) _Float16 lds[];
  _Float16* qs = lds;                  // [kRows][kQld]: the tile's queries with RoPE
  _Float16* sc = lds + kRows * kQld;   // [kRows][sld]: scores, then probabilities

  const int tid = threadIdx.x;
  if (static_cast<int>(blockIdx.x) >= p.row_blocks) {  // a cache-warming workgroup
    const int64_t wx = gridDim.x - p.row_blocks;
    cache_warm_part<kThreads>(p.warm, (static_cast<int64_t>(blockIdx.z) * gridDim.y + blockIdx.y) * wx + (blockIdx.x - p.row_blocks),
                    wx * gridDim.y * gridDim.z, tid);
    return;
  }
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

  // Phase 1's K blocks: wave w takes the 16-key blocks w, w + 8, ... through a 3-deep
  // register ring.  MFMA operand A is K[key 16*j + L%16][32*t + 8*(L/16) + 0..7].  Every
  // K (and mask) load is unconditional, with its block clamped into the buffer, so that
  // the compiler's vmcnt waits stay exact (a load under a branch makes every later wait
  // assume the path with fewer loads in flight); a wave without blocks (s_pad < 128)
  // loads one it never uses.
  const int nblk = s_pad / 16;
  const _Float16* kf = p.kv_mfma + (b * p.kvh + g) * 2 * static_cast<int64_t>(s_pad) * kD + 8 * lane;
  const int jlast = w + ((nblk - 1 - w) / kWaves) * kWaves;  // this wave's last block (w < nblk)
  const int jcap = min(jlast, nblk - 1);
  auto load_k = [&](int j, half8 (&kk)[8]) {
    const _Float16* kr = kf + min(j, jcap) * (8 * 512);
#pragma unroll
    for (int t = 0; t < 8; ++t) kk[t] = ld8(kr + 512 * t);
  };
  half8 k0[8], k1[8], k2[8];
  const bool has_mask = p.mask != nullptr;
  uint4 mraw[SCH];  // the softmax phase's mask chunks (raw bits; zeroed there without a mask)

  // ---- phase 0: the 32 query rows with RoPE, once per workgroup, into LDS.  Thread t
  // takes row t / 16 and the element pairs (c, c + 128), c = 8 * (t % 16).  Rows past the
  // group are clamped (loaded, never stored).  After the query rows, the loads of the
  // softmax's mask chunks (thread t: row t / 16, the 8-key chunks 8 * (t % 16 + 16 * ch))
  // and of the wave's first two K blocks are issued, so that their latency overlaps this
  // phase: loads complete in issue order, and the RoPE below waits for the query loads
  // only.
  {
    const int r = tid >> 4;
    const int c = (tid & 15) * 8;
    const int rr = min(row0 + r, rows - 1);
    const int64_t tk = b * S + rr / n_rep;
    const _Float16* qr = p.q + tk * p.ld_q + (g * n_rep + rr % n_rep) * kD;
    const _Float16* cr = p.cosb + tk * kD;
    const _Float16* sr = p.sinb + tk * kD;
    half8 lo = ld8(qr + c), hi = ld8(qr + 128 + c);
    const half8 clo = ld8(cr + c), chi = ld8(cr + 128 + c), slo = ld8(sr + c), shi = ld8(sr + 128 + c);
    // Every wave's query loads reach the CU's memory pipeline before any of the loads
    // below (which would otherwise queue ahead of a slower wave's query rows).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    {
      // Without a mask the loads read the first query elements (the bits are dropped).  The
      // row pointer is a global-address-space one, so that these are global (not flat)
      // loads, which count in vmcnt only.
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      typedef const __attribute__((address_space(1))) u32x2* gptr2;
      const int64_t moff = has_mask ? b * p.mask_bs + static_cast<int64_t>(rr / n_rep) * p.mask_rs : 0;
      const _Float16* mrow = (has_mask ? p.mask : p.q) + moff;
      const int mlast = has_mask ? p.mask_len - 4 : 0;
      const int mc = tid & 15;
#pragma unroll
      for (int ch = 0; ch < SCH; ++ch) {
        const int kc = 8 * (mc + 16 * ch);  // chunks at or past s_pad are never used
        const u32x2 mv0 = *(gptr2)(mrow + min(kc, mlast));
        const u32x2 mv1 = *(gptr2)(mrow + min(kc + 4, mlast));
        mraw[ch] = uint4{mv0.x, mv0.y, mv1.x, mv1.y};
      }
    }
    load_k(w, k0);
    load_k(w + kWaves, k1);
    __builtin_amdgcn_sched_barrier(0);
    rope_pair(lo, hi, clo, chi, slo, shi);
    st8(qs + r * kQld + c, lo);
    st8(qs + r * kQld + 128 + c, hi);
  }
  __syncthreads();

  // MFMA operand B of S^T = K Q^T: lane L holds Q[row 16*qb + L%16][32*t + 8*(L/16) + 0..7].
  half8 qop[2][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int t = 0; t < 8; ++t) qop[qb][t] = ld8(qs + (16 * qb + lr) * kQld + 32 * t + 8 * lg);

  // ---- phase 1: scores, the K ring loading two blocks ahead (the first two were requested
  // in phase 0).  The result lane L holds S^T[key 16*j + 4*(L/16) + i][row 16*qb + L%16],
  // i = 0..3, stored to LDS as fp16(fp16(q.k) * scaling), or -inf for the padding keys
  // past S.  The mask is added in the softmax phase.
  if (w < nblk) {
    auto scores = [&](const half8 (&kk)[8], int j) {
#pragma clang fp contract(off)
      f4 acc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
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
          const _Float16 s16 = static_cast<_Float16>(acc[qb][i]);
          sv[i] = (16 * j + 4 * lg + i < S) ? static_cast<_Float16>(static_cast<float>(s16) * p.scaling)
                                            : static_cast<_Float16>(-__builtin_inff());
        }
        *reinterpret_cast<half4*>(&sc[(16 * qb + lr) * sld + 16 * j + 4 * lg]) = sv;
      }
    };
    for (int j = w;; j += 3 * kWaves) {
      load_k(j + 2 * kWaves, k2);
      scores(k0, j);
      if (j + kWaves > jlast) break;
      load_k(j + 3 * kWaves, k0);
      scores(k1, j + kWaves);
      if (j + 2 * kWaves > jlast) break;
      load_k(j + 4 * kWaves, k1);
      scores(k2, j + 2 * kWaves);
      if (j + 3 * kWaves > jlast) break;
    }
  }
  __syncthreads();

  // Phase 3 streams V^T through a kVR-deep register ring; its first kVR steps are requested
  // during the softmax (spread over its first chunk loop, so that the waves do not stall
  // on a full memory queue before their softmax work), and their latency hides under it.
  // Wave w reads the V^T fragments of dimensions 32*w .. 32*w + 31: operand A lane L:
  // V^T[d 32*w + 16*db + L%16][keys 32*t + 8*(L/16) + 0..7].
  const int nst = s_pad / 32;
  const _Float16* vf = kf + static_cast<int64_t>(s_pad) * kD + (2 * w) * nst * 512;
  auto load_v = [&](int t, half8 (&va)[2]) {
#pragma unroll
    for (int db = 0; db < 2; ++db) va[db] = ld8(vf + (db * nst + t) * 512);
  };
  constexpr int kVR = 8;
  half8 vr[kVR][2];
  static_assert(kVR % SCH == 0 || SCH % kVR == 0, "ring steps spread evenly over the chunks");

  // ---- phase 2: softmax of row r = tid / 16 by its 16 threads, keys 8*(c + 16*ch) + 0..7:
  // s = fp16(score + mask) (padding keys are -inf), the row max (exact, in fp16), then
  // e = exp(s - max) through the hardware exp2 as exp2(s * log2 e - max * log2 e) (one
  // v_fma_mix with the fp16 s; relative error ~1e-6, far below the fp16 rounding of the
  // probabilities), the fp32 sum l, and p = fp16(e * (1 / l)), written back over the
  // scores.
  {
    const int r = tid >> 4;
    const int c = tid & 15;
    half8 sv[SCH];
    half8 mx;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx[i] = static_cast<_Float16>(-__builtin_inff());
#pragma unroll
    for (int ch = 0; ch < SCH; ++ch) {
#pragma unroll
      for (int i = ch * kVR / SCH; i < (ch + 1) * kVR / SCH; ++i) load_v(min(i, nst - 1), vr[i]);
      const int kc = 8 * (c + 16 * ch);
      sv[ch] = mx;
      if (kc < s_pad) {
        // fp16 additions round exactly like torch's fp32-opmath fp16 add.
        const uint32_t keep = has_mask ? 0xffffffffu : 0u;
        const uint4 m4 = {mraw[ch].x & keep, mraw[ch].y & keep, mraw[ch].z & keep, mraw[ch].w & keep};
        sv[ch] = ld8(&sc[r * sld + kc]) + __builtin_bit_cast(half8, m4);
        mx = __builtin_elementwise_max(mx, sv[ch]);
      }
    }
    float m = static_cast<float>(mx[0]);
#pragma unroll
    for (int i = 1; i < 8; ++i) m = fmaxf(m, static_cast<float>(mx[i]));
    // Row max and sum over the 16 lanes of a row (lane xor 1, 2, 4, 8) through DPP.
    m = fmaxf(m, lane_xor_f<0>(m));
    m = fmaxf(m, lane_xor_f<1>(m));
    m = fmaxf(m, lane_xor_f<2>(m));
    m = fmaxf(m, lane_xor_f<3>(m));
    constexpr float kLog2e = 1.4426950408889634f;
    const float ml = m * kLog2e;
    float e[SCH][8];
    float l = 0.0f;
#pragma unroll
    for (int ch = 0; ch < SCH; ++ch) {
      if (8 * (c + 16 * ch) < s_pad) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          e[ch][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(static_cast<float>(sv[ch][i]), kLog2e, -ml));
          l += e[ch][i];
        }
      }
    }
    l += lane_xor_f<0>(l);
    l += lane_xor_f<1>(l);
    l += lane_xor_f<2>(l);
    l += lane_xor_f<3>(l);
    const float rl = 1.0f / l;
#pragma unroll
    for (int ch = 0; ch < SCH; ++ch) {
      const int kc = 8 * (c + 16 * ch);
      if (kc < s_pad) {
        half8 pv;
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = static_cast<_Float16>(e[ch][i] * rl);
        st8(&sc[r * sld + kc], pv);
      }
    }
  }
  __syncthreads();

  // ---- phase 3: O^T = V^T P^T for dimensions 32*w .. 32*w + 31 over all keys.  Operand
  // B lane L: P[row 16*qb + L%16][keys 32*t + 8*(L/16) + 0..7].  Result lane L:
  // O[row 16*qb + L%16][32*w + 16*db + 4*(L/16) + i].  Each step refills its ring slot
  // with the step kVR ahead.  The main loop's loads are unconditional, which keeps the
  // compiler's vmcnt waits exact (one ring slot at a time); the last 2*kVR - 1 steps or
  // fewer run after it, loading only what they still use.
  f4 o[2][2];
#pragma unroll
  for (int db = 0; db < 2; ++db) o[db][0] = o[db][1] = f4{0, 0, 0, 0};
  auto pv_step = [&](const half8 (&va)[2], int t) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const half8 pb = ld8(&sc[(16 * qb + lr) * sld + 32 * t + 8 * lg]);
#pragma unroll
      for (int db = 0; db < 2; ++db)
        o[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[db], pb, o[db][qb], 0, 0, 0);
    }
  };
  int t0 = 0;
  for (; t0 + 2 * kVR <= nst; t0 += kVR) {
#pragma unroll
    for (int j = 0; j < kVR; ++j) {
      pv_step(vr[j], t0 + j);
      load_v(t0 + j + kVR, vr[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < kVR; ++j) {
    if (t0 + j < nst) pv_step(vr[j], t0 + j);
    if (t0 + j + kVR < nst) load_v(t0 + j + kVR, vr[j]);
  }
#pragma unroll
  for (int j = 0; j < kVR; ++j)
    if (t0 + kVR + j < nst) pv_step(vr[j], t0 + kVR + j);

  if (p.out != nullptr) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int rr = row0 + 16 * qb + lr;
      if (rr >= rows) continue;
      _Float16* orow = p.out + (b * S + rr / n_rep) * p.ld_out + (g * n_rep + rr % n_rep) * kD + 32 * w + 4 * lg;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        half4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = static_cast<_Float16>(o[db][qb][i]);
        *reinterpret_cast<half4*>(orow + 16 * db) = v;
      }
    }
  }

  // ---- phase 4 (one KV head of 8 query heads): the workgroup's 32 rows are 4 whole
  // tokens of the o-proj input (8 heads x 256 = 2048), so it quantizes them itself, as the
  // K = 2048 activation quant would: the fp16 rows are staged in LDS over the
  // probabilities and waves 2i, 2i + 1 rotate and quantize token i in registers, 16
  // elements per lane (fwht_quant_row_2wave: the last butterfly stage and the row's max
  // and code sum through LDS, behind the staged rows).
  if (p.qcodes != nullptr) {
    __syncthreads();  // every wave is done reading P
    _Float16* otile = sc;                                   // [4][kOld] fp16
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int r = 16 * qb + lr;  // n_rep == 8: token r / 8, head r % 8
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        half4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = static_cast<_Float16>(o[db][qb][i]);
        *reinterpret_cast<half4*>(otile + (r >> 3) * kOld + (r & 7) * kD + 32 * w + 16 * db + 4 * lg) = v;
      }
    }
    __syncthreads();
    const int tl = w >> 1;  // token of this wave pair
    const int tok = (row0 >> 3) + tl;
    const int t = (w & 1) * 64 + lane;
    float v[16];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const half8 h = ld8(otile + tl * kOld + 16 * t + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * c + e] = static_cast<float>(h[e]);
    }
    float* xch = reinterpret_cast<float*>(otile + 4 * kOld);  // [4][2 * 64 * 16] floats
    float* redf = xch + 4 * 2 * 64 * 16;                       // [4][2]
    int* redi = reinterpret_cast<int*>(redf + 8);              // [4][2]
    // Every wave takes part (the pair synchronises with the workgroup); rows past S are
    // computed from the clamped duplicates staged above and not stored.
    fwht_quant_row_2wave<11>(v, t, xch + tl * 2 * 64 * 16, redf + 2 * tl, redi + 2 * tl, tok < S,
                             b * S + min(tok, S - 1), p.qcodes, p.qscales, p.qcorr, p.inv_sqrt_k);
  }
}

}  // namespace

int64_t attn_s_pad(int32_t s) { return (static_cast<int64_t>(s) + 63) / 64 * 64; }

hipError_t launch_attn_kv_prep(const AttnParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.s_pad / 16), static_cast<unsigned>(p.kvh),
                  static_cast<unsigned>(p.b));
  kv_prep_kernel<<<grid, 256, 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_prefix_attention(const AttnParams& p_in, hipStream_t stream) {
  AttnParams p = p_in;
  const int64_t rows = static_cast<int64_t>(p.s) * (p.h / p.kvh);
  p.row_blocks = static_cast<int32_t>((rows + kRows - 1) / kRows);
  // Cache warming uses the CUs that the attention leaves idle (one workgroup of 8 waves
  // per CU: at ~200 VGPRs a SIMD holds two of its waves, while its ~71 KB of LDS would
  // allow two workgroups): none when the attention alone fills the device's CUs.
  const int64_t kCUs = device_cu_count();
  const int64_t attn_wgs = static_cast<int64_t>(p.row_blocks) * p.kvh * p.b;
  const int64_t warm_x = (p.warm.nbuf > 0 && attn_wgs < kCUs) ? (kCUs - attn_wgs) / (static_cast<int64_t>(p.kvh) * p.b) : 0;
  const dim3 grid(static_cast<unsigned>(p.row_blocks + warm_x), static_cast<unsigned>(p.kvh),
                  static_cast<unsigned>(p.b));
  size_t sc_bytes = static_cast<size_t>(kRows) * (p.s_pad + 8) * sizeof(_Float16);
  if (p.qcodes != nullptr) {
    // the 4 staged fp16 rows, then the quantizer's exchange (4 x 2 x 64 x 16 floats) and
    // its 16 words of reductions
    const size_t q_bytes = 4 * kOld * sizeof(_Float16) + (4 * 2 * 64 * 16 + 16) * sizeof(float);
    if (q_bytes > sc_bytes) sc_bytes = q_bytes;
  }
  const size_t lds = static_cast<size_t>(kRows) * kQld * sizeof(_Float16) + sc_bytes;
  if (p.s_pad <= 256)
    prefix_attention_kernel<2><<<grid, kThreads, lds, stream>>>(p);
  else if (p.s_pad <= 512)
    prefix_attention_kernel<4><<<grid, kThreads, lds, stream>>>(p);
  else
    prefix_attention_kernel<8><<<grid, kThreads, lds, stream>>>(p);
  return hipGetLastError();
}

}  // namespace w4a4
