// Internal declarations shared by the W4A4 HIP translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w4a4 {

// Split-K partial sums are int32 [ksplit, M, N] in the workspace.
constexpr int kMaxGroups = 3;
constexpr int kMaxKSplit = 16;

enum EpilogueMode : int {
  kEpiFp16 = 0,     // y = fp16((acc * sa) * sw)
  kEpiPartial = 1,  // int32 partial sums to the workspace (split-K)
  kEpiAcc = 2,      // raw int32 accumulators to `acc_out`
  kEpiGeluUp = 3,   // paired gate/up tiles -> fp16(gelu_tanh(g) * u)
};

// Cache warming: up to kMaxWarmBuffers device buffers of n16[i] 16-byte words that a
// kernel reads and discards with otherwise idle workgroups, so that the next kernel finds
// them in the memory-side Infinity Cache.
constexpr int kMaxWarmBuffers = 4;
struct CacheWarmParams {
  const void* ptr[kMaxWarmBuffers];
  int64_t n16[kMaxWarmBuffers];
  int32_t nbuf;
};

struct GemmGroup {
  const int32_t* w;  // MFMA-layout payload; fp32 scales at w + N*kblocks128(K)*16, wcorr after them
  void* y;           // fp16 [M, N] output (or int32 for kEpiAcc)
  int32_t n;         // output columns
  int32_t tile_begin;  // first global n-tile index of this group
};

struct GemmParams {
  const int32_t* q;   // activation codes, MFMA-fragment-major (frag_word_index), then qcorr
  const float* sa;    // fp32 [M]
  int64_t m;
  int32_t mblocks;    // ceil(M / 16): 16-row blocks held by q
  int32_t k;
  int32_t ngroups;
  GemmGroup g[kMaxGroups];
  int32_t ntiles;     // total n-tiles over the groups
  int32_t mtiles;
  int32_t ksplit;     // number of K slices
  int32_t kblocks_per_split;  // 128-deep k blocks per K slice
  int32_t mode;
  int32_t* partial;   // workspace for kEpiPartial: [ksplit, M, n_total]
  int32_t n_total;
  int32_t gelu_pair_n;  // for kEpiGeluUp: columns of the gate (= up) weight
  const _Float16* res;  // kEpiFp16, one group: fp16 [M, N] added to the output (or null)
  // Attention prep in the QKV epilogue (kEpiFp16, one KV head of 256): group rope_group - 1
  // is K with its output channels in RoPE-pair order (16-column block 2P + j holds the key
  // dimensions 16P + 128j .. + 15), finished with RoPE into its y (the key states, [M, 256]
  // in dimension order) and into the fragment-major K of kv; group vt_group - 1 is V,
  // written plain and as the fragment-major V^T of kv (the layout of kv_prep_kernel,
  // attention.hip).  0: no such group.  Rows are tokens: row r = b * seq + t.
  int32_t rope_group;
  int32_t vt_group;
  const _Float16* cosb;  // [M, 256] rotary tables of the rows
  const _Float16* sinb;
  _Float16* kv;          // per batch: K then V^T fragments, keys padded to s_pad (zeroed here)
  int32_t seq;           // tokens per batch, a multiple of 8
  int32_t s_pad;         // attn_s_pad(seq)
  // Down-projection quant riding on the paired gate/up GELU launch (gemm_w4a4_kernel with
  // QFUSE): the workgroups past the GEMM tiles rotate and quantize the rows of h (group
  // 0's output, K = gelu_pair_n) into dq / dsa (launch_quantize's layout) as soon as all
  // n-tiles of a row's 16*MI-row block are stored.  qctl: the launch's control block in
  // device memory (layout below), zero before the launch and left zero by it; qstatus: a
  // host-visible word that a bounded wait which ran out sets (or null).
  int32_t* dq;
  float* dsa;
  int32_t* qctl;
  uint32_t* qstatus;
  float dinv_sqrt_k;
  int32_t spin_limit;    // s_sleep rounds a quant workgroup waits for one row block
  int32_t wait_extra;    // completions waited for beyond ntiles (0; tests force timeouts with 1)
  CacheWarmParams warm;  // read by the quant workgroups that find no row left
  // Small-M prologue (launch_gemm_qpro): every workgroup quantizes the M <= kQproMaxRows fp16
  // rows of xpro [M, 2048] itself, after the RMSNorm with weight nwpro when that is not
  // null (eps_pro, unit_offset_pro), into LDS; q and sa are not read.
  const _Float16* xpro;
  const _Float16* nwpro;
  float eps_pro;
  int32_t unit_offset_pro;
  float inv_sqrt_k_pro;
};
constexpr int kQproMaxRows = 4;

// Control block of the fused gate/up + down-quant launch, in 128-byte lines so that the
// polled words do not share one (a hot line slows every memory request near it):
// word 0 the next row to hand out, word 16 the quant workgroups that have left, then the
// tiles-done counter of m-tile i at word kMlpCtlHeader + kMlpCtlStride * i.  The last
// quant workgroup to leave resets it to zero.
constexpr int kMlpCtlExited = 16;
constexpr int kMlpCtlHeader = 32;
constexpr int kMlpCtlStride = 32;

// MFMA-fragment-major layout of packed INT4 codes, shared by the weights (r = output
// column) and the quantized activations (r = row).  The codes of the 16-line block r/16
// and the 128-deep k block kw/16 form one 1 KB fragment of 256 words made of 64 16-byte
// slots, one per lane of a wave: slot L holds codes 32*(L/16) .. +31 of line 16*(r/16) +
// L%16 (its packed words 16*(kw/16) + 4*(L/16) .. +3).  Lane L loads slot L (one fully
// coalesced 16-byte-per-lane load fetches the whole fragment) and feeds codes 0-15 of it
// to one v_mfma_i32_16x16x64_i8 and codes 16-31 to the next, so the two MFMAs of a
// block together cover its 128 codes once.  A and B share this k permutation, which
// leaves the integer dot product unchanged.  A line's 32 consecutive codes are
// contiguous, so the quantizer writes them as whole 16-byte slots.
// K is padded to a multiple of 128; weight pad words are 0.
// Word index of packed word kw (codes 8*kw .. 8*kw+7) of line r, kb128 = ceil(K/128):
__host__ __device__ inline int64_t frag_word_index(int64_t r, int32_t kw, int32_t kb128) {
  return ((r >> 4) * kb128 + (kw >> 4)) * 256 + ((r & 15) + 16 * ((kw & 15) >> 2)) * 4 + (kw & 3);
}

// Nibble encodings.  Byte j of a packed word holds the codes of k = 2j and k = 2j + 1
// (j = 0..3 within the word's 8 codes).  A nibble is either two's complement ("tc", code
// c as c & 15) or offset binary ("ob", c + 8):
//   activations: low nibble = ob(a[2j]),   high nibble = tc(a[2j+1])
//   weights:     high nibble = tc(b[2j]),  low nibble = ob(b[2j+1])
// One AND per int8 word unpacks either operand: w & 0x0F0F0F0F gives bytes c + 8 and
// w & 0xF0F0F0F0 gives bytes 16c, both exact signed int8.  Pairing the activation's
// (a[2j] + 8) with the weight's 16 b[2j], and 16 a[2j+1] with (b[2j+1] + 8), the MFMA
// sums
//   S = 16 * sum_k a[k] b[k] + 128 * sum_{k odd} a[k] + 128 * sum_{k even} b[k]
// exactly in int32 (|S| <= 2048 K).  The last two terms are a row term and a column term,
// stored with the codes as int32 corrections
//   qcorr[m] = -128 * sum_{k odd} a[m, k]      (after the activation fragments)
//   wcorr[n] = -128 * sum_{k even} b[n, k]     (after the weight scales)
// so that S + qcorr[m] + wcorr[n] = 16 * acc[m, n].  Zero weight pad words contribute
// nothing whatever the activation pad holds.
constexpr uint32_t kLoNib = 0x0F0F0F0Fu;
constexpr uint32_t kHiNib = 0xF0F0F0F0u;
constexpr uint32_t kObFlipLo = 0x08080808u;  // tc <-> ob on the low nibbles
constexpr uint32_t kObFlipHi = 0x80808080u;  // tc <-> ob on the high nibbles

// Words of activation codes for M rows (fragments of ceil(M/16) row blocks), followed by
// qcorr for every row of those blocks.
__host__ __device__ inline int64_t q_payload_words(int64_t mblocks, int32_t kb128) {
  return mblocks * 16 * kb128 * 16;
}
__host__ __device__ inline int64_t q_total_words(int64_t mblocks, int32_t kb128) {
  return q_payload_words(mblocks, kb128) + mblocks * 16;
}

__host__ __device__ inline int32_t kblocks128(int32_t k) { return (k + 127) >> 7; }

// E3M2 (bf6) operand layouts, for gfx950's v_mfma_f32_16x16x128_f8f6f4 with both operands
// in the OCP FP6 E3M2 format (sign, 3 exponent bits with bias 3, 2 mantissa bits, no
// inf/NaN).  Every integer in [-8, 8] is an E3M2 value, so INT4 codes travel exactly;
// the MFMA's products are integers of magnitude <= 64 and its fp32 sums stay integers
// below 2^24 for K <= 2^18, so the fp32 accumulator equals the int32 dot product bit for
// bit, in any summation order.  One MFMA covers 16 x 16 x 128 at twice the int8 MFMA's
// rate and needs no unpack: lane L supplies codes 32*(L/16) .. +31 of line L%16 of its
// 128-deep block, code j in bits 6j .. 6j+5 of six dwords d0 .. d5.
//  * Activations (q6): one 1536-byte fragment per 16 rows x 128 k, fragment (mb, kb) at
//    byte (mb * kb128 + kb) * 1536: bytes [0, 1024) hold d0-d3 of lane L at 16 L, bytes
//    [1024, 1536) hold d4-d5 of lane L at 1024 + 8 L.  No row corrections (the codes are
//    signed values); sa as for the INT4 codes.
//  * Weights (w6): columns in pairs; pair p (columns 32p .. 32p+31) and k block kb form
//    3072 bytes at (p * kb128 + kb) * 3072, three 1 KB chunks: chunk c holds bytes
//    16c .. 16c+15 of each lane's 48-byte record [d0..d5 of column 32p + L%16 | d0..d5 of
//    column 32p + 16 + L%16] at 16 L.  Three 16-byte loads per lane fetch both fragments
//    with each fragment's six dwords in consecutive registers.  The fp32 column scales
//    follow the payload (N * kb128 * 24 words); the tensor is int32 [N, 3K/16 + 16].
constexpr int kE3m2FragBytes = 1536;
constexpr int kE3m2PairBytes = 3072;
__host__ __device__ inline int64_t q6_bytes(int64_t mblocks, int32_t kb128) {
  return mblocks * kb128 * kE3m2FragBytes;
}
__host__ __device__ inline int64_t w6_payload_words(int64_t n, int32_t kb128) { return n * kb128 * 24; }

// GEMM tile configurations: wave tile (16*MI) x (16*NI); K4 / K8 = the 4 / 8 waves of
// a workgroup split K (one column block per workgroup) instead of N.
enum TileCfg : int {
  kCfg7x4 = 0,    // MI 7, NI 4, 4 waves along N: workgroup tile 112 x 256
  kCfg7x2 = 1,    // MI 7, NI 2, 4 waves along N: 112 x 128
  kCfg4x2 = 2,    // MI 4, NI 2: 64 x 128
  kCfg2x2 = 3,    // MI 2, NI 2: 32 x 128
  kCfg1x2 = 4,    // MI 1, NI 2: 16 x 128
  kCfg7x4K4 = 5,  // MI 7, NI 4, 4 waves along K: 112 x 64
  kCfg7x4K8 = 6,  // MI 7, NI 4, 8 waves along K (2 per SIMD): 112 x 64, for very long K
  // Small M (weight streaming): 4 waves split K, 32-column tiles (GELU: 16 gate + 16 up).
  kCfg1x2K4 = 7,  // MI 1: 16 x 32
  kCfg2x2K4 = 8,  // MI 2: 32 x 32
  kCfg4x2K4 = 9,  // MI 4: 64 x 32
  // Mid-size M (the QKV + RoPE and o GEMMs at hundreds of rows): 4 waves split K of a
  // 64 x 64 tile, so that each operand byte of the tile is loaded once per workgroup.
  kCfg4x4K4 = 10,  // MI 4, NI 4: 64 x 64
};


// Prefix attention (attention.hip): head_dim 256, grouped-query heads, fp16.
constexpr int kAttnHeadDim = 256;
constexpr int kAttnMaxKeys = 1024;
struct AttnParams {
  const _Float16* q;      // [B, S, H, 256], token stride ld_q (elements)
  int64_t ld_q;
  const _Float16* k;      // [B, S, KVH, 256] before RoPE, token stride ld_kv
  const _Float16* v;      // [B, S, KVH, 256], token stride ld_kv
  int64_t ld_kv;
  const _Float16* cosb;   // [B, S, 256]
  const _Float16* sinb;   // [B, S, 256]
  const _Float16* mask;   // additive, element (b, sq, sk) at b*mask_bs + sq*mask_rs + sk; or null
  int64_t mask_bs;
  int64_t mask_rs;
  int32_t mask_len;       // keys per mask row (>= S, multiple of 4)
  float scaling;
  int32_t b, s, h, kvh;
  int32_t s_pad;          // keys rounded up to a multiple of 64
  _Float16* k_rope;       // [B, KVH, S, 256] with RoPE
  _Float16* kv_mfma;      // per (b, KV head): K then V^T in MFMA-fragment-major order
  _Float16* out;          // [B, S, H, 256], token stride ld_out (or null)
  int64_t ld_out;
  int32_t* qcodes;        // KVH == 1, H == 8: the output rows' K = 2048 quant (or null):
  float* qscales;         //   codes, scales and row corrections as pi05w4a4_quantize writes
  int32_t* qcorr;         //   them for M = B * S rows
  float inv_sqrt_k;
  int32_t row_blocks;     // set by the launcher: workgroups along x that own query rows
  CacheWarmParams warm;   // read by the workgroups past row_blocks (nbuf 0: none)
};
int64_t attn_s_pad(int32_t s);

// Compute units of the current device (hipDeviceAttributeMultiprocessorCount, queried
// once per device and cached; 256 on a whole MI355X, fewer on a partitioned one).  The
// tile planner, the cache-warming launches and the attention grid size their work by it.
int device_cu_count();

// Launchers (return hipError_t of the launch).
hipError_t launch_quantize(const void* x, int64_t m, int32_t k, int32_t* q, float* sa,
                           float inv_sqrt_k, hipStream_t stream, const CacheWarmParams* warm = nullptr);
hipError_t launch_repack(const int32_t* src, int32_t layout, int32_t n, int32_t k,
                         int64_t src_stride, int32_t* dst, hipStream_t stream);
// INT4 MFMA-layout weight (N % 32 == 0, K % 128 == 0) -> the E3M2 pair layout w6.
hipError_t launch_repack_e3m2(const int32_t* w_mfma, int32_t n, int32_t k, int32_t* dst, hipStream_t stream);
// K = 2048 activation quant (optionally with the fused RMSNorm, nw != null) writing E3M2
// fragments (q6) instead of INT4 codes.
hipError_t launch_quantize_e3m2(const void* x, const void* nw, float eps, int unit_offset, int64_t m,
                                int32_t k, void* q6, float* sa, float inv_sqrt_k, hipStream_t stream,
                                const CacheWarmParams* warm = nullptr);
// GEMM on E3M2 operands, tile_cfg kCfg7x4 (112 x 256 workgroup tiles, GELU pairs or
// plain) or kCfg2x2 (32 x 128), four waves along N, no K split; modes kEpiFp16 (1..3
// groups, optional residual or QKV attention prep) and kEpiGeluUp; p.q points at q6, the
// groups' w at w6.
hipError_t launch_gemm_e3m2(const GemmParams& p, int tile_cfg, hipStream_t stream);
// 16 x 32 tiles whose four waves split K (K = 2048, 1 <= M <= kQproMaxRows, one K slice,
// fp16 epilogue without the attention prep), the activation quant of p.xpro in every
// workgroup's prologue.
hipError_t launch_gemm_qpro(const GemmParams& p, hipStream_t stream);
// Chooses the tile configuration; returns the K split used (>= 1) through *ksplit_out.
hipError_t launch_gemm(GemmParams p, int tile_cfg, hipStream_t stream);
// The paired gate/up GELU GEMM (7x4 tiles, no K split) with the down-projection quant of
// its output in the same launch (p.dq .. p.warm set; nquant extra workgroups).
hipError_t launch_gemm_gelu_quant(const GemmParams& p, int nquant, hipStream_t stream);
hipError_t launch_splitk_reduce(const GemmParams& p, hipStream_t stream);
// y = fp16(gelu_tanh(g) * u) elementwise on n fp16 values (n >= 1).
hipError_t launch_gelu_up(const void* g, const void* u, int64_t n, void* y, hipStream_t stream);
hipError_t launch_rmsnorm(const void* x, const void* w, float eps, int unit_offset, int64_t m,
                          int32_t k, void* y, hipStream_t stream);
// RMSNorm fused into the K = 2048 activation quant (hipErrorInvalidValue for other K).
// With warm buffers, workgroups appended for the CUs that the rows leave idle read them.
hipError_t launch_rmsnorm_quantize(const void* x, const void* w, float eps, int unit_offset,
                                  int64_t m, int32_t k, int32_t* q, float* sa, float inv_sqrt_k,
                                  hipStream_t stream, const CacheWarmParams* warm = nullptr);
hipError_t launch_attn_kv_prep(const AttnParams& p, hipStream_t stream);
hipError_t launch_prefix_attention(const AttnParams& p, hipStream_t stream);

}  // namespace w4a4
