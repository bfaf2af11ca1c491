// extern "C" entry points of libpi05_w4a4.so (declared in include/pi05_w4a4.h).
//
// Host-side responsibilities mirror the reference's host glue
// (pi05_fast/w4a4/csrc/int4_gemm.cu:479-642): argument validation, the
// quantize-once / GEMM-many fan-out and shape-based kernel dispatch.  Unlike the
// reference, nothing here allocates device memory: the caller passes the outputs,
// the quantized-activation buffers and the split-K workspace.

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/pi05_w4a4.h"
#include "w4a4_internal.h"

namespace w4a4 {

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  const int slot = dev < kMaxDevices ? dev : kMaxDevices - 1;
  int n = cached[slot].load(std::memory_order_relaxed);
  if (n > 0 && dev < kMaxDevices) return n;
  n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;  // no device to ask (host-only callers): a whole MI355X
  if (dev < kMaxDevices) cached[slot].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace w4a4

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return PI05W4A4_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return fail(PI05W4A4_EHIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct TileCfg {
  int id, mi, ni, nwaves, kw;  // kw of the nwaves waves of a workgroup split K
  int cols(bool gelu) const { return (gelu ? 8 : 16) * ni * (nwaves / kw); }  // tile width
};
constexpr TileCfg kCfg7x4{w4a4::kCfg7x4, 7, 4, 4, 1};
constexpr TileCfg kCfg7x4K4{w4a4::kCfg7x4K4, 7, 4, 4, 4};
constexpr TileCfg kCfg7x4K8{w4a4::kCfg7x4K8, 7, 4, 8, 8};
constexpr TileCfg kCfg4x2{w4a4::kCfg4x2, 4, 2, 4, 1};
constexpr TileCfg kCfg2x2{w4a4::kCfg2x2, 2, 2, 4, 1};
constexpr TileCfg kCfg1x2{w4a4::kCfg1x2, 1, 2, 4, 1};
constexpr TileCfg kCfg1x2K4{w4a4::kCfg1x2K4, 1, 2, 4, 4};
constexpr TileCfg kCfg2x2K4{w4a4::kCfg2x2K4, 2, 2, 4, 4};
constexpr TileCfg kCfg4x2K4{w4a4::kCfg4x2K4, 4, 2, 4, 4};
constexpr TileCfg kCfg4x4K4{w4a4::kCfg4x4K4, 4, 4, 4, 4};

struct Plan {
  TileCfg cfg;
  int64_t mtiles;
  int64_t ntiles;
  int ksplit;
  int kblocks;
};

// Tile configuration, tile counts and K split for one call.
//  * M > 64: 112-row tiles (MI = 7: 776 = 7 x 112 - 8).  Wide GEMMs (gate/up) use 4 waves
//    along N (112 x 256 workgroup tiles).  When that leaves fewer than 1.5 workgroups per
//    CU (QKV, o, down):
//    - K >= 8192 (down): 8 waves split K (2 per SIMD, each with 1/8 of K), 112 x 64 tiles;
//    - otherwise 32 x 128 tiles that keep the whole K in each wave, when they fit in two
//      workgroups per CU (at M = 776 with weights streamed from HBM: o 7.8 us and QKV
//      9.3 us, against 10.1 and 12.0 with 4 waves splitting K of 112 x 64 tiles, and 9.0
//      and 10.1 with 64 x 128 tiles), else 64 x 128 tiles, else the K split.  One weight
//      (o) and the QKV + RoPE launch take 64 x 64 tiles with 4 waves splitting K instead
//      (at M = 776, weights warm: o + residual 7.16 -> 6.87 us, QKV + RoPE 9.19 -> 8.55;
//      the plain three-weight QKV launch measured 7.6 -> 9.3 us with them, and 32 x 128
//      tiles with the K split 9.0 us for QKV).
//  * M <= 64 (weight streaming): 16-, 32- or 64-row tiles of 32 columns whose four waves
//    split K and sum their parts through LDS, so that one launch streams the weights
//    (QKV at M = 1: 3.0 us, against 5.8 us for 16 x 128 tiles with a global K split and
//    its reduce launch).  A global split stays for long K (down), with at least 4 k blocks
//    per wave.  The paired gate/up GELU GEMM uses them up to M = 16 only, and 4-waves-
//    along-N tiles with the global split above that.
Plan make_plan(int64_t m, int32_t k, int ngroups, const int32_t* n, bool gelu, bool allow_split,
               bool rope = false) {
  Plan pl{};
  const int64_t kNumCUs = w4a4::device_cu_count();
  // The GELU pairing's 16-column K-split tiles make 1024 workgroups at gate/up size, each
  // staging the GELU correction table: from M = 17 on the wider tiles are faster.
  const bool stream_k = m <= 16 || (!gelu && m <= 64);
  if (m <= 16)
    pl.cfg = stream_k ? kCfg1x2K4 : kCfg1x2;
  else if (m <= 32)
    pl.cfg = stream_k ? kCfg2x2K4 : kCfg2x2;
  else if (m <= 64)
    pl.cfg = stream_k ? kCfg4x2K4 : kCfg4x2;
  else
    pl.cfg = kCfg7x4;
  const bool small = pl.cfg.kw > 1;
  auto count_tiles = [&](const TileCfg& c) {
    int64_t t = 0;
    if (gelu) {
      t = cdiv(n[0], c.cols(true));
    } else {
      for (int g = 0; g < ngroups; ++g) t += cdiv(n[g], c.cols(false));
    }
    return t;
  };
  pl.mtiles = cdiv(m, 16 * pl.cfg.mi);
  pl.ntiles = count_tiles(pl.cfg);
  if (pl.cfg.id == w4a4::kCfg7x4 && 2 * pl.mtiles * pl.ntiles < 3 * kNumCUs) {
    if (k >= 8192) {
      pl.cfg = kCfg7x4K8;
    } else if (cdiv(m, 32) * count_tiles(kCfg2x2) <= 2 * kNumCUs) {
      pl.cfg = kCfg2x2;
      // One weight, or the attention prep's launch: 64 x 64 tiles with the K split, when
      // they give every CU a workgroup (then no global split follows either way).
      if ((ngroups == 1 || rope) && cdiv(m, 64) * count_tiles(kCfg4x4K4) >= kNumCUs) pl.cfg = kCfg4x4K4;
    } else if (cdiv(m, 64) * count_tiles(kCfg4x2) <= 2 * kNumCUs) {
      pl.cfg = kCfg4x2;
    } else {
      pl.cfg = kCfg7x4K4;
    }
    pl.mtiles = cdiv(m, 16 * pl.cfg.mi);
    pl.ntiles = count_tiles(pl.cfg);
  }
  // The QKV + RoPE launch keeps the 64 x 64 K-split tiles at large M too: the attention
  // prep epilogue of its K and V tiles runs long on 112-row tiles (batch 8 x 776 tokens:
  // forward 14.36-14.38 -> 14.24-14.25 ms; the plain o GEMM measured slower on them there,
  // 25.6 -> 39.7 us, and keeps 112 x 256 tiles).
  if (rope && pl.cfg.id == w4a4::kCfg7x4 && cdiv(m, 64) * count_tiles(kCfg4x4K4) >= kNumCUs) {
    pl.cfg = kCfg4x4K4;
    pl.mtiles = cdiv(m, 16 * pl.cfg.mi);
    pl.ntiles = count_tiles(pl.cfg);
  }
  const int nkb = w4a4::kblocks128(k);
  int ks = 1;
  if (allow_split) {
    // A global split costs an int32 workspace round trip and a reduce launch; it only
    // pays when fewer than half of the CUs would get a workgroup.
    const int64_t base = pl.mtiles * pl.ntiles;
    if (2 * base < kNumCUs) ks = static_cast<int>(cdiv(kNumCUs, base));
    if (ks > w4a4::kMaxKSplit) ks = w4a4::kMaxKSplit;
    // Small M: the workgroup's waves already split K; a global split is left for long K
    // only, keeping at least 4 k blocks per wave.
    if (small) ks = std::min<int>(ks, std::max(1, nkb / (4 * pl.cfg.kw)));
  }
  if (ks > nkb) ks = nkb;
  if (ks < 1) ks = 1;
  const int per = static_cast<int>(cdiv(nkb, ks));
  pl.kblocks = per;
  pl.ksplit = static_cast<int>(cdiv(nkb, per));
  return pl;
}

// The MFMA sum S = 16 acc + row and column terms is bounded by 2048 K: int32 holds it for
// every K up to 2^19.
constexpr int32_t kMaxK = 1 << 19;

int validate_gemm_common(const int32_t* q, const float* sa, int64_t m, int32_t k) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (k <= 0 || k % 64 != 0) return fail(PI05W4A4_EINVAL, "K must be a multiple of 64, got %d", k);
  if (k > kMaxK) return fail(PI05W4A4_EINVAL, "K must be at most %d, got %d", kMaxK, k);
  if (m > 0 && (q == nullptr || sa == nullptr))
    return fail(PI05W4A4_EINVAL, "null activation codes or scales");
  if (!aligned(q, 16)) return fail(PI05W4A4_EINVAL, "activation codes must be 16-byte aligned");
  if (!aligned(sa, 4)) return fail(PI05W4A4_EINVAL, "activation scales must be 4-byte aligned");
  return PI05W4A4_OK;
}

// Output offsets inside one 112-row tile are 32-bit: N is bounded well below 2^31 / 224.
constexpr int32_t kMaxN = 1 << 20;

int validate_weight(const int32_t* w, int32_t n, const char* name) {
  if (w == nullptr) return fail(PI05W4A4_EINVAL, "%s is null", name);
  if (n <= 0 || n % 16 != 0)
    return fail(PI05W4A4_EINVAL, "%s: N must be a positive multiple of 16, got %d", name, n);
  if (n > kMaxN) return fail(PI05W4A4_EINVAL, "%s: N must be at most %d, got %d", name, kMaxN, n);
  if (!aligned(w, 16)) return fail(PI05W4A4_EINVAL, "%s must be 16-byte aligned", name);
  return PI05W4A4_OK;
}

// Attention prep of pi05w4a4_gemm_qkv_rope (groups 1 and 2 are K and V).
struct QkvRope {
  const void* cos;
  const void* sin;
  void* kv;
  int32_t seq;
};

int run_gemm(const int32_t* q, const float* sa, int64_t m, int32_t k, int ngroups,
             const int32_t* const* w, const int32_t* n, void* const* y, int mode,
             void* workspace, size_t workspace_bytes, hipStream_t stream,
             const void* residual = nullptr, const QkvRope* rope = nullptr) {
  const bool gelu = mode == w4a4::kEpiGeluUp;
  // The attention prep epilogue needs the whole K in one launch: no global split for it.
  const Plan pl = make_plan(m, k, ngroups, n, gelu, mode != w4a4::kEpiAcc && rope == nullptr, rope != nullptr);
  if (pl.mtiles > 65535) return fail(PI05W4A4_EINVAL, "M too large (%lld rows)", (long long)m);
  w4a4::GemmParams p{};
  p.q = q;
  p.sa = sa;
  p.m = m;
  p.k = k;
  p.ngroups = ngroups;
  int64_t n_total = 0;
  int tile_begin = 0;
  for (int g = 0; g < ngroups; ++g) {
    p.g[g].w = w[g];
    p.g[g].y = y[g];
    p.g[g].n = n[g];
    p.g[g].tile_begin = tile_begin;
    tile_begin += static_cast<int>(cdiv(n[g], pl.cfg.cols(false)));
    n_total += n[g];
  }
  p.ntiles = static_cast<int32_t>(pl.ntiles);
  p.mtiles = static_cast<int32_t>(pl.mtiles);
  p.ksplit = pl.ksplit;
  p.kblocks_per_split = pl.kblocks;
  p.mblocks = static_cast<int32_t>(cdiv(m, 16));
  p.n_total = static_cast<int32_t>(n_total);
  p.gelu_pair_n = gelu ? n[0] : 0;
  p.res = static_cast<const _Float16*>(residual);
  if (rope != nullptr) {
    p.rope_group = 2;
    p.vt_group = 3;
    p.cosb = static_cast<const _Float16*>(rope->cos);
    p.sinb = static_cast<const _Float16*>(rope->sin);
    p.kv = static_cast<_Float16*>(rope->kv);
    p.seq = rope->seq;
    p.s_pad = static_cast<int32_t>(w4a4::attn_s_pad(rope->seq));
  }
  if (pl.ksplit > 1) {
    const size_t need = static_cast<size_t>(pl.ksplit) * static_cast<size_t>(m) *
                        static_cast<size_t>(n_total) * sizeof(int32_t);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(PI05W4A4_EWORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                  workspace_bytes);
    if (!aligned(workspace, 16)) return fail(PI05W4A4_EINVAL, "workspace must be 16-byte aligned");
    p.partial = static_cast<int32_t*>(workspace);
    p.mode = w4a4::kEpiPartial;
    hipError_t e = w4a4::launch_gemm(p, pl.cfg.id, stream);
    if (e != hipSuccess) return hip_status(e, "gemm launch");
    p.mode = gelu ? w4a4::kEpiGeluUp : w4a4::kEpiFp16;
    return hip_status(w4a4::launch_splitk_reduce(p, stream), "split-K reduce launch");
  }
  p.mode = mode;
  return hip_status(w4a4::launch_gemm(p, pl.cfg.id, stream), "gemm launch");
}

// Shape checks shared by the two attention entry points.
int validate_attention(int64_t b, int32_t s, int32_t h, int32_t kvh, int32_t d) {
  if (d != w4a4::kAttnHeadDim)
    return fail(PI05W4A4_EINVAL, "head_dim must be %d, got %d", w4a4::kAttnHeadDim, d);
  if (b < 1 || b > 65535) return fail(PI05W4A4_EINVAL, "batch must be in [1, 65535], got %lld", (long long)b);
  if (s < 1 || s > w4a4::kAttnMaxKeys)
    return fail(PI05W4A4_EINVAL, "sequence length must be in [1, %d], got %d", w4a4::kAttnMaxKeys, s);
  if (kvh < 1 || kvh > 65535 || h < kvh || h % kvh != 0)
    return fail(PI05W4A4_EINVAL, "query heads (%d) must be a multiple of KV heads (%d)", h, kvh);
  return ok();
}
}  // namespace

extern "C" {

int pi05w4a4_version(void) { return 100; }

const char* pi05w4a4_last_error(void) { return g_last_error.c_str(); }

namespace {

// Validates the warm-buffer arguments of the cache-warming entry points and collects the
// non-empty buffers.
static int collect_warm(const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                 w4a4::CacheWarmParams* warm) {
  *warm = w4a4::CacheWarmParams{};
  if (warm_n < 0 || warm_n > w4a4::kMaxWarmBuffers)
    return fail(PI05W4A4_EINVAL, "cache warming takes 0..%d buffers, got %d", w4a4::kMaxWarmBuffers, warm_n);
  if (warm_n > 0 && (warm_ptrs == nullptr || warm_bytes == nullptr))
    return fail(PI05W4A4_EINVAL, "null pointer argument");
  for (int i = 0; i < warm_n; ++i) {
    if (warm_ptrs[i] == nullptr || !aligned(warm_ptrs[i], 16) || warm_bytes[i] % 16 != 0)
      return fail(PI05W4A4_EINVAL, "warm buffer %d must be non-null, 16-byte aligned and a multiple of 16 bytes", i);
    if (warm_bytes[i] == 0) continue;
    warm->ptr[warm->nbuf] = warm_ptrs[i];
    warm->n16[warm->nbuf] = static_cast<int64_t>(warm_bytes[i] / 16);
    ++warm->nbuf;
  }
  return ok();
}

static int quantize_call(const void* x_fp16, int64_t m, int32_t k, int32_t* q, float* sa,
                  const w4a4::CacheWarmParams* warm, void* stream) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (k <= 0 || k % 64 != 0) return fail(PI05W4A4_EINVAL, "K must be a multiple of 64, got %d", k);
  if (m == 0) return ok();
  if (x_fp16 == nullptr || q == nullptr || sa == nullptr)
    return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (!aligned(x_fp16, 16) || !aligned(q, 16) || !aligned(sa, 4))
    return fail(PI05W4A4_EINVAL, "x and q must be 16-byte aligned, sa 4-byte aligned");
  if (m > 0x7fffffffLL) return fail(PI05W4A4_EINVAL, "M too large");
  const float inv_sqrt_k = static_cast<float>(1.0 / std::sqrt(static_cast<double>(k)));
  return hip_status(w4a4::launch_quantize(x_fp16, m, k, q, sa, inv_sqrt_k,
                                          static_cast<hipStream_t>(stream), warm),
                    "quantize launch");
}

}  // namespace

int pi05w4a4_quantize(const void* x_fp16, int64_t m, int32_t k, int32_t* q, float* sa,
                      void* stream) {
  return quantize_call(x_fp16, m, k, q, sa, nullptr, stream);
}

int pi05w4a4_quantize_warm(const void* x_fp16, int64_t m, int32_t k, int32_t* q, float* sa,
                           const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                           void* stream) {
  w4a4::CacheWarmParams warm;
  const int rc = collect_warm(warm_ptrs, warm_bytes, warm_n, &warm);
  if (rc) return rc;
  return quantize_call(x_fp16, m, k, q, sa, &warm, stream);
}

size_t pi05w4a4_q_words(int64_t m, int32_t k) {
  if (m <= 0 || k <= 0) return 0;
  return static_cast<size_t>(w4a4::q_total_words(cdiv(m, 16), w4a4::kblocks128(k)));
}

size_t pi05w4a4_mfma_words(int32_t n, int32_t k) {
  if (n <= 0 || k <= 0) return 0;
  return static_cast<size_t>(n) * (static_cast<size_t>(w4a4::kblocks128(k)) * 16 + 2);
}

int pi05w4a4_repack_weight(const int32_t* src, int32_t src_layout, int32_t n, int32_t k,
                           int64_t src_stride, int32_t* dst, void* stream) {
  if (src == nullptr || dst == nullptr) return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (k <= 0 || k % 64 != 0) return fail(PI05W4A4_EINVAL, "K must be a multiple of 64, got %d", k);
  if (n <= 0 || n % 16 != 0)
    return fail(PI05W4A4_EINVAL, "N must be a positive multiple of 16, got %d", n);
  if (src_layout == PI05W4A4_LAYOUT_ROW_MAJOR) {
    if (src_stride < k / 8 + 1)
      return fail(PI05W4A4_EINVAL,
                  "row stride must contain K/8 packed words plus a scale (%lld < %d)",
                  (long long)src_stride, k / 8 + 1);
  } else if (src_layout != PI05W4A4_LAYOUT_WMMA_TILED) {
    return fail(PI05W4A4_EINVAL, "unknown source layout %d", src_layout);
  }
  return hip_status(w4a4::launch_repack(src, src_layout, n, k, src_stride, dst,
                                        static_cast<hipStream_t>(stream)),
                    "repack launch");
}

size_t pi05w4a4_gemm_workspace_bytes(int64_t m, int32_t k, int32_t ngroups, const int32_t* n,
                                     int32_t gelu) {
  if (m <= 0 || k <= 0 || ngroups < 1 || ngroups > w4a4::kMaxGroups || n == nullptr) return 0;
  const Plan pl = make_plan(m, k, ngroups, n, gelu != 0, true);
  if (pl.ksplit <= 1) return 0;
  int64_t n_total = 0;
  for (int g = 0; g < ngroups; ++g) n_total += n[g];
  return static_cast<size_t>(pl.ksplit) * static_cast<size_t>(m) * static_cast<size_t>(n_total) *
         sizeof(int32_t);
}

int pi05w4a4_gemm(const int32_t* q, const float* sa, int64_t m, int32_t k,
                  const int32_t* w_mfma, int32_t n, void* y_fp16, void* workspace,
                  size_t workspace_bytes, void* stream) {
  const int32_t* ws[1] = {w_mfma};
  const int32_t ns[1] = {n};
  void* ys[1] = {y_fp16};
  return pi05w4a4_gemm_multi(q, sa, m, k, 1, ws, ns, ys, workspace, workspace_bytes, stream);
}

int pi05w4a4_gemm_multi(const int32_t* q, const float* sa, int64_t m, int32_t k,
                        int32_t ngroups, const int32_t* const* w_mfma, const int32_t* n,
                        void* const* y_fp16, void* workspace, size_t workspace_bytes,
                        void* stream) {
  int rc = validate_gemm_common(q, sa, m, k);
  if (rc) return rc;
  if (ngroups < 1 || ngroups > w4a4::kMaxGroups || w_mfma == nullptr || n == nullptr ||
      y_fp16 == nullptr)
    return fail(PI05W4A4_EINVAL, "ngroups must be 1..3 with non-null arrays");
  for (int g = 0; g < ngroups; ++g) {
    rc = validate_weight(w_mfma[g], n[g], "weight");
    if (rc) return rc;
    if (m > 0 && y_fp16[g] == nullptr) return fail(PI05W4A4_EINVAL, "null output");
    if (!aligned(y_fp16[g], 16)) return fail(PI05W4A4_EINVAL, "output must be 16-byte aligned");
  }
  if (m == 0) return ok();
  return run_gemm(q, sa, m, k, ngroups, w_mfma, n, y_fp16, w4a4::kEpiFp16, workspace,
                  workspace_bytes, static_cast<hipStream_t>(stream));
}

int pi05w4a4_quant_gemm_small(const void* x_fp16, const void* nw_fp16, float eps, int32_t unit_offset, int64_t m,
                              int32_t k, int32_t ngroups, const int32_t* const* w_mfma, const int32_t* n,
                              void* const* y_fp16, const void* residual_fp16, void* stream) {
  if (m < 1 || m > w4a4::kQproMaxRows)
    return fail(PI05W4A4_EINVAL, "the small-M quant + GEMM takes 1..%d rows, got %lld", w4a4::kQproMaxRows,
                (long long)m);
  if (k != 2048) return fail(PI05W4A4_EINVAL, "the small-M quant + GEMM takes K = 2048, got %d", k);
  if (x_fp16 == nullptr || !aligned(x_fp16, 16)) return fail(PI05W4A4_EINVAL, "x must be non-null and 16-byte aligned");
  if (nw_fp16 != nullptr && !aligned(nw_fp16, 16)) return fail(PI05W4A4_EINVAL, "the norm weight must be 16-byte aligned");
  if (ngroups < 1 || ngroups > w4a4::kMaxGroups || w_mfma == nullptr || n == nullptr || y_fp16 == nullptr)
    return fail(PI05W4A4_EINVAL, "ngroups must be 1..3 with non-null arrays");
  if (residual_fp16 != nullptr && (ngroups != 1 || !aligned(residual_fp16, 16)))
    return fail(PI05W4A4_EINVAL, "a residual takes one weight and 16-byte alignment");
  w4a4::GemmParams p{};
  int tile_begin = 0;
  int64_t n_total = 0;
  for (int g = 0; g < ngroups; ++g) {
    const int rc = validate_weight(w_mfma[g], n[g], "weight");
    if (rc) return rc;
    if (y_fp16[g] == nullptr || !aligned(y_fp16[g], 16)) return fail(PI05W4A4_EINVAL, "outputs must be non-null and 16-byte aligned");
    p.g[g].w = w_mfma[g];
    p.g[g].y = y_fp16[g];
    p.g[g].n = n[g];
    p.g[g].tile_begin = tile_begin;
    tile_begin += static_cast<int>(cdiv(n[g], kCfg1x2K4.cols(false)));
    n_total += n[g];
  }
  p.q = static_cast<const int32_t*>(x_fp16);  // not read: the prologue's codes stay in LDS
  p.sa = nullptr;
  p.m = m;
  p.k = k;
  p.ngroups = ngroups;
  p.ntiles = tile_begin;
  p.mtiles = 1;
  p.ksplit = 1;
  p.kblocks_per_split = w4a4::kblocks128(k);
  p.mblocks = 1;
  p.n_total = static_cast<int32_t>(n_total);
  p.mode = w4a4::kEpiFp16;
  p.res = static_cast<const _Float16*>(residual_fp16);
  p.xpro = static_cast<const _Float16*>(x_fp16);
  p.nwpro = static_cast<const _Float16*>(nw_fp16);
  p.eps_pro = eps;
  p.unit_offset_pro = unit_offset != 0;
  p.inv_sqrt_k_pro = static_cast<float>(1.0 / std::sqrt(static_cast<double>(k)));
  return hip_status(w4a4::launch_gemm_qpro(p, static_cast<hipStream_t>(stream)), "small-M quant + gemm launch");
}

int pi05w4a4_gemm_residual(const int32_t* q, const float* sa, int64_t m, int32_t k,
                           const int32_t* w_mfma, int32_t n, const void* residual_fp16,
                           void* y_fp16, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = validate_gemm_common(q, sa, m, k);
  if (rc) return rc;
  rc = validate_weight(w_mfma, n, "weight");
  if (rc) return rc;
  if (m == 0) return ok();
  if (y_fp16 == nullptr || residual_fp16 == nullptr) return fail(PI05W4A4_EINVAL, "null output or residual");
  if (!aligned(y_fp16, 16) || !aligned(residual_fp16, 16))
    return fail(PI05W4A4_EINVAL, "output and residual must be 16-byte aligned");
  const int32_t* ws[1] = {w_mfma};
  const int32_t ns[1] = {n};
  void* ys[1] = {y_fp16};
  return run_gemm(q, sa, m, k, 1, ws, ns, ys, w4a4::kEpiFp16, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream), residual_fp16);
}

int pi05w4a4_gemm_qkv_rope(const int32_t* q, const float* sa, int64_t m, int32_t k,
                           const int32_t* w_q_mfma, int32_t n_q, const int32_t* w_k_rope,
                           const int32_t* w_v_mfma, const void* cos_fp16, const void* sin_fp16,
                           int64_t b, int32_t s, void* y_q, void* k_rope, void* y_v, void* kv_mfma,
                           void* stream) {
  int rc = validate_gemm_common(q, sa, m, k);
  if (rc) return rc;
  if (b < 1 || s < 1 || s % 8 != 0 || s > w4a4::kAttnMaxKeys || m != b * s)
    return fail(PI05W4A4_EINVAL, "gemm_qkv_rope: M = B * S with S a multiple of 8 in [8, %d], got M=%lld B=%lld S=%d",
                w4a4::kAttnMaxKeys, (long long)m, (long long)b, s);
  rc = validate_weight(w_q_mfma, n_q, "q weight");
  if (rc) return rc;
  rc = validate_weight(w_k_rope, w4a4::kAttnHeadDim, "k weight");
  if (rc) return rc;
  rc = validate_weight(w_v_mfma, w4a4::kAttnHeadDim, "v weight");
  if (rc) return rc;
  const void* ptrs[] = {y_q, k_rope, y_v, kv_mfma, cos_fp16, sin_fp16};
  for (const void* ptr : ptrs) {
    if (ptr == nullptr) return fail(PI05W4A4_EINVAL, "gemm_qkv_rope: null output or rotary table");
    if (!aligned(ptr, 16)) return fail(PI05W4A4_EINVAL, "gemm_qkv_rope: outputs and rotary tables must be 16-byte aligned");
  }
  const int32_t* ws[3] = {w_q_mfma, w_k_rope, w_v_mfma};
  const int32_t ns[3] = {n_q, w4a4::kAttnHeadDim, w4a4::kAttnHeadDim};
  void* ys[3] = {y_q, k_rope, y_v};
  const QkvRope rope{cos_fp16, sin_fp16, kv_mfma, s};
  return run_gemm(q, sa, m, k, 3, ws, ns, ys, w4a4::kEpiFp16, nullptr, 0, static_cast<hipStream_t>(stream),
                  nullptr, &rope);
}

int pi05w4a4_permute_rope_pairs(const int32_t* src_mfma, int32_t k, int32_t* dst_mfma, void* stream) {
  if (src_mfma == nullptr || dst_mfma == nullptr) return fail(PI05W4A4_EINVAL, "null weight");
  if (k <= 0 || k % 64 != 0 || k > kMaxK) return fail(PI05W4A4_EINVAL, "K must be a multiple of 64, got %d", k);
  if (src_mfma == dst_mfma) return fail(PI05W4A4_EINVAL, "permute_rope_pairs is not in place");
  const int64_t block = static_cast<int64_t>(w4a4::kblocks128(k)) * 256;  // words per 16-row block
  const int64_t payload = 16 * block;                                     // 256 rows
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int nb = 0; nb < 16; ++nb) {
    const int src_nb = (nb >> 1) + 8 * (nb & 1);
    hipError_t e = hipMemcpyAsync(dst_mfma + nb * block, src_mfma + src_nb * block, block * 4,
                                  hipMemcpyDeviceToDevice, st);
    // scales (256 floats after the payload), then the column corrections
    if (e == hipSuccess)
      e = hipMemcpyAsync(dst_mfma + payload + nb * 16, src_mfma + payload + src_nb * 16, 64,
                         hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
      e = hipMemcpyAsync(dst_mfma + payload + 256 + nb * 16, src_mfma + payload + 256 + src_nb * 16, 64,
                         hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return hip_status(e, "permute_rope_pairs copy");
  }
  return ok();
}

}  // extern "C"

namespace {
static int rmsnorm_quantize_call(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                 int64_t m, int32_t k, int32_t* q, float* sa,
                                 const w4a4::CacheWarmParams* warm, void* stream) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (k != 2048) return fail(PI05W4A4_EINVAL, "the fused RMSNorm quantizer takes K = 2048, got %d", k);
  if (m == 0) return ok();
  if (!x_fp16 || !w_fp16 || !q || !sa) return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (!aligned(x_fp16, 16) || !aligned(w_fp16, 16) || !aligned(q, 16) || !aligned(sa, 4))
    return fail(PI05W4A4_EINVAL, "x, w and q must be 16-byte aligned, sa 4-byte aligned");
  if (m > 0x7fffffffLL) return fail(PI05W4A4_EINVAL, "M too large");
  return hip_status(w4a4::launch_rmsnorm_quantize(x_fp16, w_fp16, eps, unit_offset != 0, m, k, q, sa,
                                                  static_cast<float>(1.0 / std::sqrt(2048.0)),
                                                  static_cast<hipStream_t>(stream), warm),
                    "rmsnorm quantize launch");
}
}  // namespace

extern "C" {

int pi05w4a4_rmsnorm_quantize(const void* x_fp16, const void* w_fp16, float eps,
                              int32_t unit_offset, int64_t m, int32_t k, int32_t* q, float* sa,
                              void* stream) {
  return rmsnorm_quantize_call(x_fp16, w_fp16, eps, unit_offset, m, k, q, sa, nullptr, stream);
}

int pi05w4a4_rmsnorm_quantize_warm(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                   int64_t m, int32_t k, int32_t* q, float* sa, const void* const* warm_ptrs,
                                   const size_t* warm_bytes, int32_t warm_n, void* stream) {
  w4a4::CacheWarmParams warm;
  const int rc = collect_warm(warm_ptrs, warm_bytes, warm_n, &warm);
  if (rc) return rc;
  return rmsnorm_quantize_call(x_fp16, w_fp16, eps, unit_offset, m, k, q, sa, &warm, stream);
}

// ---- E3M2 operand form (the q6 / w6 layouts of w4a4_internal.h)

size_t pi05w4a4_q_e3m2_bytes(int64_t m, int32_t k) {
  if (m <= 0 || k <= 0) return 0;
  return static_cast<size_t>(w4a4::q6_bytes(cdiv(m, 16), w4a4::kblocks128(k)));
}

size_t pi05w4a4_e3m2_words(int32_t n, int32_t k) {
  if (n <= 0 || k <= 0) return 0;
  return static_cast<size_t>(w4a4::w6_payload_words(n, w4a4::kblocks128(k))) + static_cast<size_t>(n);
}

namespace {
// The fp32 sums of the E3M2 MFMA are exact while |acc| <= 64 K < 2^24.
constexpr int32_t kMaxKE3m2 = 1 << 18;

static int validate_e3m2_shape(int32_t n, int32_t k, const char* name) {
  if (k <= 0 || k % 128 != 0 || k > kMaxKE3m2)
    return fail(PI05W4A4_EINVAL, "%s: E3M2 operands need K %% 128 == 0 and K <= %d, got %d", name, kMaxKE3m2, k);
  if (n <= 0 || n % 32 != 0 || n > kMaxN)
    return fail(PI05W4A4_EINVAL, "%s: E3M2 weights need N %% 32 == 0 (column pairs) and N <= %d, got %d", name,
                kMaxN, n);
  return PI05W4A4_OK;
}

static int quantize_e3m2_call(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset, int64_t m,
                              int32_t k, void* q6, float* sa, void* stream,
                              const w4a4::CacheWarmParams* warm = nullptr) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (k != 2048) return fail(PI05W4A4_EINVAL, "the E3M2 quantizer takes K = 2048, got %d", k);
  if (m == 0) return ok();
  if (!x_fp16 || !q6 || !sa) return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (!aligned(x_fp16, 16) || (w_fp16 != nullptr && !aligned(w_fp16, 16)) || !aligned(q6, 16) || !aligned(sa, 4))
    return fail(PI05W4A4_EINVAL, "x, w and q6 must be 16-byte aligned, sa 4-byte aligned");
  if (m > 0x7fffffffLL) return fail(PI05W4A4_EINVAL, "M too large");
  return hip_status(w4a4::launch_quantize_e3m2(x_fp16, w_fp16, eps, unit_offset != 0, m, k, q6, sa,
                                               static_cast<float>(1.0 / std::sqrt(2048.0)),
                                               static_cast<hipStream_t>(stream), warm),
                    "E3M2 quantize launch");
}
}  // namespace

int pi05w4a4_repack_weight_e3m2(const int32_t* w_mfma, int32_t n, int32_t k, int32_t* w6, void* stream) {
  if (w_mfma == nullptr || w6 == nullptr) return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (w_mfma == w6) return fail(PI05W4A4_EINVAL, "the E3M2 repack is not in place");
  const int rc = validate_e3m2_shape(n, k, "weight");
  if (rc) return rc;
  if (!aligned(w_mfma, 16) || !aligned(w6, 16)) return fail(PI05W4A4_EINVAL, "weights must be 16-byte aligned");
  return hip_status(w4a4::launch_repack_e3m2(w_mfma, n, k, w6, static_cast<hipStream_t>(stream)),
                    "E3M2 repack launch");
}

int pi05w4a4_quantize_e3m2(const void* x_fp16, int64_t m, int32_t k, void* q6, float* sa, void* stream) {
  return quantize_e3m2_call(x_fp16, nullptr, 0.0f, 0, m, k, q6, sa, stream);
}

int pi05w4a4_rmsnorm_quantize_e3m2(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                   int64_t m, int32_t k, void* q6, float* sa, void* stream) {
  if (m > 0 && w_fp16 == nullptr) return fail(PI05W4A4_EINVAL, "null pointer argument");
  return quantize_e3m2_call(x_fp16, w_fp16, eps, unit_offset, m, k, q6, sa, stream);
}

int pi05w4a4_rmsnorm_quantize_e3m2_warm(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                                        int64_t m, int32_t k, void* q6, float* sa, const void* const* warm_ptrs,
                                        const size_t* warm_bytes, int32_t warm_n, void* stream) {
  if (m > 0 && w_fp16 == nullptr) return fail(PI05W4A4_EINVAL, "null pointer argument");
  w4a4::CacheWarmParams warm;
  const int rc = collect_warm(warm_ptrs, warm_bytes, warm_n, &warm);
  if (rc) return rc;
  return quantize_e3m2_call(x_fp16, w_fp16, eps, unit_offset, m, k, q6, sa, stream, &warm);
}

int pi05w4a4_gemm_e3m2(const void* q6, const float* sa, int64_t m, int32_t k, int32_t ngroups,
                       const int32_t* const* w6, const int32_t* n, void* const* y_fp16, int32_t gelu_up,
                       void* stream) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (w6 == nullptr || n == nullptr || y_fp16 == nullptr)
    return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (gelu_up != 0 ? ngroups != 2 : (ngroups < 1 || ngroups > w4a4::kMaxGroups))
    return fail(PI05W4A4_EINVAL, "ngroups must be 2 with gelu_up, else 1..3, got %d", ngroups);
  if (gelu_up != 0 && n[0] != n[1])
    return fail(PI05W4A4_EINVAL, "gate and up weights must have the same N (%d != %d)", n[0], n[1]);
  for (int g = 0; g < ngroups; ++g) {
    int rc = validate_e3m2_shape(n[g], k, "weight");
    if (rc) return rc;
    if (w6[g] == nullptr || !aligned(w6[g], 16)) return fail(PI05W4A4_EINVAL, "weights must be non-null and 16-byte aligned");
    if (g < (gelu_up != 0 ? 1 : ngroups) && m > 0 && (y_fp16[g] == nullptr || !aligned(y_fp16[g], 16)))
      return fail(PI05W4A4_EINVAL, "outputs must be non-null and 16-byte aligned");
  }
  if (m == 0) return ok();
  if (q6 == nullptr || sa == nullptr) return fail(PI05W4A4_EINVAL, "null activation codes or scales");
  if (!aligned(q6, 16) || !aligned(sa, 4))
    return fail(PI05W4A4_EINVAL, "q6 must be 16-byte aligned, sa 4-byte aligned");
  // Tiles: 112 x 256 (GELU: 112 x 128 gate + up) when they give at least 1.5 workgroups per
  // CU, else 32 x 128 (the narrow GEMMs: QKV, o).
  const int64_t cus = w4a4::device_cu_count();
  const int64_t m7 = cdiv(m, 112);
  int64_t n7 = 0, n2 = 0;
  for (int g = 0; g < ngroups; ++g) {
    n7 += cdiv(n[g], gelu_up != 0 ? 128 : 256);
    n2 += cdiv(n[g], 128);
  }
  if (gelu_up != 0) n7 = cdiv(n[0], 128);
  const bool narrow = gelu_up == 0 && 2 * m7 * n7 < 3 * cus;
  const int tile_cfg = narrow ? w4a4::kCfg2x2 : w4a4::kCfg7x4;
  const int64_t mtiles = narrow ? cdiv(m, 32) : m7;
  if (mtiles > 65535) return fail(PI05W4A4_EINVAL, "M too large (%lld rows)", (long long)m);
  w4a4::GemmParams p{};
  p.q = static_cast<const int32_t*>(q6);
  p.sa = sa;
  p.m = m;
  p.k = k;
  p.ngroups = ngroups;
  const int tile_cols = gelu_up != 0 ? 128 : (narrow ? 128 : 256);  // 4 waves x 64 (GELU: 32 + 32) or 32 columns
  int tile_begin = 0;
  int64_t n_total = 0;
  for (int g = 0; g < ngroups; ++g) {
    p.g[g].w = w6[g];
    p.g[g].y = gelu_up != 0 ? y_fp16[0] : y_fp16[g];
    p.g[g].n = n[g];
    p.g[g].tile_begin = tile_begin;
    tile_begin += static_cast<int>(cdiv(n[g], tile_cols));
    n_total += n[g];
  }
  p.ntiles = gelu_up != 0 ? static_cast<int32_t>(cdiv(n[0], tile_cols)) : tile_begin;
  p.mtiles = static_cast<int32_t>(mtiles);
  p.ksplit = 1;
  p.kblocks_per_split = w4a4::kblocks128(k);
  p.mblocks = static_cast<int32_t>(cdiv(m, 16));
  p.n_total = static_cast<int32_t>(n_total);
  p.gelu_pair_n = gelu_up != 0 ? n[0] : 0;
  p.mode = gelu_up != 0 ? w4a4::kEpiGeluUp : w4a4::kEpiFp16;
  return hip_status(w4a4::launch_gemm_e3m2(p, tile_cfg, static_cast<hipStream_t>(stream)), "E3M2 gemm launch");
}

int pi05w4a4_gemm_gelu_up(const int32_t* q, const float* sa, int64_t m, int32_t k,
                          const int32_t* w_gate_mfma, const int32_t* w_up_mfma, int32_t n,
                          void* h_fp16, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = validate_gemm_common(q, sa, m, k);
  if (rc) return rc;
  rc = validate_weight(w_gate_mfma, n, "gate weight");
  if (rc) return rc;
  rc = validate_weight(w_up_mfma, n, "up weight");
  if (rc) return rc;
  if (m > 0 && h_fp16 == nullptr) return fail(PI05W4A4_EINVAL, "null output");
  if (!aligned(h_fp16, 16)) return fail(PI05W4A4_EINVAL, "output must be 16-byte aligned");
  if (m == 0) return ok();
  const int32_t* ws[2] = {w_gate_mfma, w_up_mfma};
  const int32_t ns[2] = {n, n};
  void* ys[2] = {h_fp16, h_fp16};
  return run_gemm(q, sa, m, k, 2, ws, ns, ys, w4a4::kEpiGeluUp, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream));
}

size_t pi05w4a4_mlp_ctl_words(int64_t m) {
  if (m <= 0) return 0;
  // header, then one 128-byte line per possible m-tile (at most one per 16 rows)
  return static_cast<size_t>(w4a4::kMlpCtlHeader + w4a4::kMlpCtlStride * cdiv(m, 16));
}

namespace {
// Host-visible word set by a bounded wait of the fused gate/up + down-quant launch that ran
// out (pinned, mapped host memory shared by every device; allocated once).
std::mutex g_status_mu;
uint32_t* g_status_host = nullptr;
uint32_t* g_status_dev = nullptr;

static uint32_t* mlp_status_device_word() {
  std::lock_guard<std::mutex> lk(g_status_mu);
  if (g_status_dev != nullptr) return g_status_dev;
  void* hp = nullptr;
  if (hipHostMalloc(&hp, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) return nullptr;
  void* dp = nullptr;
  if (hipHostGetDevicePointer(&dp, hp, 0) != hipSuccess) {
    (void)hipHostFree(hp);
    return nullptr;
  }
  g_status_host = static_cast<uint32_t*>(hp);
  *reinterpret_cast<volatile uint32_t*>(g_status_host) = 0;
  g_status_dev = static_cast<uint32_t*>(dp);
  return g_status_dev;
}
}  // namespace

int64_t pi05w4a4_mlp_status(int32_t clear) {
  if (mlp_status_device_word() == nullptr) return -1;
  volatile uint32_t* w = g_status_host;
  const uint32_t v = *w;
  if (clear) *w = 0;
  return static_cast<int64_t>(v);
}

int pi05w4a4_gemm_gelu_up_quant(const int32_t* q, const float* sa, int64_t m, int32_t k,
                                const int32_t* w_gate_mfma, const int32_t* w_up_mfma, int32_t n,
                                void* h_fp16, int32_t* dq, float* dsa, int32_t* ctl,
                                const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                                int32_t spin_limit, int32_t wait_extra, void* stream) {
  int rc = validate_gemm_common(q, sa, m, k);
  if (rc) return rc;
  rc = validate_weight(w_gate_mfma, n, "gate weight");
  if (rc) return rc;
  rc = validate_weight(w_up_mfma, n, "up weight");
  if (rc) return rc;
  if (n % 64 != 0) return fail(PI05W4A4_EINVAL, "the down-projection quant needs N %% 64 == 0, got %d", n);
  if (spin_limit < 0 || wait_extra < 0) return fail(PI05W4A4_EINVAL, "spin_limit and wait_extra must be >= 0");
  w4a4::CacheWarmParams warm;
  rc = collect_warm(warm_ptrs, warm_bytes, warm_n, &warm);
  if (rc) return rc;
  if (m == 0) return ok();
  if (h_fp16 == nullptr || dq == nullptr || dsa == nullptr || ctl == nullptr)
    return fail(PI05W4A4_EINVAL, "null output, codes, scales or control block");
  if (!aligned(h_fp16, 16) || !aligned(dq, 16) || !aligned(dsa, 4) || !aligned(ctl, 4))
    return fail(PI05W4A4_EINVAL, "h and the codes must be 16-byte aligned, scales and control block 4-byte aligned");
  if (m > 0x7fffffffLL) return fail(PI05W4A4_EINVAL, "M too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int32_t* ws[2] = {w_gate_mfma, w_up_mfma};
  const int32_t ns[2] = {n, n};
  const Plan pl = make_plan(m, k, 2, ns, true, true);
  const float inv_sqrt_n = static_cast<float>(1.0 / std::sqrt(static_cast<double>(n)));
  const bool fused = pl.cfg.id == w4a4::kCfg7x4 && pl.ksplit == 1 && n == 16384 && pl.mtiles <= 65535;
  if (!fused) {
    // Any other plan: the GEMM, then the standalone quantizer (same codes, two launches).
    void* ys[2] = {h_fp16, h_fp16};
    rc = run_gemm(q, sa, m, k, 2, ws, ns, ys, w4a4::kEpiGeluUp, nullptr, 0, st);  // no K split at N = 16384
    if (rc) return rc;
    return hip_status(w4a4::launch_quantize(h_fp16, m, n, dq, dsa, inv_sqrt_n, st, &warm), "quantize launch");
  }
  uint32_t* status = mlp_status_device_word();
  if (status == nullptr) return fail(PI05W4A4_EHIP, "gemm_gelu_up_quant: no host-visible status word");
  w4a4::GemmParams p{};
  p.q = q;
  p.sa = sa;
  p.m = m;
  p.k = k;
  p.ngroups = 2;
  p.g[0] = w4a4::GemmGroup{w_gate_mfma, h_fp16, n, 0};
  p.g[1] = w4a4::GemmGroup{w_up_mfma, h_fp16, n, static_cast<int32_t>(cdiv(n, pl.cfg.cols(false)))};
  p.ntiles = static_cast<int32_t>(pl.ntiles);
  p.mtiles = static_cast<int32_t>(pl.mtiles);
  p.ksplit = 1;
  p.kblocks_per_split = pl.kblocks;
  p.mblocks = static_cast<int32_t>(cdiv(m, 16));
  p.n_total = 2 * n;
  p.gelu_pair_n = n;
  p.mode = w4a4::kEpiGeluUp;
  p.dq = dq;
  p.dsa = dsa;
  p.qctl = ctl;
  p.qstatus = status;
  p.dinv_sqrt_k = inv_sqrt_n;
  // ~2^20 rounds of s_sleep 127 (about 4 us each): seconds, far beyond any real wait.
  p.spin_limit = spin_limit > 0 ? spin_limit : (1 << 20);
  p.wait_extra = wait_extra;
  p.warm = warm;
  const int nquant = static_cast<int>(std::min<int64_t>(m, 2 * static_cast<int64_t>(w4a4::device_cu_count())));
  return hip_status(w4a4::launch_gemm_gelu_quant(p, nquant, st), "gemm_gelu_up_quant launch");
}

int pi05w4a4_gemm_acc(const int32_t* q, int64_t m, int32_t k, const int32_t* w_mfma,
                      int32_t n, int32_t* acc, void* stream) {
  static const float kDummy = 0.0f;
  int rc = validate_gemm_common(q, &kDummy, m, k);
  if (rc) return rc;
  rc = validate_weight(w_mfma, n, "weight");
  if (rc) return rc;
  if (m > 0 && acc == nullptr) return fail(PI05W4A4_EINVAL, "null accumulator output");
  if (!aligned(acc, 4)) return fail(PI05W4A4_EINVAL, "accumulator output must be 4-byte aligned");
  if (m == 0) return ok();
  const int32_t* ws[1] = {w_mfma};
  const int32_t ns[1] = {n};
  void* ys[1] = {acc};
  return run_gemm(q, nullptr, m, k, 1, ws, ns, ys, w4a4::kEpiAcc, nullptr, 0,
                  static_cast<hipStream_t>(stream));
}

int pi05w4a4_rmsnorm(const void* x_fp16, const void* w_fp16, float eps, int32_t unit_offset,
                      int64_t m, int32_t k, void* y_fp16, void* stream) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (k <= 0 || k % 8 != 0 || k > 16384)
    return fail(PI05W4A4_EINVAL, "RMSNorm width must be a multiple of 8 up to 16384, got %d", k);
  if (m == 0) return ok();
  if (x_fp16 == nullptr || w_fp16 == nullptr || y_fp16 == nullptr)
    return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (!aligned(x_fp16, 16) || !aligned(w_fp16, 16) || !aligned(y_fp16, 16))
    return fail(PI05W4A4_EINVAL, "x, w and y must be 16-byte aligned");
  if (m > 0x7fffffffLL) return fail(PI05W4A4_EINVAL, "M too large");
  return hip_status(w4a4::launch_rmsnorm(x_fp16, w_fp16, eps, unit_offset != 0, m, k, y_fp16,
                                         static_cast<hipStream_t>(stream)),
                    "rmsnorm launch");
}


int pi05w4a4_gelu_tanh_mul(const void* gate_fp16, const void* up_fp16, int64_t n, void* y_fp16,
                            void* stream) {
  if (n < 0) return fail(PI05W4A4_EINVAL, "n must be >= 0, got %lld", (long long)n);
  if (n == 0) return ok();
  if (gate_fp16 == nullptr || up_fp16 == nullptr || y_fp16 == nullptr)
    return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (!aligned(gate_fp16, 2) || !aligned(up_fp16, 2) || !aligned(y_fp16, 2))
    return fail(PI05W4A4_EINVAL, "gate, up and y must be 2-byte aligned");
  return hip_status(w4a4::launch_gelu_up(gate_fp16, up_fp16, n, y_fp16, static_cast<hipStream_t>(stream)),
                    "gelu_tanh_mul launch");
}

size_t pi05w4a4_attn_kv_mfma_elems(int64_t b, int32_t s, int32_t kvh, int32_t d) {
  if (b < 1 || s < 1 || kvh < 1 || d < 1) return 0;
  return static_cast<size_t>(b) * kvh * 2 * d * static_cast<size_t>(w4a4::attn_s_pad(s));
}

int pi05w4a4_attn_kv_prep(const void* k, const void* v, int64_t ld_kv, const void* cos_fp16,
                          const void* sin_fp16, int64_t b, int32_t s, int32_t kvh, int32_t d,
                          void* k_rope, void* kv_mfma, void* stream) {
  int rc = validate_attention(b, s, kvh, kvh, d);
  if (rc) return rc;
  if (!k || !v || !cos_fp16 || !sin_fp16 || !k_rope || !kv_mfma) return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (ld_kv < static_cast<int64_t>(kvh) * d || ld_kv % 8 != 0)
    return fail(PI05W4A4_EINVAL, "K/V token stride must be a multiple of 8 and >= KVH*head_dim, got %lld",
                (long long)ld_kv);
  if (!aligned(k, 16) || !aligned(v, 16) || !aligned(cos_fp16, 16) || !aligned(sin_fp16, 16) ||
      !aligned(k_rope, 16) || !aligned(kv_mfma, 16))
    return fail(PI05W4A4_EINVAL, "k, v, cos, sin, k_rope and kv_mfma must be 16-byte aligned");
  w4a4::AttnParams p{};
  p.k = static_cast<const _Float16*>(k);
  p.v = static_cast<const _Float16*>(v);
  p.ld_kv = ld_kv;
  p.cosb = static_cast<const _Float16*>(cos_fp16);
  p.sinb = static_cast<const _Float16*>(sin_fp16);
  p.b = static_cast<int32_t>(b);
  p.s = s;
  p.h = kvh;
  p.kvh = kvh;
  p.s_pad = static_cast<int32_t>(w4a4::attn_s_pad(s));
  p.k_rope = static_cast<_Float16*>(k_rope);
  p.kv_mfma = static_cast<_Float16*>(kv_mfma);
  return hip_status(w4a4::launch_attn_kv_prep(p, static_cast<hipStream_t>(stream)), "attention K/V prep launch");
}

}  // extern "C"

namespace {
int prefix_attention_call(const void* q, int64_t ld_q, const void* kv_mfma, const void* cos_fp16,
                          const void* sin_fp16, const void* mask, int64_t mask_bs, int64_t mask_rs,
                          int32_t mask_len, float scaling, int64_t b, int32_t s, int32_t h, int32_t kvh,
                          int32_t d, void* out, int64_t ld_out, int32_t* q_codes, float* q_scales,
                          const w4a4::CacheWarmParams& warm, void* stream) {
  int rc = validate_attention(b, s, h, kvh, d);
  if (rc) return rc;
  if (!q || !kv_mfma || !cos_fp16 || !sin_fp16 || (!out && !q_codes))
    return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (q_codes != nullptr) {
    if (kvh != 1 || h * d != 2048)
      return fail(PI05W4A4_EINVAL, "the fused output quant takes one KV head and H * head_dim = 2048");
    if (!q_scales || !aligned(q_codes, 16) || !aligned(q_scales, 4))
      return fail(PI05W4A4_EINVAL, "q_codes must be 16-byte aligned and q_scales non-null");
  }
  if (ld_q < static_cast<int64_t>(h) * d || ld_q % 8 != 0)
    return fail(PI05W4A4_EINVAL, "query token stride must be a multiple of 8 and >= H*head_dim, got %lld",
                (long long)ld_q);
  if (out != nullptr && (ld_out < static_cast<int64_t>(h) * d || ld_out % 4 != 0))
    return fail(PI05W4A4_EINVAL, "output token stride must be a multiple of 4 and >= H*head_dim, got %lld",
                (long long)ld_out);
  if (!aligned(q, 16) || !aligned(kv_mfma, 16) || !aligned(cos_fp16, 16) ||
      !aligned(sin_fp16, 16) || (out != nullptr && !aligned(out, 8)))
    return fail(PI05W4A4_EINVAL, "q, kv_mfma, cos and sin must be 16-byte aligned, out 8-byte aligned");
  if (mask != nullptr) {
    if (mask_len < s || mask_len % 4 != 0)
      return fail(PI05W4A4_EINVAL, "mask rows must hold a multiple of 4 keys >= S, got %d", mask_len);
    if (mask_bs < 0 || mask_bs % 4 != 0 || mask_rs < mask_len || mask_rs % 4 != 0)
      return fail(PI05W4A4_EINVAL, "mask strides must be multiples of 4 (row stride >= row length)");
    if (!aligned(mask, 8)) return fail(PI05W4A4_EINVAL, "mask must be 8-byte aligned");
  }
  w4a4::AttnParams p{};
  p.q = static_cast<const _Float16*>(q);
  p.ld_q = ld_q;
  p.cosb = static_cast<const _Float16*>(cos_fp16);
  p.sinb = static_cast<const _Float16*>(sin_fp16);
  p.mask = static_cast<const _Float16*>(mask);
  p.mask_bs = mask_bs;
  p.mask_rs = mask_rs;
  p.mask_len = mask_len;
  p.scaling = scaling;
  p.b = static_cast<int32_t>(b);
  p.s = s;
  p.h = h;
  p.kvh = kvh;
  p.s_pad = static_cast<int32_t>(w4a4::attn_s_pad(s));
  p.kv_mfma = const_cast<_Float16*>(static_cast<const _Float16*>(kv_mfma));
  p.out = static_cast<_Float16*>(out);
  p.ld_out = ld_out;
  if (q_codes != nullptr) {
    const int64_t rows = b * s;
    p.qcodes = q_codes;
    p.qscales = q_scales;
    p.qcorr = q_codes + w4a4::q_payload_words((rows + 15) / 16, w4a4::kblocks128(2048));
    p.inv_sqrt_k = static_cast<float>(1.0 / std::sqrt(2048.0));
  }
  p.warm = warm;
  return hip_status(w4a4::launch_prefix_attention(p, static_cast<hipStream_t>(stream)), "prefix attention launch");
}
}  // namespace

extern "C" {

int pi05w4a4_prefix_attention(const void* q, int64_t ld_q, const void* kv_mfma,
                              const void* cos_fp16, const void* sin_fp16, const void* mask,
                              int64_t mask_bs, int64_t mask_rs, int32_t mask_len, float scaling,
                              int64_t b, int32_t s, int32_t h, int32_t kvh, int32_t d, void* out,
                              int64_t ld_out, int32_t* q_codes, float* q_scales, void* stream) {
  return prefix_attention_call(q, ld_q, kv_mfma, cos_fp16, sin_fp16, mask, mask_bs, mask_rs, mask_len, scaling, b,
                               s, h, kvh, d, out, ld_out, q_codes, q_scales, w4a4::CacheWarmParams{}, stream);
}

int pi05w4a4_prefix_attention_warm(const void* q, int64_t ld_q, const void* kv_mfma,
                                   const void* cos_fp16, const void* sin_fp16, const void* mask,
                                   int64_t mask_bs, int64_t mask_rs, int32_t mask_len, float scaling,
                                   int64_t b, int32_t s, int32_t h, int32_t kvh, int32_t d, void* out,
                                   int64_t ld_out, int32_t* q_codes, float* q_scales,
                                   const void* const* warm_ptrs, const size_t* warm_bytes, int32_t warm_n,
                                   void* stream) {
  w4a4::CacheWarmParams warm;
  const int rc = collect_warm(warm_ptrs, warm_bytes, warm_n, &warm);
  if (rc) return rc;
  return prefix_attention_call(q, ld_q, kv_mfma, cos_fp16, sin_fp16, mask, mask_bs, mask_rs, mask_len, scaling, b,
                               s, h, kvh, d, out, ld_out, q_codes, q_scales, warm, stream);
}

int pi05w4a4_int4_gemm(const void* x_fp16, int64_t m, int32_t k, const int32_t* w_mfma,
                       int32_t n, void* y_fp16, int32_t* qbuf, float* sabuf, void* workspace,
                       size_t workspace_bytes, void* stream) {
  int rc = pi05w4a4_quantize(x_fp16, m, k, qbuf, sabuf, stream);
  if (rc) return rc;
  return pi05w4a4_gemm(qbuf, sabuf, m, k, w_mfma, n, y_fp16, workspace, workspace_bytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// Allocation-free int4_gemm (pi05w4a4_int4_gemm_noalloc).  The quantized activations, their
// scales and the split-K partials of a call live in `scratch`, a fixed device array that
// the code object holds on every GPU it is loaded on, instead of caller-allocated buffers.
// In host code `scratch` names a host-side stand-in, never device memory: its device
// address is looked up once per device with hipGetSymbolAddress and only that address is
// passed to kernels.
namespace {

static __device__ __align__(256) uint8_t scratch[PI05W4A4_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (hipGetSymbolAddress on its first use
// there); sets the last error and returns null on failure.
void* scratch_for_current_device() {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(PI05W4A4_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    fail(PI05W4A4_EINVAL, "device %d is beyond the %d devices the scratch table holds", dev, kMaxScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t se = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (se != hipSuccess || ptr == nullptr) {
      fail(PI05W4A4_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(se));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

extern "C" int pi05w4a4_int4_gemm_noalloc(const void* x_fp16, int64_t m, int32_t k, const int32_t* w_mfma,
                                          int32_t n, void* y_fp16, void* stream) {
  if (m < 0) return fail(PI05W4A4_EINVAL, "M must be >= 0, got %lld", (long long)m);
  if (k <= 0 || k % 64 != 0) return fail(PI05W4A4_EINVAL, "K must be a multiple of 64, got %d", k);
  int rc = validate_weight(w_mfma, n, "weight");
  if (rc) return rc;
  if (m == 0) return ok();
  if (x_fp16 == nullptr || y_fp16 == nullptr) return fail(PI05W4A4_EINVAL, "null pointer argument");
  if (m > 0x7fffffffLL) return fail(PI05W4A4_EINVAL, "M too large");
  // Scratch layout: codes + row corrections | row scales | split-K partials, 256-byte aligned.
  const size_t q_bytes = align256(pi05w4a4_q_words(m, k) * sizeof(int32_t));
  const size_t sa_bytes = align256(static_cast<size_t>(m) * sizeof(float));
  const size_t ws_bytes = pi05w4a4_gemm_workspace_bytes(m, k, 1, &n, 0);
  const size_t need = q_bytes + sa_bytes + ws_bytes;
  if (need > PI05W4A4_NOALLOC_SCRATCH_BYTES)
    return fail(PI05W4A4_EINVAL, "M=%lld K=%d N=%d needs %zu bytes of scratch, more than the %zu the library holds",
                (long long)m, k, n, need, static_cast<size_t>(PI05W4A4_NOALLOC_SCRATCH_BYTES));
  uint8_t* base = static_cast<uint8_t*>(scratch_for_current_device());
  if (base == nullptr) return PI05W4A4_EHIP;
  int32_t* q = reinterpret_cast<int32_t*>(base);
  float* sa = reinterpret_cast<float*>(base + q_bytes);
  void* ws = ws_bytes > 0 ? static_cast<void*>(base + q_bytes + sa_bytes) : nullptr;
  // Nothing needs to start at zero: the quantizer writes every code, scale and correction
  // that the GEMM keeps (pad rows and pad k codes meet discarded rows or zero weight
  // words), and every split-K slice writes all of its partials before the reduce reads them.
  return pi05w4a4_int4_gemm(x_fp16, m, k, w_mfma, n, y_fp16, q, sa, ws, ws_bytes, stream);
}
