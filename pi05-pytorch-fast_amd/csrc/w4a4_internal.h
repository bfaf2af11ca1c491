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

struct GemmGroup {
  const int32_t* w;  // MFMA-layout payload (scales follow at w + N*K/8)
  void* y;           // fp16 [M, N] output (or int32 for kEpiAcc)
  int32_t n;         // output columns
  int32_t tile_begin;  // first global n-tile index of this group
};

struct GemmParams {
  const int32_t* q;   // int32 [M, K/8]
  const float* sa;    // fp32 [M]
  int64_t m;
  int32_t k;
  int32_t ngroups;
  GemmGroup g[kMaxGroups];
  int32_t ntiles;     // total n-tiles over the groups
  int32_t mtiles;
  int32_t ksplit;     // number of K slices
  int32_t kstages_per_split;  // 128-deep stages per K slice
  int32_t mode;
  int32_t* partial;   // workspace for kEpiPartial: [ksplit, M, n_total]
  int32_t n_total;
  int32_t gelu_pair_n;  // for kEpiGeluUp: columns of the gate (= up) weight
};

// Launchers (return hipError_t of the launch).
hipError_t launch_quantize(const void* x, int64_t m, int32_t k, int32_t* q, float* sa,
                           float inv_sqrt_k, hipStream_t stream);
hipError_t launch_repack(const int32_t* src, int32_t layout, int32_t n, int32_t k,
                         int64_t src_stride, int32_t* dst, hipStream_t stream);
// Chooses the tile configuration; returns the K split used (>= 1) through *ksplit_out.
hipError_t launch_gemm(GemmParams p, int tile_cfg, hipStream_t stream);
hipError_t launch_splitk_reduce(const GemmParams& p, hipStream_t stream);

}  // namespace w4a4
