// Cache warming: workgroups that a launch would leave without work read device buffers
// and discard the data, so that the kernels after it find them in the memory-side
// Infinity Cache (256 MB) instead of HBM.
#pragma once

#include "w4a4_internal.h"

namespace w4a4 {

// Slice `part` of `nparts` of the buffers in w, read by a THREADS-thread workgroup with 8
// loads of 16 bytes in flight per thread; the data feed an empty asm.  The eight loads are
// written as one asm block each and always issued (indices past the buffer are clamped to
// its last word), then awaited together: with the compiler's own code for guarded loads the
// 776-token forward took 2.366-2.369 ms against 2.341-2.342 (one box, three rounds; with
// clamped loads in plain C++ 2.373-2.379).
template <int THREADS>
__device__ __forceinline__ void cache_warm_part(const CacheWarmParams& w, int64_t part, int64_t nparts, int tid) {
  constexpr int kLoads = 8;
  const int64_t stride = nparts * THREADS * kLoads;
  uint32_t acc = 0;
#pragma unroll 1
  for (int bi = 0; bi < w.nbuf; ++bi) {
    const uint4* src = static_cast<const uint4*>(w.ptr[bi]);
    const int64_t n = w.n16[bi];
    for (int64_t base = part * THREADS * kLoads + tid; base < n; base += stride) {
      typedef int v4i_w __attribute__((ext_vector_type(4)));
      v4i_w v[kLoads];
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int64_t idx = min(base + static_cast<int64_t>(i) * THREADS, n - 1);
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v[i]) : "v"(src + idx) : "memory");
      }
      // The asm loads are invisible to the compiler's counters: wait for them here.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < kLoads; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
  }
  asm volatile("" ::"v"(acc));
}

}  // namespace w4a4
