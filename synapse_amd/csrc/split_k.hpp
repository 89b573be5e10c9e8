// One-launch K split for float GEMVs at one activation row.  Every slice of
// a 64-row panel adds its row sums as int64 fixed point (kqf_fix, value *
// 2^32) into the panel's accumulators with device-scope atomics and waits for
// them to return: an atomic's return means it has been performed at the point
// of coherence that every XCD's atomics go to.  The slice then counts its
// arrival on the panel's counter; the one that arrives last reads the totals
// back by atomic exchange with 0 and clears the counter, so the buffers are
// zero again for the next call.  Fixed-point sums are exact in any order, so
// the result does not depend on which slice finishes when.
#pragma once

#include <algorithm>

#include "common.hpp"

namespace syn {

// The steps, for kernels whose threads hold several (row, activation row)
// entries: sk_add for each entry (OR the returns together), then sk_arrive
// (every thread) tells whether this workgroup is the panel's last slice,
// which then reads each entry with sk_take and calls sk_reset once.
__device__ __forceinline__ unsigned long long sk_add(unsigned long long *p, float v) {
  return __hip_atomic_fetch_add(p, (unsigned long long)kqf_fix(v), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool sk_arrive(unsigned long long seen, int *cnt, int nslices,
                                          int *s_flag) {
  asm volatile("" ::"v"(seen));  // every add of this thread has returned
  __syncthreads();
  if (threadIdx.x == 0)
    *s_flag = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              nslices - 1;
  __syncthreads();
  return *s_flag != 0;
}
__device__ __forceinline__ float sk_take(unsigned long long *p) {
  return kqf_unfix(
      (long long)__hip_atomic_exchange(p, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void sk_reset(int *cnt) {
  if (threadIdx.x == 0) __hip_atomic_exchange(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One activation row: threads tid < 64 pass the slice sum v of row tid of the
// panel (acc, cnt: that panel's 64 accumulators and its counter; nslices:
// the panel's slices).  Returns, in every thread, whether this workgroup is
// the panel's last slice; then threads tid < 64 find the row's total in
// *tot.  s_flag: a workgroup-shared int.
__device__ __forceinline__ bool sk_fixed_last(float v, unsigned long long *acc, int *cnt,
                                              int nslices, float *tot, int *s_flag) {
  const int tid = threadIdx.x;
  const unsigned long long seen = tid < 64 ? sk_add(acc + tid, v) : 0ull;
  if (!sk_arrive(seen, cnt, nslices, s_flag)) return false;
  if (tid < 64) *tot = sk_take(acc + tid);
  sk_reset(cnt);
  return true;
}

// The accumulators [rows][panels * 64] and counters [panels] of one handle,
// zero between calls (allocated and cleared once, outside any graph capture)
struct SplitKFixed {
  DevBuf acc, cnt;
  int panels = 0, rows = 0;
  syn_status_t ensure(int panels_, int rows_ = 1) {
    if (panels >= panels_ && rows >= rows_) return SYN_OK;
    panels_ = std::max(panels_, panels);
    rows_ = std::max(rows_, rows);
    SYN_HIP(hipDeviceSynchronize());  // the old buffers may still be in use by queued work
    SYN_TRY(acc.alloc((size_t)rows_ * panels_ * 64 * sizeof(long long)));
    SYN_TRY(cnt.alloc((size_t)panels_ * sizeof(int)));
    SYN_HIP(hipMemset(acc.p, 0, acc.bytes));
    SYN_HIP(hipMemset(cnt.p, 0, cnt.bytes));
    SYN_HIP(hipDeviceSynchronize());  // the memsets run on the null stream, not the caller's
    panels = panels_;
    rows = rows_;
    return SYN_OK;
  }
  unsigned long long *acc_panel(int p) const {
    return reinterpret_cast<unsigned long long *>(acc.p) + (size_t)p * 64;
  }
};

}  // namespace syn
