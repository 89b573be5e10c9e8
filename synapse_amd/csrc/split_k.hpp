// One-launch K split for float GEMVs at one or a few activation rows.  Every
// slice of a 64-row panel writes its f32 row sums into its own slot with a
// device-scope atomic exchange and waits for it to return: an atomic's
// return means it has been performed at the point of coherence that every
// XCD's atomics go to (plain stores and loads go through each XCD's own L2,
// and a load there can return a stale copy of a line another XCD's slice
// wrote).  The slice then counts its arrival on the panel's counter; the one
// that arrives last reads every slot back with device-scope atomic loads,
// adds them in slice order in f32 and clears the counter for the next call
// (slots are written before they are read in every call, so they need no
// clearing).  The total
// therefore does not depend on which slice finishes when (the sum order is
// fixed), and it has f32's range: no fixed-point scale limits tiny or huge
// rows, and NaN / Inf partials reach the output as they do in a plain f32
// sum.
//
// Memory order: the atomics are relaxed, with no release / acquire fences.
// Every word the slices share (slots, counters) is only ever touched by
// device-scope atomics (read-modify-writes, and the last slice's loads), and
// a slice waits for the return of
// each of its slot exchanges before its counter add is issued (the value
// dependency in sk_arrive); on gfx950 a returned device-scope RMW has been
// performed at the coherence point, where all RMWs to one address are
// ordered, and a device-scope atomic load is served there too.  So the last
// slice's loads observe every slot.  An agent-scope
// release / acquire pair would instead write back and invalidate the whole
// L2 of each XCD, at several times the kernel's cost.  A counter is left
// non-zero only by a grid that stops part way, which on this device means a
// fault that ends the context with it.
#pragma once

#include <algorithm>

#include "common.hpp"

namespace syn {

// The steps, for kernels whose threads hold several (row, activation row)
// entries: sk_put for each entry (OR the returns together), then sk_arrive
// (every thread) tells whether this workgroup is the panel's last slice,
// which then reads each entry with sk_sum and calls sk_reset once.
__device__ __forceinline__ unsigned sk_put(unsigned *slot, float v) {
  return __hip_atomic_exchange(slot, __float_as_uint(v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool sk_arrive(unsigned seen, int *cnt, int nslices, int *s_flag) {
  asm volatile("" ::"v"(seen));  // every exchange of this thread has returned
  __syncthreads();
  if (threadIdx.x == 0)
    *s_flag = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              nslices - 1;
  __syncthreads();
  return *s_flag != 0;
}
// the slots of one entry, slice 0 first, `stride` apart, added in slice
// order; the loads go out 16 at a time (clamped indices, every one issued
// before the first add), so the sum waits for one round trip per 16 slices
__device__ __forceinline__ float sk_sum(unsigned *slot0, size_t stride, int nslices) {
  float t = 0.0f;
  for (int s0 = 0; s0 < nslices; s0 += 16) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++)
      v[i] = __uint_as_float(__hip_atomic_load(slot0 + (size_t)min(s0 + i, nslices - 1) * stride,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float r = t + v[i];
      t = s0 + i < nslices ? r : t;
    }
  }
  return t;
}
__device__ __forceinline__ void sk_reset(int *cnt) {
  if (threadIdx.x == 0) __hip_atomic_exchange(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One activation row: threads tid < 64 pass the slice sum v of row tid of the
// panel (slots: the panel's slice-0 slots, `stride` floats between slices;
// slice: this workgroup's slice; cnt: the panel's counter; nslices: the
// panel's slices).  Returns, in every thread, whether this workgroup is the
// panel's last slice; then threads tid < 64 find the row's total in *tot.
// s_flag: a workgroup-shared int.
__device__ __forceinline__ bool sk_slots_last(float v, unsigned *slots, size_t stride, int slice,
                                              int *cnt, int nslices, float *tot, int *s_flag) {
  const int tid = threadIdx.x;
  const unsigned seen = tid < 64 ? sk_put(slots + (size_t)slice * stride + tid, v) : 0u;
  if (!sk_arrive(seen, cnt, nslices, s_flag)) return false;
  if (tid < 64) *tot = sk_sum(slots + tid, stride, nslices);
  sk_reset(cnt);
  return true;
}

// The slots [rows][slices][panels * 64] and counters [panels] of one handle.
// Counters are zero between calls (allocated and cleared once, outside any
// graph capture); slots are written before they are read in every call.
struct SplitKSlots {
  DevBuf part, cnt;
  int panels = 0, rows = 0, slices = 0;
  syn_status_t ensure(int panels_, int rows_, int slices_) {
    if (panels >= panels_ && rows >= rows_ && slices >= slices_) return SYN_OK;
    panels_ = std::max(panels_, panels);
    rows_ = std::max(rows_, rows);
    slices_ = std::max(slices_, slices);
    SYN_HIP(hipDeviceSynchronize());  // the old buffers may still be in use by queued work
    SYN_TRY(part.alloc((size_t)rows_ * slices_ * panels_ * 64 * sizeof(unsigned)));
    SYN_TRY(cnt.alloc((size_t)panels_ * sizeof(int)));
    SYN_HIP(hipMemset(cnt.p, 0, cnt.bytes));
    SYN_HIP(hipDeviceSynchronize());  // the memset runs on the null stream, not the caller's
    panels = panels_;
    rows = rows_;
    slices = slices_;
    return SYN_OK;
  }
  unsigned *slots() const { return part.as<unsigned>(); }
  int *counters() const { return cnt.as<int>(); }
};

}  // namespace syn
