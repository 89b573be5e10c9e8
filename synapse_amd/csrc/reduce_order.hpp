// Reductions in the reference's floating-point order, shared by the device
// kernels: the sum of squares of syn_vmul + syn_vreduce_sum
// (exports.zig:366-375, 503-514) and plain sequential sums.
#pragma once

#include "common.hpp"

namespace syn {

template <int NT>
__device__ __forceinline__ void bar() {
  if constexpr (NT > 64) __syncthreads();
  else __builtin_amdgcn_wave_barrier();
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Makes the registers of `a` an input and output of an empty asm statement:
// every load that produces them completes before this point, and no
// arithmetic that uses them moves ahead of it.  A dependent add chain that
// follows then runs from registers (one VALU op every ~4.7 clocks) instead
// of waiting for an LDS read every few operations (~20 clocks each).
template <int N>
__device__ __forceinline__ void pin_regs(f32x4 (&a)[N]) {
#pragma unroll
  for (int i = 0; i < N; i++) asm volatile("" : "+v"(a[i]));
}

// acc + v[0] + v[1] + ... + v[n-1], added one at a time in index order (v
// in LDS, 16-byte aligned, readable up to round_up4(n)).  The values pass
// through registers in blocks of 32; the reads of the next block are issued
// before the adds of the current one, so the chain never waits for LDS.
__device__ __forceinline__ float lds_seq_sum(const float *v, int n, float acc) {
  const f32x4 *v4 = reinterpret_cast<const f32x4 *>(v);
  const int nb = n >> 5;
  f32x4 a[8], b[8];
  auto load = [&](f32x4(&r)[8], int blk) {
#pragma unroll
    for (int k = 0; k < 8; k++) r[k] = v4[blk * 8 + k];
  };
  auto add = [&](f32x4(&r)[8]) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      acc = acc + r[k].x;
      acc = acc + r[k].y;
      acc = acc + r[k].z;
      acc = acc + r[k].w;
    }
  };
  int blk = 0;
  if (nb > 0) {
    load(a, 0);
    for (; blk + 1 < nb; blk += 2) {
      load(b, blk + 1);
      __builtin_amdgcn_sched_barrier(0);
      pin_regs(a);
      add(a);
      load(a, min(blk + 2, nb - 1));  // in bounds; unused past the end
      __builtin_amdgcn_sched_barrier(0);
      pin_regs(b);
      add(b);
    }
    if (blk < nb) {
      pin_regs(a);
      add(a);
    }
  }
  // the last n % 32 values: one batch of reads (up to round_up4(n), which
  // the callers' buffers hold), then the adds of the valid ones
  const int rem = n - nb * 32;
  if (rem > 0) {
    const int ng = (rem + 3) >> 2;
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = v4[nb * 8 + min(k, ng - 1)];
    pin_regs(a);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float c[4] = {a[k].x, a[k].y, a[k].z, a[k].w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float r = acc + c[j];
        acc = k * 4 + j < rem ? r : acc;
      }
    }
  }
  return acc;
}

// One chain of the reference sum-of-squares order (syn_vmul +
// syn_vreduce_sum, exports.zig:366-375, 503-514): the sequential sum of
// sq[4i+l] over the 4-aligned prefix, for chain l in 0..3.  sq holds the
// squares of the prefix transposed (chain l contiguous at sq[l*q4 ..])
// followed by the tail squares at sq[n4 ..]; sq is 16-byte aligned.
__device__ __forceinline__ float sumsq_chain(const float *sq, int n, int l) {
  const int n4 = n & ~3, q4 = n4 >> 2;
  const float *p = sq + l * q4;
  if ((q4 & 3) == 0) return lds_seq_sum(p, q4, 0.0f);  // chain start stays 16-byte aligned
  float acc = 0.0f;
  for (int i = 0; i < q4; i++) acc = acc + p[i];
  return acc;
}

// the four chain results combined as ((a0+a1)+a2)+a3, then the tail in order
__device__ __forceinline__ float sumsq_combine(const float *r4, const float *sq, int n) {
  float s = ((r4[0] + r4[1]) + r4[2]) + r4[3];
  for (int i = n & ~3; i < n; i++) s = s + sq[i];
  return s;
}

// The four chains of sumsq_chain at once on one wave, chain l on the lanes
// of 16-lane row l, from registers: lane j of the row holds values 16j ..
// 16j+15 of each 256-value pass; the running sum visits the row's lanes in
// order (lane j adds its 16 values, then a DPP row_ror:1 hands the sum to
// lane j+1), so every add is one dependent VALU op and no LDS read sits in
// the chain (the sumsq_chain form reads its values from LDS in blocks of 32
// between the adds).  Same adds in the same order.  Requires q4 = n/4
// rounded down to be a multiple of 4 (16-byte aligned chains); returns chain
// l's sum in every lane of row l.  Call with all 64 lanes of the wave.
__device__ __forceinline__ float sumsq_chain_rows(const float *sq, int n) {
  const int lane = threadIdx.x & 63, l = lane >> 4, j = lane & 15;
  const int q4 = (n & ~3) >> 2;
  const float *p = sq + l * q4;
  auto rot = [](float x) {  // lane j <- lane j-1 of the same 16-lane row
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf,
                                                      false));
  };
  float acc = 0.0f;
  for (int base = 0; base < q4; base += 256) {
    f32x4 r[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = min(base + 16 * j + 4 * k, (q4 - 1) & ~3);  // in bounds; unused past q4
      r[k] = *reinterpret_cast<const f32x4 *>(p + i);
    }
    pin_regs(r);
    const int left = min(q4 - base, 256), full = left >> 4;
    for (int t = 0; t < full; t++) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        acc = acc + r[k].x;
        acc = acc + r[k].y;
        acc = acc + r[k].z;
        acc = acc + r[k].w;
      }
      acc = rot(acc);
    }
    if (left & 15) {  // the last, partial turn
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const float c[4] = {r[k].x, r[k].y, r[k].z, r[k].w};
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (4 * k + i < (left & 15)) acc = acc + c[i];
      }
      acc = rot(acc);
    }
    // the pass's sum sits in the row's lane after its last turn
    acc = __shfl(acc, (l << 4) | (((left + 15) >> 4) & 15));
  }
  return acc;
}

// The whole reference-order sum of squares: the four chains on wave 0
// (sumsq_chain_rows, or lanes 0-3 reading LDS when the chains are not
// 16-byte aligned), every thread gets the result.  Callers place a barrier
// between writing sq and this call; red[32..35] is used.
template <int NT>
__device__ float sumsq_chains(const float *sq, int n, float *red) {
  if (((n >> 2) & 3) == 0) {
    if (threadIdx.x < 64) {
      const float s = sumsq_chain_rows(sq, n);
      if ((threadIdx.x & 15) == 0) red[32 + (threadIdx.x >> 4)] = s;
    }
  } else if (threadIdx.x < 4) {
    red[32 + threadIdx.x] = sumsq_chain(sq, n, threadIdx.x);
  }
  bar<NT>();
  return sumsq_combine(red + 32, sq, n);
}

// where the square of element j goes in the sumsq_chains layout
__device__ __forceinline__ int sq_slot(int j, int n) {
  const int n4 = n & ~3;
  return j < n4 ? (j & 3) * (n4 >> 2) + (j >> 2) : j;
}

// Sum of squares of v[0..n) held in LDS, reference order.
template <int NT>
__device__ float sumsq_lds(const float *v, int n, float *sq, float *red) {
  for (int j = threadIdx.x; j < n; j += NT) {
    const float x = v[j];
    sq[sq_slot(j, n)] = x * x;
  }
  bar<NT>();
  return sumsq_chains<NT>(sq, n, red);
}

// acc0 + v[0] + ... + v[n-1] one at a time in index order, run by a whole
// wave (v in LDS, 16-byte aligned, readable up to round_up4(n)).  Lane l
// holds v[16l .. 16l+16) of each 1024-value pass in registers; the running sum visits the lanes in order:
// lane l adds its 16 values, then a DPP wave_ror:1 hands the sum to lane l+1
// (lane 63 to lane 0 for the next pass).  Every add is one dependent VALU
// op of the wave (the other lanes' sums are discarded), so the chain runs
// at the register rate with no memory access inside it.  Values at index
// >= n are skipped by a select.  Returns the sum in every lane.
__device__ __forceinline__ float wave_seq_sum(const float *v, int n, float acc0) {
  const int lane = threadIdx.x & 63;
  float acc = acc0;
  auto rot = [](float x) {  // lane l+1 <- lane l, lane 0 <- lane 63
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x13C, 0xf, 0xf,
                                                      false));
  };
  for (int base = 0; base < n; base += 1024) {
    f32x4 r[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int j = min(base + 16 * lane + 4 * k, (n - 1) & ~3);  // in bounds; unused past n
      r[k] = *reinterpret_cast<const f32x4 *>(v + j);
    }
    pin_regs(r);
    const int left = min(n - base, 1024), full = left >> 4;
    for (int l = 0; l < full; l++) {  // turns of 16 values
#pragma unroll
      for (int k = 0; k < 4; k++) {
        acc = acc + r[k].x;
        acc = acc + r[k].y;
        acc = acc + r[k].z;
        acc = acc + r[k].w;
      }
      acc = rot(acc);
    }
    if (left & 15) {  // the last, partial turn
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const float c[4] = {r[k].x, r[k].y, r[k].z, r[k].w};
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (4 * k + i < (left & 15)) acc = acc + c[i];
      }
      acc = rot(acc);
    }
    // the pass's sum now sits in the lane after its last turn
    const int turns = (left + 15) >> 4;
    acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), turns & 63));
  }
  return acc;
}

// wave_seq_sum for long rows (a model width, ~1024 values): the same adds in
// the same order (v in LDS, 16-byte aligned, readable up to round_up4(n)).
// Lane j of each 16-lane row holds v[64j .. 64j+64) of each 1024-value pass
// in registers; lane j adds its 64 values, then a DPP row_ror:1 hands the
// sum to lane j+1 (lane 15 to lane 0 for the next pass): 16 hand-offs per
// pass instead of wave_seq_sum's 64 wave-wide rotates (~31 cycles each,
// which made a 1024-long chain 7.0 cycles per add against 5.0 for the adds
// alone).  Short rows keep wave_seq_sum: their partial turn would run 64
// guarded adds instead of 16.  Returns the sum in every lane.
__device__ __forceinline__ float wave_seq_sum_long(const float *v, int n, float acc0) {
  const int j = threadIdx.x & 15;
  float acc = acc0;
  auto rot = [](float x) {  // lane j+1 <- lane j of the same row, lane 0 <- lane 15
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf,
                                                      false));
  };
  for (int base = 0; base < n; base += 1024) {
    f32x4 r[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int i = min(base + 64 * j + 4 * k, (n - 1) & ~3);  // in bounds; unused past n
      r[k] = *reinterpret_cast<const f32x4 *>(v + i);
    }
    pin_regs(r);
    const int left = min(n - base, 1024), full = left >> 6;
    for (int t = 0; t < full; t++) {  // turns of 64 values
#pragma unroll
      for (int k = 0; k < 16; k++) {
        acc = acc + r[k].x;
        acc = acc + r[k].y;
        acc = acc + r[k].z;
        acc = acc + r[k].w;
      }
      acc = rot(acc);
    }
    if (left & 63) {  // the last, partial turn
#pragma unroll
      for (int k = 0; k < 16; k++) {
        const float c[4] = {r[k].x, r[k].y, r[k].z, r[k].w};
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (4 * k + i < (left & 63)) acc = acc + c[i];
      }
      acc = rot(acc);
    }
    // the pass's sum now sits in the row's lane after its last turn
    const int turns = (left + 63) >> 6;
    acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), turns & 15));
  }
  return acc;
}

// Sequential sum of v[0..n) (a single accumulator, in index order).
__device__ __forceinline__ float seq_sum(const float *v, int n) {
  if ((reinterpret_cast<uintptr_t>(v) & 15) == 0) return lds_seq_sum(v, n, 0.0f);
  float s = 0.0f;
  for (int i = 0; i < n; i++) s = s + v[i];
  return s;
}

// The same sequential sum (v 16-byte aligned).
__device__ __forceinline__ float seq_sum_pipelined(const float *v, int n) {
  return lds_seq_sum(v, n, 0.0f);
}

}  // namespace syn
