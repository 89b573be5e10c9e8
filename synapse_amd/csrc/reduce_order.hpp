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

// One chain of the reference sum-of-squares order (syn_vmul +
// syn_vreduce_sum, exports.zig:366-375, 503-514): the sequential sum of
// sq[4i+l] over the 4-aligned prefix, for chain l in 0..3.  sq holds the
// squares of the prefix transposed (chain l contiguous at sq[l*q4 ..])
// followed by the tail squares at sq[n4 ..]; the next 32 values are loaded
// while the current 32 are added.
__device__ __forceinline__ float sumsq_chain(const float *sq, int n, int l) {
  const int n4 = n & ~3, q4 = n4 >> 2;
  const float *p = sq + l * q4;
  float acc = 0.0f;
  int i = 0;
  if (q4 > 0 && (q4 & 31) == 0) {
    const float4 *p4 = reinterpret_cast<const float4 *>(p);
    const int groups = q4 >> 5;
    float4 a[8];
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = p4[k];
    for (int gi = 0; gi < groups; gi++) {
      const int nx = min(gi + 1, groups - 1) * 8;
      float4 b[8];
#pragma unroll
      for (int k = 0; k < 8; k++) b[k] = p4[nx + k];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        acc = acc + a[k].x;
        acc = acc + a[k].y;
        acc = acc + a[k].z;
        acc = acc + a[k].w;
      }
#pragma unroll
      for (int k = 0; k < 8; k++) a[k] = b[k];
    }
    i = q4;
  } else if ((q4 & 3) == 0) {
    for (; i + 16 <= q4; i += 16) {
      const float4 a = *reinterpret_cast<const float4 *>(p + i);
      const float4 b = *reinterpret_cast<const float4 *>(p + i + 4);
      const float4 c = *reinterpret_cast<const float4 *>(p + i + 8);
      const float4 d = *reinterpret_cast<const float4 *>(p + i + 12);
      acc = acc + a.x; acc = acc + a.y; acc = acc + a.z; acc = acc + a.w;
      acc = acc + b.x; acc = acc + b.y; acc = acc + b.z; acc = acc + b.w;
      acc = acc + c.x; acc = acc + c.y; acc = acc + c.z; acc = acc + c.w;
      acc = acc + d.x; acc = acc + d.y; acc = acc + d.z; acc = acc + d.w;
    }
  }
  for (; i < q4; i++) acc = acc + p[i];
  return acc;
}

// the four chain results combined as ((a0+a1)+a2)+a3, then the tail in order
__device__ __forceinline__ float sumsq_combine(const float *r4, const float *sq, int n) {
  float s = ((r4[0] + r4[1]) + r4[2]) + r4[3];
  for (int i = n & ~3; i < n; i++) s = s + sq[i];
  return s;
}

// The whole reference-order sum of squares: lanes 0-3 run the chains, every
// thread gets the result.  Callers place a barrier between writing sq and
// this call; red[32..35] is used.
template <int NT>
__device__ float sumsq_chains(const float *sq, int n, float *red) {
  if (threadIdx.x < 4) red[32 + threadIdx.x] = sumsq_chain(sq, n, threadIdx.x);
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

// Sequential sum of v[0..n) (a single accumulator, in index order).
__device__ __forceinline__ float seq_sum(const float *v, int n) {
  float s = 0.0f;
  int i = 0;
  if ((reinterpret_cast<uintptr_t>(v) & 15) == 0) {
    for (; i + 16 <= n; i += 16) {
      const float4 a = *reinterpret_cast<const float4 *>(v + i);
      const float4 b = *reinterpret_cast<const float4 *>(v + i + 4);
      const float4 c = *reinterpret_cast<const float4 *>(v + i + 8);
      const float4 d = *reinterpret_cast<const float4 *>(v + i + 12);
      s = s + a.x; s = s + a.y; s = s + a.z; s = s + a.w;
      s = s + b.x; s = s + b.y; s = s + b.z; s = s + b.w;
      s = s + c.x; s = s + c.y; s = s + c.z; s = s + c.w;
      s = s + d.x; s = s + d.y; s = s + d.z; s = s + d.w;
    }
  }
  for (; i < n; i++) s = s + v[i];
  return s;
}

// The same sequential sum with its LDS reads double-buffered: the next 16
// values are requested while the current 16 are added (v 16-byte aligned).
__device__ __forceinline__ float seq_sum_pipelined(const float *v, int n) {
  const float4 *v4 = reinterpret_cast<const float4 *>(v);
  const int nb = n >> 4;  // whole blocks of 16
  float s = 0.0f;
  float4 a[4];
#pragma unroll
  for (int k = 0; k < 4; k++) a[k] = v4[k];
  for (int b = 0; b < nb; b++) {
    float4 c[4];
    const int nx = min(b + 1, max(nb - 1, 0)) * 4;
#pragma unroll
    for (int k = 0; k < 4; k++) c[k] = v4[nx + k];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      s = s + a[k].x;
      s = s + a[k].y;
      s = s + a[k].z;
      s = s + a[k].w;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) a[k] = c[k];
  }
  for (int i = nb * 16; i < n; i++) s = s + v[i];
  return s;
}

}  // namespace syn
