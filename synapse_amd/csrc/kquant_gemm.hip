// Prefill GEMM for the GGUF block formats on the f16 matrix cores (A12/A13).
//
// The reference runs these formats as f32 sgemmTiled over weights
// dequantized at load (ops/matmul.rs:55-79, matmul.zig:157-183).  Here a
// workgroup owns a 128 x 128 tile of Y = X W^T and walks K 32 elements at a
// time (one Q8_0 block / one Q4_K sub-block / two Q6_K sub-blocks): the
// weight tile is decoded once per workgroup from the HBM plane layout into
// f16 in LDS (value = the reference dequantizer's f32 value rounded to f16),
// activations are pre-converted to f16, and v_mfma_f32_16x16x32_f16
// accumulates in f32.  The two f16 roundings (relative 2^-11 each) keep the
// result well inside the 1e-3 per-row tolerance (measured in the tests).
#include <algorithm>

#include "kquant.hpp"

namespace syn {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int QBM = 128, QBN = 128, QBK = 32, QLD = QBK + 8;  // LDS row stride in halfs

__global__ void k_f32_to_f16(const float *__restrict__ x, int ldx, _Float16 *__restrict__ xh,
                             int ldh, int M, int K) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = K / 4;
  if (i >= M * per_row) return;
  const int m = i / per_row, c = (i - m * per_row) * 4;
  const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)m * ldx + c);
  _Float16 *o = xh + (size_t)m * ldh + c;
  o[0] = (_Float16)v.x;
  o[1] = (_Float16)v.y;
  o[2] = (_Float16)v.z;
  o[3] = (_Float16)v.w;
}

// Decode 16 consecutive weights (k = 16*half .. +15 of K step ks) of row n.
template <int FMT>
__device__ __forceinline__ void kq_decode16(const u32x4 *__restrict__ W,
                                            const uint16_t *__restrict__ Wd, int B, int n, int N,
                                            int ks, int half, _Float16 *out) {
  if (n >= N) {
#pragma unroll
    for (int i = 0; i < 16; i++) out[i] = (_Float16)0.0f;
    return;
  }
  const size_t panel = (size_t)(n >> 6), rp = (size_t)(n & 63);
  if (FMT == SYN_HIP_FMT_Q8_0) {
    const size_t blk = (size_t)ks;
    const float d = syn_f16_to_f32_rs(Wd[(panel * B + blk) * 64 + rp]);
    const u32x4 q = W[((panel * B + blk) * 2 + half) * 64 + rp];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float v = d * (float)(int8_t)(w[i >> 2] >> (8 * (i & 3)));  // gguf.rs:283
      out[i] = (_Float16)v;
    }
  } else if (FMT == SYN_HIP_FMT_Q4_K) {
    const size_t sb = (size_t)(ks >> 3);
    const int s = ks & 7;
    const u32x4 h = W[((panel * B + sb) * 9 + 0) * 64 + rp];
    const u32x4 q = W[((panel * B + sb) * 9 + 1 + s) * 64 + rp];
    const float d = syn_f16_to_f32_rs(h.x & 0xffffu), dmin = syn_f16_to_f32_rs(h.x >> 16);
    const uint32_t sbw[3] = {h.y, h.z, h.w};
    auto SB = [&](int i) -> uint32_t { return (sbw[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    uint32_t sc, mn;
    if (s < 4) {
      sc = SB(s) & 63u;
      mn = ((SB(s + 4) >> 4) | ((SB(s + 8) & 15u) << 4)) & 0xffu;
    } else {
      sc = (SB(s) & 15u) | ((SB(s - 4) >> 6) << 4);
      mn = ((SB(s + 4) >> 4) | (((SB(s - 4) >> 4) & 12u) << 4)) & 0xffu;
    }
    const float scf = d * (float)sc, mf = dmin * (float)mn;  // gguf.rs:416-417
    // elements 16*half + 2i, +2i+1 <- byte 8*half + i (low, high nibble)
    const uint32_t w0 = half ? q.z : q.x, w1 = half ? q.w : q.y;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t byte = ((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xffu;
      const float lo = (float)(byte & 15u) * scf - mf;  // gguf.rs:424-425
      const float hi = (float)(byte >> 4) * scf - mf;
      out[2 * i] = (_Float16)lo;
      out[2 * i + 1] = (_Float16)hi;
    }
  } else {  // Q6_K: K step ks covers sub-blocks 2j, 2j+1 of superblock ks/8
    const size_t sb = (size_t)(ks >> 3);
    const int j = ks & 7, s = 2 * j + half;
    const u32x4 ql = W[((panel * B + sb) * 13 + (s >> 1)) * 64 + rp];
    const u32x4 qh = W[((panel * B + sb) * 13 + 8 + (s >> 2)) * 64 + rp];
    const u32x4 sc = W[((panel * B + sb) * 13 + 12) * 64 + rp];
    const float d = syn_f16_to_f32_rs(Wd[(panel * B + sb) * 64 + rp]);
    const uint32_t lo0 = (s & 1) ? ql.z : ql.x, lo1 = (s & 1) ? ql.w : ql.y;
    const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
    const uint32_t hi = hw[s & 3];
    const uint32_t sw[4] = {sc.x, sc.y, sc.z, sc.w};
    const float scale = (float)(int8_t)(sw[s >> 2] >> (8 * (s & 3))) * d;  // gguf.rs:466
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t lo = ((i < 8 ? lo0 : lo1) >> (4 * (i & 7))) & 15u;
      const uint32_t h2 = (hi >> (2 * i)) & 3u;
      const float qv = (float)((int)(lo | (h2 << 4)) - 32);
      out[i] = (_Float16)(qv * scale);  // gguf.rs:480-481
    }
  }
}

template <int FMT>
__global__ void __launch_bounds__(256)
    k_gemm_kq(const _Float16 *__restrict__ Xh, int ldh, int M, int K,
              const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd, int N, int B,
              float *__restrict__ Y, int ldy) {
  __shared__ __attribute__((aligned(16))) _Float16 As[QBM * QLD];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[QBN * QLD];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * QBN, m0 = blockIdx.y * QBM;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int lr = lane & 15, lg = lane >> 4;
  const int ksteps = K / QBK;
  f32x4 acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // A: 128 rows x 32 halfs = 512 x 16 B, two per thread
  u32x4 ga[2];
  auto fetch_a = [&](int ks) {
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int idx = tid + it * 256, r = idx >> 2, c = (idx & 3) * 8;
      ga[it] = u32x4{0u, 0u, 0u, 0u};
      if (m0 + r < M)
        ga[it] = *reinterpret_cast<const u32x4 *>(Xh + (size_t)(m0 + r) * ldh + ks * QBK + c);
    }
  };
  _Float16 wb[16];
  const int brow = tid >> 1, bhalf = tid & 1;

  fetch_a(0);
  kq_decode16<FMT>(W, Wd, B, n0 + brow, N, 0, bhalf, wb);
  for (int ks = 0; ks < ksteps; ks++) {
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int idx = tid + it * 256;
      *reinterpret_cast<u32x4 *>(&As[(idx >> 2) * QLD + (idx & 3) * 8]) = ga[it];
    }
#pragma unroll
    for (int i = 0; i < 16; i++) Bs[brow * QLD + bhalf * 16 + i] = wb[i];
    __syncthreads();
    if (ks + 1 < ksteps) {  // next step's loads and decode overlap the MFMAs
      fetch_a(ks + 1);
      kq_decode16<FMT>(W, Wd, B, n0 + brow, N, ks + 1, bhalf, wb);
    }
    f16x8 a[4], b[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
      a[mt] = *reinterpret_cast<const f16x8 *>(&As[(wm + mt * 16 + lr) * QLD + lg * 8]);
#pragma unroll
    for (int nt = 0; nt < 4; nt++)
      b[nt] = *reinterpret_cast<const f16x8 *>(&Bs[(wn + nt * 16 + lr) * QLD + lg * 8]);
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
      for (int nt = 0; nt < 4; nt++)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
  }
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const int n = n0 + wn + nt * 16 + lr;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm + mt * 16 + 4 * lg + r;
        if (m < M && n < N) Y[(size_t)m * ldy + n] = acc[mt][nt][r];
      }
    }
}

syn_status_t QLinearKQ::gemm(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                             hipStream_t s) {
  if (ldx % 4) {
    set_error("GEMM activation stride must be a multiple of 4 floats");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  const size_t ldh = k;  // k is a multiple of 32
  if (xh_elems < m * ldh) {
    SYN_HIP(hipDeviceSynchronize());
    SYN_TRY(xh.alloc(m * ldh * 2));
    xh_elems = m * ldh;
  }
  const int total = (int)(m * (k / 4));
  hipLaunchKernelGGL(k_f32_to_f16, dim3(cdiv(total, 256)), dim3(256), 0, s, d_x, (int)ldx,
                     xh.as<_Float16>(), (int)ldh, (int)m, (int)k);
  SYN_LAUNCH_CHECK();
  dim3 grid((unsigned)cdiv(n, QBN), (unsigned)cdiv(m, QBM));
  const u32x4 *W = wq.as<u32x4>();
  const uint16_t *Wd = wd.as<uint16_t>();
  const _Float16 *X = xh.as<_Float16>();
  if (fmt == SYN_HIP_FMT_Q8_0)
    hipLaunchKernelGGL(k_gemm_kq<SYN_HIP_FMT_Q8_0>, grid, dim3(256), 0, s, X, (int)ldh, (int)m,
                       (int)k, W, Wd, (int)n, blocks, d_y, (int)ldy);
  else if (fmt == SYN_HIP_FMT_Q4_K)
    hipLaunchKernelGGL(k_gemm_kq<SYN_HIP_FMT_Q4_K>, grid, dim3(256), 0, s, X, (int)ldh, (int)m,
                       (int)k, W, Wd, (int)n, blocks, d_y, (int)ldy);
  else
    hipLaunchKernelGGL(k_gemm_kq<SYN_HIP_FMT_Q6_K>, grid, dim3(256), 0, s, X, (int)ldh, (int)m,
                       (int)k, W, Wd, (int)n, blocks, d_y, (int)ldy);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn
