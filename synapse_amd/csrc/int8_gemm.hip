// INT8 W8A8 prefill GEMM on the matrix cores (A4).
//
// Reference: int8GemmTiled for M > 16 (qmatmul.zig:68-99, 442-548): the
// exact i32 sum of each KC = 512 chunk of K is converted and added in chunk
// order, C += (f32(acc_chunk) * sa[i]) * sb[j].  Here each workgroup owns a
// 128 x 128 tile of C; K advances 64 bytes per step through
// v_mfma_i32_16x16x64_i8 (exact integer products), and every 8 steps (one KC
// chunk) the i32 accumulators are folded into an f32 tile in that order.
//
// Operands: activations int8 [M, ldx] row-major; weights in the 64-row panel
// layout (linear.hpp), so a 64-byte K step of a panel is 4 contiguous 1 KiB
// chunk blocks.  LDS holds A [128][64] and B [128][64] (+16 B row padding).
// Lane mapping (16x16x64): lane l supplies row/col l%16 and K bytes
// 16*(l/16)..+15 of both operands; the 4 result registers of lane l are rows
// 4*(l/16)+r, column l%16.
#include <algorithm>

#include "linear.hpp"

namespace syn {

constexpr int GBM = 128, GBN = 128, GBK = 64, GPAD = 16, GLD = GBK + GPAD;

__global__ void __launch_bounds__(256)
    k_gemm_w8a8(const int8_t *__restrict__ xq, int ldx, const float *__restrict__ sx, int M,
                const i32x4 *__restrict__ W, const float *__restrict__ ws, int N, int C,
                float *__restrict__ y, int ldy) {
  __shared__ __attribute__((aligned(16))) int8_t As[GBM * GLD];
  __shared__ __attribute__((aligned(16))) int8_t Bs[GBN * GLD];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * GBM;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int P = (N + 63) >> 6;
  const int nsteps = (C + 3) >> 2;
  const int lr = lane & 15, lg = lane >> 4;

  float sa[4][4], sb[4];
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = m0 + wm + mt * 16 + 4 * lg + r;
      sa[mt][r] = m < M ? sx[m] : 0.0f;
    }
#pragma unroll
  for (int nt = 0; nt < 4; nt++) {
    const int n = n0 + wn + nt * 16 + lr;
    sb[nt] = n < N ? ws[n] : 0.0f;
  }

  i32x4 acc[4][4];
  float cf[4][4][4];
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      acc[mt][nt] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; r++) cf[mt][nt][r] = 0.0f;
    }

  // global -> register staging for one K step (2 x 16 B per thread per operand)
  i32x4 ga[2], gb[2];
  auto fetch = [&](int step) {
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int idx = tid + it * 256;
      const int r = idx >> 2, cc = idx & 3;
      const int row = m0 + r, kb = step * GBK + cc * 16;
      ga[it] = i32x4{0, 0, 0, 0};
      if (row < M && kb < ldx) ga[it] = *reinterpret_cast<const i32x4 *>(xq + (size_t)row * ldx + kb);
      const int br = idx & 63, bc = (idx >> 6) & 3, pp = idx >> 8;
      const int panel = (n0 >> 6) + pp, chunk = step * 4 + bc;
      gb[it] = i32x4{0, 0, 0, 0};
      if (panel < P && chunk < C) gb[it] = __builtin_nontemporal_load(W + ((size_t)panel * C + chunk) * 64 + br);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int idx = tid + it * 256;
      *reinterpret_cast<i32x4 *>(&As[(idx >> 2) * GLD + (idx & 3) * 16]) = ga[it];
      const int br = idx & 63, bc = (idx >> 6) & 3, pp = idx >> 8;
      *reinterpret_cast<i32x4 *>(&Bs[(pp * 64 + br) * GLD + bc * 16]) = gb[it];
    }
  };

  fetch(0);
  for (int step = 0; step < nsteps; step++) {
    __syncthreads();  // previous step's LDS reads are done
    stash();
    __syncthreads();
    if (step + 1 < nsteps) fetch(step + 1);  // overlaps the MFMAs below
    i32x4 a[4], b[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
      a[mt] = *reinterpret_cast<const i32x4 *>(&As[(wm + mt * 16 + lr) * GLD + lg * 16]);
#pragma unroll
    for (int nt = 0; nt < 4; nt++)
      b[nt] = *reinterpret_cast<const i32x4 *>(&Bs[(wn + nt * 16 + lr) * GLD + lg * 16]);
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
      for (int nt = 0; nt < 4; nt++)
        acc[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
    if (((step + 1) & 7) == 0 || step + 1 == nsteps) {  // end of a KC=512 chunk
#pragma unroll
      for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float f = (float)acc[mt][nt][r] * sa[mt][r];
            const float t = f * sb[nt];
            cf[mt][nt][r] = cf[mt][nt][r] + t;
          }
          acc[mt][nt] = i32x4{0, 0, 0, 0};
        }
    }
  }
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const int n = n0 + wn + nt * 16 + lr;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm + mt * 16 + 4 * lg + r;
        if (m < M && n < N) y[(size_t)m * ldy + n] = cf[mt][nt][r];
      }
    }
}

syn_status_t launch_gemm_w8a8(const int8_t *xq, size_t ldx, const float *sx, size_t M,
                              const void *W, const float *ws, size_t N, int C, float *y,
                              size_t ldy, hipStream_t s) {
  if (ldx % 16) {
    set_error("activation row stride must be a multiple of 16 bytes");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  dim3 grid((unsigned)cdiv(N, GBN), (unsigned)cdiv(M, GBM));
  hipLaunchKernelGGL(k_gemm_w8a8, grid, dim3(256), 0, s, xq, (int)ldx, sx, (int)M,
                     (const i32x4 *)W, ws, (int)N, C, y, (int)ldy);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn
