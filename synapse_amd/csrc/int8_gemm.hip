// INT8 W8A8 prefill GEMM on the matrix cores (A4).
//
// Reference: int8GemmTiled for M > 16 (qmatmul.zig:68-99, 442-548): the
// exact i32 sum of each KC = 512 chunk of K is converted and added in chunk
// order, C += (f32(acc_chunk) * sa[i]) * sb[j].  Here K advances 64 bytes per
// step through v_mfma_i32_32x32x32_i8 (exact integer products), and every 8
// steps (one KC chunk) the i32 accumulators are folded into an f32 tile in
// that order, so the result is bit-identical to the reference.
//
// Operands: activations int8 [M, ldx] row-major; weights in the 64-row panel
// layout (linear.hpp), so a 64-byte K step of a panel is 4 contiguous 1 KiB
// chunk blocks.
#include <algorithm>

#include "linear.hpp"

namespace syn {

// ---------------------------------------------------------------------------
// Wave-specialised form.  A workgroup owns a TM x 128 tile of C (TM = 256 or
// 128): TM/32 consumer waves (TM/64 x 2, each 64 x 64 as 2 x 2 tiles of
// 32 x 32) read operand fragments from LDS and issue MFMAs;
// four producer waves keep the next kWDepth K steps of raw int8 bytes in a
// register ring and copy step t+1 into the other LDS stage while the
// consumers multiply step t.  One barrier per 128-byte K step (16 MFMAs per
// consumer wave between barriers); every 4 steps (one KC = 512 chunk) the
// consumers fold the exact i32 chunk sums into the f32 tile in chunk order,
// C += (f32(acc) * sa) * sb, as the reference does.  LDS rows are 144 bytes
// (128 + 16 pad): 16
// consecutive rows' 16-byte fragment reads land on distinct bank groups.
// Operand layout (32x32x32 i8): lane l holds row/column l%32 and K bytes
// 16*(l/32)..+15 of a 32-byte K slice; result register r of lane l is row
// 8*(r/4) + 4*(l/32) + r%4, column l%32.
constexpr int WBN = 128, WBK = 128, WLD = WBK + 16;
constexpr int WCH = WBK / 16;  // 16-byte chunks per row and step
// producer ring depth (K steps in registers): 2 for 256-row tiles, whose
// 768 threads leave 170 VGPRs a lane
template <int TM> constexpr int w_depth() { return TM == 256 ? 2 : 3; }
template <int TM> constexpr int w_stage() { return (TM + WBN) * WLD; }  // bytes per LDS stage

typedef int i32x16 __attribute__((ext_vector_type(16)));

template <int TM>
__global__ void __launch_bounds__(TM * 2 + 256)
    k_gemm_w8a8_ws(const int8_t *__restrict__ xq, int ldx, const float *__restrict__ sx, int M,
                   const i32x4 *__restrict__ W, const float *__restrict__ ws, int N, int C,
                   float *__restrict__ y, int ldy) {
  constexpr int W_STAGE = w_stage<TM>(), NC = TM / 32, AI = TM / 32, kWDepth = w_depth<TM>();
  extern __shared__ __attribute__((aligned(16))) int8_t wlds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * WBN, m0 = blockIdx.y * TM;
  const int nsteps = (C + WCH - 1) / WCH;
  const int P = (N + 63) >> 6;
  if (wave >= NC) {
    // ------------------------------------------------------------ producer
    const int pt = tid - NC * 64;  // 0..255
    // A: TM rows x 8 chunks per step, TM/32 per thread (row pt/8 + 32 i,
    // chunk pt%8); B: 128 rows x 8 chunks, four per thread (row pt%64 of
    // panel pt/128, chunks (pt/64)%2 + 2h)
    const int ac = pt & 7;
    const int8_t *arow[AI];
#pragma unroll
    for (int i = 0; i < AI; i++)
      arow[i] = xq + (size_t)min(m0 + (pt >> 3) + 32 * i, M - 1) * ldx + ac * 16;
    const int br = pt & 63, bpp = pt >> 7, bc0 = (pt >> 6) & 1;
    const int bpanel = min((n0 >> 6) + bpp, P - 1);
    const i32x4 *bsrc = W + (size_t)bpanel * C * 64 + br;
    i32x4 ra[kWDepth][AI], rb[kWDepth][4];
    auto load = [&](int slot, int t) {
      const int step = min(t, nsteps - 1);
      // an A chunk past the row's end reads the last in-bounds chunk (its
      // value is replaced by zeros when staged)
      const size_t aoff = (size_t)min(step * WCH + ac, C - 1) * 16 - (size_t)ac * 16;
#pragma unroll
      for (int i = 0; i < AI; i++)
        ra[slot][i] = *reinterpret_cast<const i32x4 *>(arow[i] + aoff);
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const int c = min(step * WCH + bc0 + 2 * h, C - 1);
        rb[slot][h] = __builtin_nontemporal_load(bsrc + (size_t)c * 64);
      }
    };
    auto stage = [&](int slot, int t, int buf) {
      int8_t *As = wlds + buf * W_STAGE, *Bs = As + TM * WLD;
      const bool a_in = t * WCH + ac < C;  // chunks past K are zero
#pragma unroll
      for (int i = 0; i < AI; i++) {
        const i32x4 v = a_in ? ra[slot][i] : i32x4{0, 0, 0, 0};
        *reinterpret_cast<i32x4 *>(&As[((pt >> 3) + 32 * i) * WLD + ac * 16]) = v;
      }
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const int c = bc0 + 2 * h;
        const i32x4 v = t * WCH + c < C ? rb[slot][h] : i32x4{0, 0, 0, 0};
        *reinterpret_cast<i32x4 *>(&Bs[(bpp * 64 + br) * WLD + c * 16]) = v;
      }
      load(slot, t + kWDepth);
    };
#pragma unroll
    for (int i = 0; i < kWDepth; i++) load(i, i);
    stage(0, 0, 0);
    __syncthreads();
    int t0 = 0;
    for (; t0 + 2 * kWDepth < nsteps; t0 += 2 * kWDepth) {
#pragma unroll
      for (int j = 0; j < 2 * kWDepth; j++) {
        stage((j + 1) % kWDepth, t0 + j + 1, (j + 1) & 1);
        __syncthreads();
      }
    }
#pragma unroll
    for (int j = 0; j < 2 * kWDepth; j++) {
      if (t0 + j < nsteps) {
        if (t0 + j + 1 < nsteps) stage((j + 1) % kWDepth, t0 + j + 1, (j + 1) & 1);
        __syncthreads();
      }
    }
    return;
  }
  // -------------------------------------------------------------- consumer
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int l32 = lane & 31, lh = lane >> 5;
  // the tile's row scales go to LDS (read at each chunk fold), the two
  // column scales of the lane stay in registers
  float *sa_l = reinterpret_cast<float *>(wlds + 2 * W_STAGE);
  if (tid < TM) sa_l[tid] = sx[min(m0 + tid, M - 1)];
  float sb[2];
#pragma unroll
  for (int nt = 0; nt < 2; nt++) sb[nt] = ws[min(n0 + wn + nt * 32 + l32, P * 64 - 1)];
  i32x16 acc[2][2];
  float cf[2][2][16];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        acc[mt][nt][r] = 0;
        cf[mt][nt][r] = 0.0f;
      }
  // fragments of one 32-byte K slice, double-buffered: the slice after the
  // current one is read while the current one's four MFMAs run
  i32x4 fa[2][2], fb[2][2];
  auto read = [&](int t, int kk, int b) {
    const int8_t *As = wlds + (t & 1) * W_STAGE, *Bs = As + TM * WLD;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
      fa[b][mt] = *reinterpret_cast<const i32x4 *>(
          &As[(wm + mt * 32 + l32) * WLD + kk * 32 + lh * 16]);
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
      fb[b][nt] = *reinterpret_cast<const i32x4 *>(
          &Bs[(wn + nt * 32 + l32) * WLD + kk * 32 + lh * 16]);
  };
  auto mma = [&](int b) {
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int nt = 0; nt < 2; nt++)
        acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[b][mt], fb[b][nt], acc[mt][nt],
                                                            0, 0, 0);
  };
  // end of a KC = 512 chunk (4 steps) or of K: C += (f32(acc)*sa)*sb
  auto fold = [&]() {
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float f = (float)acc[mt][nt][r] * sa_l[wm + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)];
          const float t = f * sb[nt];
          cf[mt][nt][r] = cf[mt][nt][r] + t;
          acc[mt][nt][r] = 0;
        }
  };
  __syncthreads();  // step 0 staged
  for (int t = 0; t < nsteps; t++) {
    read(t, 0, 0);
#pragma unroll
    for (int kk = 0; kk < WCH / 2; kk++) {
      if (kk + 1 < WCH / 2) read(t, kk + 1, (kk + 1) & 1);
      mma(kk & 1);
    }
    if (((t + 1) & 3) == 0 || t + 1 == nsteps) fold();
    __syncthreads();
  }
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
      const int n = n0 + wn + nt * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
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
  // 256-row tiles, or 128-row tiles when the larger ones cannot fill the GPU
  // (K is never split: the chunked f32 epilogue must run in chunk order)
  // two LDS stages of 128-byte K steps exceed the default 64 KiB
  static bool attr_set[2] = {false, false};
  if (cdiv(M, 256) * cdiv(N, WBN) >= 256) {
    dim3 grid((unsigned)cdiv(N, WBN), (unsigned)cdiv(M, 256));
    const size_t shm = 2 * (size_t)w_stage<256>() + 256 * sizeof(float);
    if (!attr_set[0]) {
      SYN_HIP(hipFuncSetAttribute((const void *)k_gemm_w8a8_ws<256>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
      attr_set[0] = true;
    }
    hipLaunchKernelGGL(k_gemm_w8a8_ws<256>, grid, dim3(768), shm, s, xq, (int)ldx, sx, (int)M,
                       (const i32x4 *)W, ws, (int)N, C, y, (int)ldy);
  } else {
    dim3 grid((unsigned)cdiv(N, WBN), (unsigned)cdiv(M, 128));
    const size_t shm = 2 * (size_t)w_stage<128>() + 128 * sizeof(float);
    if (!attr_set[1]) {
      SYN_HIP(hipFuncSetAttribute((const void *)k_gemm_w8a8_ws<128>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
      attr_set[1] = true;
    }
    hipLaunchKernelGGL(k_gemm_w8a8_ws<128>, grid, dim3(512), shm, s, xq, (int)ldx, sx, (int)M,
                       (const i32x4 *)W, ws, (int)N, C, y, (int)ldy);
  }
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn
