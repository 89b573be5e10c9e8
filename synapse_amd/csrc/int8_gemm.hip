// INT8 W8A8 prefill GEMM on the matrix cores (A4).
//
// Reference: int8GemmTiled for M > 16 (qmatmul.zig:68-99, 442-548): the
// exact i32 sum of each KC = 512 chunk of K is converted and added in chunk
// order, C += (f32(acc_chunk) * sa[i]) * sb[j].  Here K advances 128 bytes
// per step through v_mfma_i32_32x32x32_i8 (exact integer products), and every
// 4 steps (one KC chunk) the i32 accumulators are folded into an f32 tile in
// that order, so the result is bit-identical to the reference.  Two forms:
// k_gemm_w8a8_dl (direct global->LDS loads; K a multiple of 128) and
// k_gemm_w8a8_ws (producer waves staging through registers; any K).
//
// Operands: activations int8 [M, ldx] row-major; weights in the 64-row panel
// layout (linear.hpp), so a 128-byte K step of a panel is 8 contiguous 1 KiB
// chunk blocks.
#include <algorithm>
#include <type_traits>

#include "linear.hpp"
#include "lds_dma.hpp"

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

// ---------------------------------------------------------------------------
// Direct-load form, for K a multiple of 128.  2 WR waves own a TM x TN tile
// of C; wave (wr, wc) the (TM/WR) x (TN/2) sub-tile at rows wr*TM/WR,
// columns wc*TN/2, as (TM/WR/32) x (TN/64) MFMA tiles of 32 x 32, so every
// 16-byte fragment read from LDS feeds that many MFMAs.  Both operands go from
// global memory straight into LDS (gfx950 global_load_lds_dwordx4: no
// staging registers, no ds_write), NS 128-byte K steps deep:
//  - activations as TM rows of 128 bytes; the eight 16-byte chunks of row r
//    sit XOR-swizzled (chunk c at slot c ^ ((r / 2) % 8)): the 64 banks of
//    4 bytes span two rows, and the fragment reads of 16 consecutive rows
//    hit 16 distinct 16-byte bank groups (with c ^ (r % 8), rows r and r + 8
//    collide: 31 % of the LDS cycles were bank conflicts);
//  - weights as stored, [panel][chunk][64 rows][16 bytes]: one 1 KiB direct
//    load per (panel, chunk), read back conflict-free.
// One barrier per step; the i32 sums of each KC = 512 chunk (4 steps) are
// folded into the f32 tile as in k_gemm_w8a8_ws: after the chunk's last
// step, or (DF) from a second accumulator set, four elements per step
// between the next chunk's MFMAs, so that the fold's VALU work overlaps the
// matrix cores (every fold still adds the chunks in order).  NS stages: the loads run
// NS - 1 steps ahead (3 stages of the 128 x 128 tile keep a second
// workgroup off the CU).  WR = 4 gives two waves per SIMD in one workgroup,
// which is what hides the per-step barrier and the LDS waits (WR = 2 with a
// single workgroup per CU leaves one wave per SIMD).
template <int TM, int TN> constexpr int dl_stage() { return (TM + TN) * 128; }
template <int TM, int TN, int NS> constexpr size_t dl_lds_bytes() {
  return (size_t)NS * dl_stage<TM, TN>() + TM * sizeof(float);
}

template <int TM, int TN, int NS, int WR, bool DF>
__global__ void __launch_bounds__(128 * WR)
    k_gemm_w8a8_dl(const int8_t *__restrict__ xq, int ldx, const float *__restrict__ sx, int M,
                   const i32x4 *__restrict__ W, const float *__restrict__ ws, int N, int C,
                   float *__restrict__ y, int ldy) {
  constexpr int NWAVE = 2 * WR, WM = TM / WR, WN = TN / 2, MT = WM / 32, NT = WN / 32;
  constexpr int LA = TM / 8 / NWAVE, LB = TN / 8 / NWAVE;  // direct loads per wave and step
  static_assert(LA * NWAVE * 8 == TM && LB * NWAVE * 8 == TN, "whole loads per wave");
  constexpr int A_BYTES = TM * 128, STAGE = dl_stage<TM, TN>(), AFTER = LA + LB;
  extern __shared__ __attribute__((aligned(16))) int8_t dlds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, lh = lane >> 5, wr = wave >> 1, wc = wave & 1;
  const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
  const int nsteps = C >> 3;
  const int last_panel = (N - 1) >> 6;
  // activation load i of this wave: rows 8 (wave * LA + i) .. + 7, lane l
  // bringing chunk (l % 8) ^ ((row / 2) % 8) of row 8 (wave * LA + i) + l / 8
  // into slot l % 8; rows past M read row M - 1 (never stored)
  uint32_t aoff[LA];
#pragma unroll
  for (int i = 0; i < LA; i++) {
    const int row = (wave * LA + i) * 8 + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
    aoff[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)ldx + (uint32_t)c * 16u;
  }
  // weight load j of this wave: q = wave * LB + j is (panel q / 8 of the
  // tile, clamped to the matrix's last; chunk q % 8 of the step)
  const i32x4 *wsrc[LB];
#pragma unroll
  for (int j = 0; j < LB; j++) {
    const int q = wave * LB + j;
    const size_t panel = (size_t)min((n0 >> 6) + (q >> 3), last_panel);
    wsrc[j] = W + (panel * C + (q & 7)) * 64 + lane;
  }
  const uint32_t lds_base = lds_addr_of(dlds);
  auto dma = [&](int t, int stage) {
    const int step = min(t, nsteps - 1);
    const uint32_t sb = lds_base + (uint32_t)(stage * STAGE);
    const uint32_t wa = (uint32_t)__builtin_amdgcn_readfirstlane(wave * LA * 1024);
    const uint32_t wb = (uint32_t)__builtin_amdgcn_readfirstlane(A_BYTES + wave * LB * 1024);
#pragma unroll
    for (int i = 0; i < LA; i++)
      kr_dma(xq + aoff[i] + (size_t)step * 128, sb + wa + (uint32_t)(i * 1024));
#pragma unroll
    for (int j = 0; j < LB; j++)
      kr_dma(wsrc[j] + (size_t)step * 8 * 64, sb + wb + (uint32_t)(j * 1024));
  };
#pragma unroll
  for (int i = 0; i < NS; i++) dma(i, i);

  // row scales of the tile through LDS (into registers after the first
  // barrier), the lane's column scales in registers
  float *sa_l = reinterpret_cast<float *>(dlds + NS * STAGE);
  if (tid < TM) sa_l[tid] = sx[min(m0 + tid, M - 1)];
  float sb[NT];
#pragma unroll
  for (int nt = 0; nt < NT; nt++)
    sb[nt] = ws[min(n0 + wc * WN + nt * 32 + l32, (last_panel + 1) * 64 - 1)];
  // two accumulator sets: chunk c adds into acc[c % 2] while the fold of
  // chunk c - 1 (VALU) runs between its MFMAs
  i32x16 acc[2][MT][NT];
  float cf[MT][NT][16];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        acc[0][mt][nt][r] = 0;
        acc[1][mt][nt][r] = 0;
        cf[mt][nt][r] = 0.0f;
      }
  // fragment addresses inside a stage: A row (wr*WM + mt*32 + l32), whose
  // swizzle is (l32 / 2) % 8; B panel col / 64, row col % 64 of column
  // wc*WN + nt*32 + l32
  const int arow = (wr * WM + l32) * 128, asw = (l32 >> 1) & 7;
  int boff[NT];
#pragma unroll
  for (int nt = 0; nt < NT; nt++) {
    const int col = wc * WN + nt * 32 + l32;
    boff[nt] = A_BYTES + (col >> 6) * 8 * 1024 + (col & 63) * 16;
  }
  i32x4 fa[2][MT], fb[2][NT];
  auto read = [&](int stage, int kk, int b) {
    const int8_t *st = dlds + stage * STAGE;
    const int c = 2 * kk + lh;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
      fa[b][mt] = *reinterpret_cast<const i32x4 *>(st + arow + mt * 32 * 128 + ((c ^ asw) << 4));
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
      fb[b][nt] = *reinterpret_cast<const i32x4 *>(st + boff[nt] + c * 1024);
  };
  auto mma = [&](auto Pc, const i32x4 (&a)[MT], const i32x4 (&b)[NT]) {
    constexpr int P = decltype(Pc)::value;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int nt = 0; nt < NT; nt++)
        acc[P][mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mt], b[nt], acc[P][mt][nt],
                                                               0, 0, 0);
  };
  // fold of accumulator element r of set Q: C += (f32(acc) * sa) * sb, and
  // the element starts the set's next chunk at zero
  // the row scales of the fold in registers, except with three stages,
  // whose 256 VGPRs then spill (13 against 3; 256 x 4096 x 16384: 992-999
  // TOP/s with them in registers against 1032-1044 from LDS)
  constexpr bool kSar = DF && NS < 3;
  float sar[MT][16];
  auto fold_el = [&](auto Qc, int r) {
    constexpr int Q = decltype(Qc)::value;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int nt = 0; nt < NT; nt++) {
        const float sa = kSar ? sar[mt][r] : sa_l[wr * WM + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)];
        const float f = (float)acc[Q][mt][nt][r] * sa;
        const float t = f * sb[nt];
        cf[mt][nt][r] = cf[mt][nt][r] + t;
        acc[Q][mt][nt][r] = 0;
      }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using NoFold = std::false_type;
  using Fold = std::true_type;

  // Step t lives in stage t % NS.  Step t: K slices 0-2 (each beside the
  // reads of the next slice); the barrier that publishes step t+1 (and the
  // row scales, before the first); the load of step t+NS into the stage
  // step t has left; step t+1's slice 0 reads beside step t's slice 3
  // (clamped, unused data after the last step).  Step s of a chunk also
  // folds elements 4s .. 4s+3 of the other set (the previous chunk), one
  // after each slice's MFMAs.
  auto step = [&](int t, int s, auto Pc, auto Fc) {
    constexpr int P = decltype(Pc)::value;
    constexpr bool F = decltype(Fc)::value;
    using Q = std::integral_constant<int, 1 - P>;
    const int cur = t % NS, nxt = cur == NS - 1 ? 0 : cur + 1;
#pragma unroll
    for (int kk = 0; kk < 3; kk++) {
      read(cur, kk + 1, (kk + 1) & 1);
      mma(Pc, fa[kk & 1], fb[kk & 1]);
      if constexpr (F) fold_el(Q{}, 4 * s + kk);
    }
    kr_publish<(NS - 2) * AFTER>();
    dma(t + NS, cur);
    i32x4 a3[MT], b3[NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) a3[mt] = fa[1][mt];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) b3[nt] = fb[1][nt];
    read(nxt, 0, 0);
    mma(Pc, a3, b3);
    if constexpr (F) fold_el(Q{}, 4 * s + 3);
  };
  // whole chunk c (steps 4c .. 4c+3) into set P, folding the other set
  // (the previous chunk) when F
  auto chunk = [&](int c, auto Pc, auto Fc) {
#pragma unroll
    for (int s = 0; s < 4; s++) step(4 * c + s, s, Pc, Fc);
  };
  auto fold_all = [&](auto Qc) {
#pragma unroll
    for (int r = 0; r < 16; r++) fold_el(Qc, r);
  };
  // a last, shorter chunk c into set P: the previous chunk's fold first
  auto tail = [&](int c, auto Pc) {
    using Q = std::integral_constant<int, 1 - decltype(Pc)::value>;
    if (c > 0) fold_all(Q{});
    for (int t = 4 * c; t < nsteps; t++) step(t, 0, Pc, NoFold{});
    fold_all(Pc);
  };

  kr_publish<(NS - 1) * AFTER>();
  if constexpr (kSar) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        sar[mt][r] = sa_l[wr * WM + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)];
  }
  read(0, 0, 0);
  if constexpr (!DF) {
    // one accumulator set, folded after each chunk's last step (element
    // order mt, nt, r)
    auto fold1 = [&]() {
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const float f = (float)acc[0][mt][nt][r] *
                            sa_l[wr * WM + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)];
            const float t = f * sb[nt];
            cf[mt][nt][r] = cf[mt][nt][r] + t;
            acc[0][mt][nt][r] = 0;
          }
    };
    for (int t = 0; t < nsteps; t++) {
      step(t, 0, P0{}, NoFold{});
      if (((t + 1) & 3) == 0 || t + 1 == nsteps) fold1();
    }
  } else {
    const int nfull = nsteps >> 2;
    int c = 0;
    if (nfull > 0) {
      chunk(0, P0{}, NoFold{});
      for (c = 1; c + 1 < nfull; c += 2) {
        chunk(c, P1{}, Fold{});
        chunk(c + 1, P0{}, Fold{});
      }
      if (c < nfull) {
        chunk(c, P1{}, Fold{});
        c++;
      }
    }
    // c == nfull: set (nfull - 1) % 2 holds the last whole chunk
    if (nsteps & 3) {
      if (c & 1)
        tail(c, P1{});
      else
        tail(c, P0{});
    } else if (c & 1) {
      fold_all(P0{});
    } else if (c > 0) {
      fold_all(P1{});
    }
  }
  // the prefetches past the last step must land before the workgroup's LDS
  // can go to another workgroup
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
      const int n = n0 + wc * WN + nt * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wr * WM + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < M && n < N) y[(size_t)m * ldy + n] = cf[mt][nt][r];
      }
    }
}

template <int TM, int TN, int NS, int WR, bool DF>
static syn_status_t launch_w8a8_dl(const int8_t *xq, size_t ldx, const float *sx, size_t M,
                                   const void *W, const float *ws, size_t N, int C, float *y,
                                   size_t ldy, hipStream_t s) {
  static bool attr_set = false;  // more than the default 64 KiB of dynamic LDS
  constexpr size_t shm = dl_lds_bytes<TM, TN, NS>();
  if (!attr_set) {
    SYN_HIP(hipFuncSetAttribute((const void *)k_gemm_w8a8_dl<TM, TN, NS, WR, DF>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
    attr_set = true;
  }
  const dim3 grid((unsigned)cdiv(N, TN), (unsigned)cdiv(M, TM));
  SYN_LAUNCH((k_gemm_w8a8_dl<TM, TN, NS, WR, DF>), grid, dim3(128 * WR), shm, s, xq, (int)ldx, sx, (int)M,
             (const i32x4 *)W, ws, (int)N, C, y, (int)ldy);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

syn_status_t launch_gemm_w8a8(const int8_t *xq, size_t ldx, const float *sx, size_t M,
                              const void *W, const float *ws, size_t N, int C, float *y,
                              size_t ldy, hipStream_t s) {
  if (ldx % 16) {
    set_error("activation row stride must be a multiple of 16 bytes");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  // K is never split: the chunked f32 epilogue must run in chunk order.
  // Direct-load tiles when K is whole 128-byte steps (the loads cannot
  // zero a K tail) and the byte offsets fit 32 bits, eight waves (2 x 4
  // sub-tiles) on 128 x 128 when that gives every CU a workgroup: three
  // stages when the tiles fit one workgroup per CU, else two (two
  // workgroups per CU); else 128 x 64 with eight waves and four stages when
  // that gives every CU a workgroup, else 64 x 64 with four stages (two
  // workgroups per CU).  Measured (int8 TOPS): 2048 x 4096 x 4096 1351-1354
  // with eight waves and two stages against 1185-1232 with four waves,
  // 2048 x 14336 x 4096 1298-1357 against 1236-1290, 512 x 14336 x 4096
  // 1339-1344 against 1248 (with four waves there is one wave per SIMD per
  // workgroup: little hides the barriers and LDS waits); 1024 x 4096 x 4096
  // (256 tiles) 1151-1154 with three stages against 926-932 with two;
  // earlier, 256 x 128 tiles 968 (four waves) and 1201 (eight), 988 for
  // k_gemm_w8a8_ws.  512 x 4096 x 4096 787-798 against 695-708 for 128 x
  // 64 with four waves and three stages (more stages alone did not help),
  // 767-773 with eight waves and three, 767-779 for 64 x 64; 128 x 3072 x
  // 1024 119 for 64 x 64 against 110 and 93.  The fold of a chunk runs
  // under the next chunk's MFMAs (DF) where one workgroup's waves are all
  // a SIMD has: 512 x 4096 x 4096 936-943 against 785-793, 1024 x 4096 x
  // 4096 1158-1164 against 1097-1105 (three stages; 1005-1037 with two),
  // 128 x 3072 x 1024 128 against 122.  With two workgroups per CU the other
  // workgroup hides the fold, and DF's second accumulator set (221 VGPRs
  // on 128 x 128) would leave room for one: 2048 x 4096 x 4096 1047-1076
  // with DF and three stages, 1033-1103 with two.
  if (C % 8 == 0 && (uintptr_t)xq % 16 == 0 && M * ldx < ((size_t)1 << 31)) {
    const size_t tiles = cdiv(M, 128) * cdiv(N, 128);
    if (tiles == 256)
      return launch_w8a8_dl<128, 128, 3, 4, true>(xq, ldx, sx, M, W, ws, N, C, y, ldy, s);
    if (tiles > 256)
      return launch_w8a8_dl<128, 128, 2, 4, false>(xq, ldx, sx, M, W, ws, N, C, y, ldy, s);
    if (cdiv(M, 128) * cdiv(N, 64) >= 256)
      return launch_w8a8_dl<128, 64, 4, 4, true>(xq, ldx, sx, M, W, ws, N, C, y, ldy, s);
    return launch_w8a8_dl<64, 64, 4, 2, true>(xq, ldx, sx, M, W, ws, N, C, y, ldy, s);
  }
  // otherwise 256-row tiles, or 128-row tiles when the larger ones cannot
  // fill the GPU
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
