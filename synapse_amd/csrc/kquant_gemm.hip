// Prefill GEMM for the GGUF block formats on the f16 matrix cores (A12/A13).
//
// The reference runs these formats as f32 sgemmTiled over weights
// dequantized at load (ops/matmul.rs:55-79, matmul.zig:157-183); Q4_0 rows
// run q4_0GemvRow one row at a time (q4_linear.rs:126-150).  Here a
// workgroup owns a 256 x 256 tile of Y = X W^T (four waves, k_gemm_kq5; used
// when such tiles cover three quarters of the CUs) or a 256 x 128 tile
// (twelve waves, k_gemm_kq2, split over K for small grids) and walks K 64
// elements at a time: the weight tile is decoded once per workgroup from the
// HBM plane layout into f16 in LDS (value = the reference dequantizer's f32
// value rounded to f16), activations are pre-converted to f16, and
// v_mfma_f32_32x32x16_f16 accumulates in f32.  Q4_0 on large grids runs
// k_gemm_kqr instead: both operands reach LDS by direct global->LDS loads
// and each wave decodes its weight fragments in registers.  The two f16 roundings
// (relative 2^-11 each) keep the result well inside the 1e-3 per-row
// tolerance (measured in the tests).
#include <algorithm>
#include <type_traits>

#include "decode_fused.hpp"
#include "kquant.hpp"
#include "lds_dma.hpp"

namespace syn {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// x f32 [M, ldx] -> xh f16 [M, ldh], columns K..ldh-1 zero (K a multiple of
// 8, ldh of 64, ldx of 4), one workgroup per row.  Each row is scaled by a
// power of two that puts its largest magnitude in [2^14, 2^15) before the
// f16 rounding, and rowmul[m] holds the inverse power for the GEMM epilogue:
// rows far above f16's range (which would round to inf) or far below it
// (subnormal f16, lost precision) keep f16's full relative precision, and
// both scalings are exact in f32.  A row whose maximum is zero or not finite
// is not scaled.  perm8: each 8-element chunk is stored in the k order
// 0,2,4,6,1,3,5,7 of the Q4_0 direct-load kernel's fragments (k_gemm_kqr).
// y0 (when not null): row m of the GEMM's output [M, ldy] is cleared (its
// first ny floats; ldy a multiple of 4, y0 16-byte aligned) for a K-split
// GEMM that adds its partial tiles into it, saving a kernel of its own.
__global__ void __launch_bounds__(256)
    k_f32_to_f16(const float *__restrict__ x, int ldx, _Float16 *__restrict__ xh, int ldh,
                 float *__restrict__ rowmul, int K, int perm8, float *__restrict__ y0, int ldy,
                 int ny) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const float *xr = x + (size_t)m * ldx;
  if (y0) {
    float4 *yr = reinterpret_cast<float4 *>(y0 + (size_t)m * ldy);
    for (int c = tid; c < ny / 4; c += 256) yr[c] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = (ny & ~3) + tid; c < ny; c += 256) y0[(size_t)m * ldy + c] = 0.0f;
  }
  float mx = 0.0f;
  for (int c = tid * 4; c < K; c += 1024) {
    const float4 a = *reinterpret_cast<const float4 *>(xr + c);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float up = 1.0f, down = 1.0f;  // x * up rounds to f16; y * down undoes it
  if (mx > 0.0f && mx <= 3.4028235e38f) {
    int e;
    (void)frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
    up = ldexpf(1.0f, 15 - e);
    down = ldexpf(1.0f, e - 15);
  }
  if (tid == 0) rowmul[m] = down;
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  for (int c = tid * 8; c < ldh; c += 2048) {
    float4 a = float4{0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (c < K) {
      a = *reinterpret_cast<const float4 *>(xr + c);
      b = *reinterpret_cast<const float4 *>(xr + c + 4);
    }
    a.x *= up; a.y *= up; a.z *= up; a.w *= up;
    b.x *= up; b.y *= up; b.z *= up; b.w *= up;
    const h8 o = perm8 ? h8{(_Float16)a.x, (_Float16)a.z, (_Float16)b.x, (_Float16)b.z,
                            (_Float16)a.y, (_Float16)a.w, (_Float16)b.y, (_Float16)b.w}
                       : h8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                            (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    *reinterpret_cast<h8 *>(xh + (size_t)m * ldh + c) = o;
  }
}

// The row multipliers (rowmul) of a lane's epilogue rows in MFMA tile mt,
// requested together before the tile's stores (a load per element, each
// waited for before its multiply, put ~64 dependent L2 round trips into
// every lane's epilogue): row mbase + mt*32 + 8*(r/4) + 4*lh + r%4 for
// accumulator r, clamped in bounds (rows past M are not stored)
__device__ __forceinline__ void load_rowmul(const float *__restrict__ rowmul, int mbase, int lh,
                                            int M, float (&rm)[16]) {
#pragma unroll
  for (int r = 0; r < 16; r++)
    rm[r] = rowmul[min(mbase + 8 * (r >> 2) + 4 * lh + (r & 3), M - 1)];
}

// ---------------------------------------------------------------------------
// Tiling.  A workgroup owns a 256 x 128 tile of Y and walks its K range 64
// elements per step through two LDS stages of A [256][72] and B [128][72]
// f16.  Weights are decoded from the HBM plane layout into f16 (the reference
// dequantizer's value rounded once to f16); loads are unconditional from
// clamped (in-bounds) rows and steps.  Shapes with fewer tiles than the GPU
// has CUs split K over the grid's z dimension and add their partial tiles
// with f32 atomics into a zeroed Y.
constexpr int PGM = 256, PGN = 128, PGK = 64, PGLD = PGK + 8;  // LDS row stride in halfs

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// (d as a 16-bit field: held as a 32-bit value, the ring's copies at the
// producer loop's back edge zero-extended each pending scale load, and the
// wait for it drained the ring every iteration)
struct RawW {
  u32x4 q0, q1, q2;  // quant planes (format-dependent)
  uint16_t d;        // f16 bits of the block scale (Q8_0, Q6_K)
};

__device__ __forceinline__ uint32_t u32x4_word(const u32x4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// elements 16q .. 16q+15 of step `step` of row n (q = 0..3)
template <int FMT>
__device__ __forceinline__ void pg_load_w(RawW &r, const u32x4 *__restrict__ W,
                                          const uint16_t *__restrict__ Wd, int B, int n, int step,
                                          int q) {
  const size_t panel = (size_t)(n >> 6), rp = (size_t)(n & 63);
  if (FMT == SYN_HIP_FMT_Q8_0) {  // block 2*step + q/2 (clamped, see pg_decode_w), plane q%2
    const size_t blk = (size_t)min(2 * step + (q >> 1), B - 1);
    r.q0 = W[((panel * B + blk) * 2 + (q & 1)) * 64 + rp];
    r.d = Wd[(panel * B + blk) * 64 + rp];
  } else if (FMT == SYN_HIP_FMT_Q4_0) {  // block 2*step + q/2 (clamped), its one nibble plane
    const size_t blk = (size_t)min(2 * step + (q >> 1), B - 1);
    r.q0 = W[(panel * B + blk) * 64 + rp];
    r.d = Wd[(panel * B + blk) * 64 + rp];
  } else if (FMT == SYN_HIP_FMT_Q4_K) {  // sub-block 2*(step%4) + q/2, nibble bytes 8*(q%2)..+7
    const size_t sb = (size_t)(step >> 2);
    const int sub = 2 * (step & 3) + (q >> 1);
    r.q0 = W[((panel * B + sb) * 9 + 0) * 64 + rp];
    r.q1 = W[((panel * B + sb) * 9 + 1 + sub) * 64 + rp];
  } else {  // Q6_K: elements e0 = 64*(step%4) + 16q .. +15 of superblock step/4
    const size_t sb = (size_t)(step >> 2);
    const int st = step & 3;
    r.q0 = W[((panel * B + sb) * 13 + 2 * st + (q >> 1)) * 64 + rp];  // ql bytes
    r.q1 = W[((panel * B + sb) * 13 + 8 + st) * 64 + rp];             // qh bytes
    r.q2 = W[((panel * B + sb) * 13 + 12) * 64 + rp];                 // scales
    r.d = Wd[(panel * B + sb) * 64 + rp];
  }
}

// the 16 weights as 8 f16 pairs (element order), each the reference
// dequantizer's f32 value (gguf.rs:255-487) rounded once to f16.  Q8_0 with K
// % 64 == 32: the block past the row's end decodes to zeros, against the
// zero padding of the activations.
template <int FMT, bool EXACT>
__device__ __forceinline__ void pg_decode_w(const RawW &r, int step, int q, int B,
                                            uint32_t (&out)[8]) {
  if (FMT == SYN_HIP_FMT_Q8_0) {
    const bool valid = 2 * step + (q >> 1) < B;
    const float d = valid ? syn_f16_to_f32_rs_hw(r.d) : 0.0f;
    if (EXACT) {
      // every scale of the matrix is an f16 value (checked at upload), and
      // d*q is exact in f32 (11 x 8 significant bits), so rounding it to f16
      // equals one f16 multiply of the exact f16 values d and q; q comes from
      // the byte as f16(1024 + (q ^ 0x80)) - 1152, built with byte permutes
      const _Float16 dh = (_Float16)d;
      const f16x2 dd = f16x2{dh, dh}, bias = f16x2{(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t u = u32x4_word(r.q0, w) ^ 0x80808080u;
        const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
        const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
        const f16x2 v01 = (__builtin_bit_cast(f16x2, p01) + bias) * dd;
        const f16x2 v23 = (__builtin_bit_cast(f16x2, p23) + bias) * dd;
        out[2 * w] = __builtin_bit_cast(uint32_t, v01);
        out[2 * w + 1] = __builtin_bit_cast(uint32_t, v23);
      }
    } else {  // some scale is not an f16 value (a halved subnormal): f32 products
#pragma unroll
      for (int i = 0; i < 8; i++) {
        f16x2 v;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int e = 2 * i + h;
          const uint32_t w = u32x4_word(r.q0, e >> 2);
          v[h] = (_Float16)(d * (float)(int8_t)(w >> (8 * (e & 3))));  // gguf.rs:283
        }
        out[i] = __builtin_bit_cast(uint32_t, v);
      }
    }
  } else if (FMT == SYN_HIP_FMT_Q4_0) {
    // Q4Linear blocks (q4_linear.rs:64-121): element 2i = low nibble of byte
    // i, 2i+1 = high; value = (nibble - 8) * d.  nibble - 8 and d are exact
    // f16 values, so one f16 multiply rounds the exact product once.  The
    // pair (1024 + lo, 1024 + hi) of byte i comes from a byte permute.
    const bool valid = 2 * step + (q >> 1) < B;
    const _Float16 dh = valid ? __builtin_bit_cast(_Float16, (uint16_t)r.d) : (_Float16)0.0f;
    const f16x2 dd = f16x2{dh, dh}, bias = f16x2{(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
    for (int w = 0; w < 2; w++) {
      const uint32_t v = u32x4_word(r.q0, 2 * (q & 1) + w);
      const uint32_t lo = v & 0x0f0f0f0fu, hi = (v >> 4) & 0x0f0f0f0fu;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        // bytes: lo.b, 0, hi.b, 0 -> halfs 0x64 lo.b, 0x64 hi.b
        const uint32_t sel = (uint32_t)b | (0x0cu << 8) | ((uint32_t)(4 + b) << 16) | (0x0cu << 24);
        const uint32_t pr = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
        const f16x2 val = (__builtin_bit_cast(f16x2, pr) + bias) * dd;
        out[4 * w + b] = __builtin_bit_cast(uint32_t, val);
      }
    }
  } else if (FMT == SYN_HIP_FMT_Q4_K) {
    const int s = 2 * (step & 3) + (q >> 1);
    const float d = syn_f16_to_f32_rs_hw(r.q0.x & 0xffffu), dmin = syn_f16_to_f32_rs_hw(r.q0.x >> 16);
    const uint32_t sbw[3] = {r.q0.y, r.q0.z, r.q0.w};
    auto SB = [&](int i) -> uint32_t { return (sbw[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    // gguf.rs:383-399 for sub-block s (both branches evaluated, one selected)
    const int sl = s & 3;
    const uint32_t sc_lo = SB(sl) & 63u;
    const uint32_t mn_lo = ((SB(sl + 4) >> 4) | ((SB(sl + 8) & 15u) << 4)) & 0xffu;
    const uint32_t sc_hi = (SB(sl + 4) & 15u) | ((SB(sl) >> 6) << 4);
    const uint32_t mn_hi = ((SB(sl + 8) >> 4) | (((SB(sl) >> 4) & 12u) << 4)) & 0xffu;
    const uint32_t sc = s < 4 ? sc_lo : sc_hi, mn = s < 4 ? mn_lo : mn_hi;
    const float scf = d * (float)sc, mf = dmin * (float)mn;  // gguf.rs:416-417
#pragma unroll
    for (int i = 0; i < 8; i++) {  // element 2i: low nibble of byte i, 2i+1: high
      const int bi = 8 * (q & 1) + i;
      const uint32_t byte = (u32x4_word(r.q1, bi >> 2) >> (8 * (bi & 3))) & 0xffu;
      const float lo = (float)(byte & 15u) * scf - mf;  // gguf.rs:424-425
      const float hi = (float)(byte >> 4) * scf - mf;
      out[i] = __builtin_bit_cast(uint32_t, f16x2{(_Float16)lo, (_Float16)hi});
    }
  } else {
    const int st = step & 3;
    const float d = syn_f16_to_f32_rs_hw(r.d);
    // ql byte (e0+i)/2 = plane byte 8*(q%2) + i/2, nibble i%2; qh byte
    // (e0+i)/4 = plane byte 4q + i/4, bits 2*(i%4); scale (e0+i)/16 = 4st + q
    const int si = 4 * st + q;
    const float scale = (float)(int8_t)(u32x4_word(r.q2, si >> 2) >> (8 * (si & 3))) * d;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      f16x2 v;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int e = 2 * i + h;
        const int lb = 8 * (q & 1) + (e >> 1);
        const uint32_t qlb = (u32x4_word(r.q0, lb >> 2) >> (8 * (lb & 3))) & 0xffu;
        const uint32_t lo = (e & 1) ? (qlb >> 4) : (qlb & 15u);
        const int hb = 4 * q + (e >> 2);
        const uint32_t qhb = (u32x4_word(r.q1, hb >> 2) >> (8 * (hb & 3))) & 0xffu;
        const uint32_t h2 = (qhb >> (2 * (e & 3))) & 3u;
        const float qv = (float)((int)(lo | (h2 << 4)) - 32);
        v[h] = (_Float16)(qv * scale);  // gguf.rs:480-481
      }
      out[i] = __builtin_bit_cast(uint32_t, v);
    }
  }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// LDS: two stages of A [TM][72] and B [128][72] f16 (110,592 bytes for
// TM = 256, 73,728 for 128: two workgroups per CU)
template <int TM> constexpr int pg_stage() { return (TM + PGN) * PGLD; }

// ---------------------------------------------------------------------------
// Wave-specialised form: TM/32 consumer waves and 4 producers (12 waves for
// TM = 256, 8 for 128).  The consumer waves ((TM/64) x 2, each a 64 x 64
// sub-tile of the TM x 128 tile) only
// read operand fragments from LDS and issue MFMAs; the four producer waves
// only move data: they keep the raw global bytes of the next kPDepth steps in
// a register ring, write step t+1's activations and decoded f16 weights into
// the other LDS stage while the consumers multiply step t, and refill the
// ring.  One barrier per step separates the stages.  On each SIMD the matrix
// core work of two consumer waves overlaps the loads, decode and LDS stores
// of one producer wave.  Each role runs its own loop (its values stay out of
// the other role's registers); both meet the same barriers.  Ring depth:
// four steps for TM = 128 (its 137 consumer VGPRs already keep a second
// workgroup off the CU, so the producers' extra registers cost nothing),
// two for TM = 256 (three waves per SIMD: at most 170 VGPRs).  Measured at
// M = 512 (Q8_0 Mistral set): 597-603 TF/s against 593-596 with two steps
// and 584-587 before the scale fix in RawW.
template <int TM> constexpr int pg_depth() { return TM == 128 ? 4 : 2; }
template <int TM> constexpr int pg_threads() { return TM * 2 + 256; }

template <int FMT, bool EXACT, int TM>
__global__ void __launch_bounds__(pg_threads<TM>())
    k_gemm_kq2(const _Float16 *__restrict__ Xh, int ldh, int M, int K,
               const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd, int N, int B,
               float *__restrict__ Y, int ldy, const float *__restrict__ rowmul,
               int steps_per_split) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  constexpr int NC = TM / 32, AI = TM / 32, PG_STAGE = pg_stage<TM>(), kPDepth = pg_depth<TM>();
  const int n0 = blockIdx.x * PGN, m0 = blockIdx.y * TM;
  const int s_begin = blockIdx.z * steps_per_split;
  const int nsteps = min((K + PGK - 1) / PGK - s_begin, steps_per_split);
  if (wave >= NC) {
    // ------------------------------------------------------------ producer
    const int pt = tid - NC * 64;  // 0..255
    // A: TM * 8 chunks of 16 B per step, TM / 32 per producer thread
    const _Float16 *arow[AI];
#pragma unroll
    for (int i = 0; i < AI; i++) {
      const int idx = pt + i * 256;
      arow[i] = Xh + (size_t)min(m0 + (idx >> 3), M - 1) * ldh + (idx & 7) * 8;
    }
    // W: row n0 + pt/2 (clamped), quarters 2*(pt%2), 2*(pt%2)+1 of the step
    const int brow = pt >> 1, bq0 = 2 * (pt & 1);
    const int bn = min(n0 + brow, N - 1);
    u32x4 ra[kPDepth][AI];
    RawW rw[kPDepth][2];
    auto load = [&](int slot, int t) {
      const int step = s_begin + min(t, nsteps - 1);
#pragma unroll
      for (int i = 0; i < AI; i++)
        ra[slot][i] = *reinterpret_cast<const u32x4 *>(arow[i] + (size_t)step * PGK);
      pg_load_w<FMT>(rw[slot][0], W, Wd, B, bn, step, bq0);
      pg_load_w<FMT>(rw[slot][1], W, Wd, B, bn, step, bq0 + 1);
    };
    auto stage = [&](int slot, int t, int buf) {
      _Float16 *As = lds + buf * PG_STAGE, *Bs = As + TM * PGLD;
#pragma unroll
      for (int i = 0; i < AI; i++) {
        const int idx = pt + i * 256;
        *reinterpret_cast<u32x4 *>(&As[(idx >> 3) * PGLD + (idx & 7) * 8]) = ra[slot][i];
      }
#pragma unroll
      for (int h = 0; h < 2; h++) {
        uint32_t wv[8];
        pg_decode_w<FMT, EXACT>(rw[slot][h], s_begin + t, bq0 + h, B, wv);
        u32x4 *dst = reinterpret_cast<u32x4 *>(&Bs[brow * PGLD + (bq0 + h) * 16]);
        dst[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
        dst[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
      }
      load(slot, t + kPDepth);
    };
#pragma unroll
    for (int i = 0; i < kPDepth; i++) load(i, i);
    stage(0, 0, 0);
    __syncthreads();
    // iteration t stages step t+1 (ring slot (t+1) % kPDepth) into stage (t+1)%2
    int t0 = 0;
    for (; t0 + 2 * kPDepth < nsteps; t0 += 2 * kPDepth) {
#pragma unroll
      for (int j = 0; j < 2 * kPDepth; j++) {
        stage((j + 1) % kPDepth, t0 + j + 1, (j + 1) & 1);
        __syncthreads();
      }
    }
#pragma unroll
    for (int j = 0; j < 2 * kPDepth; j++) {
      if (t0 + j < nsteps) {
        if (t0 + j + 1 < nsteps) stage((j + 1) % kPDepth, t0 + j + 1, (j + 1) & 1);
        __syncthreads();
      }
    }
    return;
  }
  // -------------------------------------------------------------- consumer
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int l32 = lane & 31, lh = lane >> 5;
  f32x16 acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mt][nt][r] = 0.0f;
  // Two consumer groups half a step apart: the first half of the waves read
  // step t's fragments and multiply them; the second half first multiply
  // step t-1's fragments (held in registers across the barrier), then read
  // step t's.  With eight consumers each SIMD holds one wave of each group,
  // so one wave's LDS reads overlap the other's matrix-core work.
  const bool lag = wave >= NC / 2;
  f16x8 fa[4][2], fb[4][2];
  auto read = [&](int t) {
    const _Float16 *As = lds + (t & 1) * PG_STAGE, *Bs = As + TM * PGLD;
#pragma unroll
    for (int k16 = 0; k16 < 4; k16++) {
#pragma unroll
      for (int mt = 0; mt < 2; mt++)
        fa[k16][mt] = *reinterpret_cast<const f16x8 *>(
            &As[(wm + mt * 32 + l32) * PGLD + k16 * 16 + lh * 8]);
#pragma unroll
      for (int nt = 0; nt < 2; nt++)
        fb[k16][nt] = *reinterpret_cast<const f16x8 *>(
            &Bs[(wn + nt * 32 + l32) * PGLD + k16 * 16 + lh * 8]);
    }
  };
  auto mma = [&]() {
#pragma unroll
    for (int k16 = 0; k16 < 4; k16++)
#pragma unroll
      for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[k16][mt], fb[k16][nt],
                                                               acc[mt][nt], 0, 0, 0);
  };
  __syncthreads();  // step 0 staged
  if (!lag) {
    for (int t = 0; t < nsteps; t++) {
      read(t);
      mma();
      __syncthreads();
    }
  } else {
    read(0);
    __syncthreads();
    for (int t = 1; t < nsteps; t++) {
      mma();
      read(t);
      __syncthreads();
    }
    mma();
  }
  const bool atomic = gridDim.z > 1;
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
    float rm[16];
    load_rowmul(rowmul, m0 + wm + mt * 32, lh, M, rm);
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
      const int n = n0 + wn + nt * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < M && n < N) {
          const float v = acc[mt][nt][r] * rm[r];
          if (atomic) atomicAdd(&Y[(size_t)m * ldy + n], v);
          else Y[(size_t)m * ldy + n] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 256 x 256 tiles, four waves (one per SIMD), each a 128 x 128 sub-tile: 4 x 4
// MFMA tiles, 256 f32 accumulators per lane (the accumulation registers of
// the SIMD, which a single resident wave has to itself).  Per 64-element K
// step a wave reads 32 KiB of fragments from LDS for 64 MFMAs, half the LDS
// bytes per multiply-add of 64 x 64 sub-tiles.
//
// Fetching: thread i brings row i of the weight tile (every distinct plane of
// the step once) and eight 16-byte activation chunks.  Two register bundles
// alternate: iteration t issues the fetch of step t+2 into one bundle at its
// start, then, between its four k16 rounds of MFMAs, decodes a quarter of
// step t+1 from the other bundle into the free LDS stage.  The loop has no
// data-dependent branches, so the memory-counter waits stay exact (the
// oldest bundle only).
constexpr int PG3M = 256, PG3N = 256;
constexpr int PG3_STAGE = (PG3M + PG3N) * PGLD;  // halfs per stage

template <int FMT>
struct WBundle;
template <>
struct WBundle<SYN_HIP_FMT_Q8_0> {  // blocks 2s, 2s+1: planes 0, 1 and scales
  u32x4 pl[4];
  uint32_t d[2];  // the dword holding the row's f16 scale (half rp % 2)
};
template <>
struct WBundle<SYN_HIP_FMT_Q4_0> {  // blocks 2s, 2s+1: their nibble planes and scales
  u32x4 pl[2];
  uint32_t d[2];  // the dword holding the row's f16 scale (half rp % 2)
};
template <>
struct WBundle<SYN_HIP_FMT_Q4_K> {  // scale plane, sub-block planes 2(s%4), 2(s%4)+1
  u32x4 sc, pl[2];
};
template <>
struct WBundle<SYN_HIP_FMT_Q6_K> {  // ql planes 2st, 2st+1, qh plane 8+st, scales, d
  u32x4 ql[2], qh, sc;
  uint32_t d;  // the dword holding the row's f16 scale (half rp % 2)
};

// The f16 scales are fetched as the aligned dword holding them (rows 2j and
// 2j+1): a 16-bit load would be masked right after it arrives, which makes
// the compiler wait for it at once instead of a step later.
template <int FMT>
__device__ __forceinline__ void pg_fetch_w(WBundle<FMT> &w, const u32x4 *__restrict__ W,
                                           const uint16_t *__restrict__ Wd, int B, int n,
                                           int step) {
  const size_t panel = (size_t)(n >> 6), rp = (size_t)(n & 63);
  const uint32_t *Wd32 = reinterpret_cast<const uint32_t *>(Wd);
  if constexpr (FMT == SYN_HIP_FMT_Q8_0) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const size_t blk = (size_t)min(2 * step + h, B - 1);
      w.pl[2 * h] = W[((panel * B + blk) * 2 + 0) * 64 + rp];
      w.pl[2 * h + 1] = W[((panel * B + blk) * 2 + 1) * 64 + rp];
      w.d[h] = Wd32[((panel * B + blk) * 64 + rp) >> 1];
    }
  } else if constexpr (FMT == SYN_HIP_FMT_Q4_0) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const size_t blk = (size_t)min(2 * step + h, B - 1);
      w.pl[h] = W[(panel * B + blk) * 64 + rp];
      w.d[h] = Wd32[((panel * B + blk) * 64 + rp) >> 1];
    }
  } else if constexpr (FMT == SYN_HIP_FMT_Q4_K) {
    const size_t sb = (size_t)(step >> 2);
    const int sub = 2 * (step & 3);
    w.sc = W[((panel * B + sb) * 9 + 0) * 64 + rp];
    w.pl[0] = W[((panel * B + sb) * 9 + 1 + sub) * 64 + rp];
    w.pl[1] = W[((panel * B + sb) * 9 + 2 + sub) * 64 + rp];
  } else {
    const size_t sb = (size_t)(step >> 2);
    const int st = step & 3;
    w.ql[0] = W[((panel * B + sb) * 13 + 2 * st) * 64 + rp];
    w.ql[1] = W[((panel * B + sb) * 13 + 2 * st + 1) * 64 + rp];
    w.qh = W[((panel * B + sb) * 13 + 8 + st) * 64 + rp];
    w.sc = W[((panel * B + sb) * 13 + 12) * 64 + rp];
    w.d = Wd32[((panel * B + sb) * 64 + rp) >> 1];
  }
}

// the RawW of quarter q (pg_load_w's view) inside a bundle; odd: row n is odd
template <int FMT>
__device__ __forceinline__ RawW pg_quarter(const WBundle<FMT> &w, int q, bool odd) {
  RawW r;
  if constexpr (FMT == SYN_HIP_FMT_Q8_0) {
    r.q0 = w.pl[q];
    r.d = odd ? w.d[q >> 1] >> 16 : w.d[q >> 1] & 0xffffu;
  } else if constexpr (FMT == SYN_HIP_FMT_Q4_0) {
    r.q0 = w.pl[q >> 1];
    r.d = odd ? w.d[q >> 1] >> 16 : w.d[q >> 1] & 0xffffu;
  } else if constexpr (FMT == SYN_HIP_FMT_Q4_K) {
    r.q0 = w.sc;
    r.q1 = w.pl[q >> 1];
  } else {
    r.q0 = w.ql[q >> 1];
    r.q1 = w.qh;
    r.q2 = w.sc;
    r.d = odd ? w.d >> 16 : w.d & 0xffffu;
  }
  return r;
}

template <int FMT>
struct Fetch {
  u32x4 a[8];
  WBundle<FMT> w;
};

template <int FMT, bool EXACT>
__global__ void __launch_bounds__(256)
    k_gemm_kq5(const _Float16 *__restrict__ Xh, int ldh, int M, int K,
               const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd, int N, int B,
               float *__restrict__ Y, int ldy, const float *__restrict__ rowmul,
               int steps_per_split) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * PG3N, m0 = blockIdx.y * PG3M;
  const int s_begin = blockIdx.z * steps_per_split;
  const int nsteps = min((K + PGK - 1) / PGK - s_begin, steps_per_split);
  // A: 2048 chunks of 8 halfs per step, eight per thread (row idx/8, idx =
  // tid + 256 i); W: row tid (clamped)
  const _Float16 *arow[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int idx = tid + i * 256;
    arow[i] = Xh + (size_t)min(m0 + (idx >> 3), M - 1) * ldh + (idx & 7) * 8;
  }
  const int bn = min(n0 + tid, N - 1);
  auto fetch = [&](Fetch<FMT> &f, int t) {
    const int step = s_begin + min(t, nsteps - 1);
#pragma unroll
    for (int i = 0; i < 8; i++)
      f.a[i] = *reinterpret_cast<const u32x4 *>(arow[i] + (size_t)step * PGK);
    pg_fetch_w<FMT>(f.w, W, Wd, B, bn, step);
  };
  // part p (0..3) of staging step t: A chunks 2p, 2p+1 and weight quarter p
  auto stage_part = [&](const Fetch<FMT> &f, int t, int buf, int p) {
    _Float16 *As = lds + buf * PG3_STAGE, *Bs = As + PG3M * PGLD;
#pragma unroll
    for (int i = 2 * p; i < 2 * p + 2; i++) {
      const int idx = tid + i * 256;
      *reinterpret_cast<u32x4 *>(&As[(idx >> 3) * PGLD + (idx & 7) * 8]) = f.a[i];
    }
    uint32_t wv[8];
    pg_decode_w<FMT, EXACT>(pg_quarter<FMT>(f.w, p, bn & 1), s_begin + t, p, B, wv);
    u32x4 *dst = reinterpret_cast<u32x4 *>(&Bs[tid * PGLD + p * 16]);
    dst[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
    dst[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
  };
  const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
  const int l32 = lane & 31, lh = lane >> 5;
  f32x16 acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mt][nt][r] = 0.0f;
  f16x8 fa[2][4], fb[2][4];
  auto read = [&](int t, int k16, int b) {
    const _Float16 *As = lds + (t & 1) * PG3_STAGE, *Bs = As + PG3M * PGLD;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
      fa[b][mt] = *reinterpret_cast<const f16x8 *>(
          &As[(wm + mt * 32 + l32) * PGLD + k16 * 16 + lh * 8]);
#pragma unroll
    for (int nt = 0; nt < 4; nt++)
      fb[b][nt] = *reinterpret_cast<const f16x8 *>(
          &Bs[(wn + nt * 32 + l32) * PGLD + k16 * 16 + lh * 8]);
  };
  auto mma = [&](int b) {
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
      for (int nt = 0; nt < 4; nt++)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[b][mt], fb[b][nt], acc[mt][nt],
                                                             0, 0, 0);
  };
  // iteration t: fetch step t+2 into `next`, multiply step t, stage step t+1
  // from `cur` (the last iterations fetch and stage clamped, in-bounds data
  // that no one reads).  The MFMAs of step t's last k16 group wait until the
  // next iteration has issued its first fragment reads: their operands are
  // in registers (read before the barrier), so they cover the LDS latency
  // that follows the barrier.
  // (Not for Q8_0 with f32 products, whose decode registers would spill.)
  constexpr bool kDefer = !(FMT == SYN_HIP_FMT_Q8_0 && !EXACT);
  auto iteration = [&](int t, Fetch<FMT> &cur, Fetch<FMT> &next) {
    fetch(next, t + 2);
    read(t, 0, 0);
    if (kDefer && t > 0) mma(1);
#pragma unroll
    for (int k16 = 0; k16 < 4; k16++) {
      if (k16 < 3) read(t, k16 + 1, (k16 + 1) & 1);
      if (k16 < 3 || !kDefer) mma(k16 & 1);
      stage_part(cur, t + 1, (t + 1) & 1, k16);
    }
    __syncthreads();
  };
  Fetch<FMT> f0, f1;
  fetch(f0, 0);
  fetch(f1, 1);
#pragma unroll
  for (int p = 0; p < 4; p++) stage_part(f0, 0, 0, p);
  __syncthreads();
  int t = 0;
  for (; t + 2 <= nsteps; t += 2) {
    iteration(t, f1, f0);
    iteration(t + 1, f0, f1);
  }
  if (t < nsteps) iteration(t, f1, f0);
  if (kDefer) mma(1);
  const bool atomic = gridDim.z > 1;
#pragma unroll
  for (int mt = 0; mt < 4; mt++) {
    float rm[16];
    load_rowmul(rowmul, m0 + wm + mt * 32, lh, M, rm);
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const int n = n0 + wn + nt * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < M && n < N) {
          const float v = acc[mt][nt][r] * rm[r];
          if (atomic) atomicAdd(&Y[(size_t)m * ldy + n], v);
          else Y[(size_t)m * ldy + n] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Direct-load form (Q4_0).  Four waves own a 256 x 256 tile; wave (wr, wc)
// the 128 x 128 sub-tile at rows wr*128, columns wc*128.  Both operands go
// from global memory straight into LDS (gfx950 global_load_lds_dwordx4: no
// registers, no ds_write), KR_NS stages deep, two steps ahead:
//  - activations (f16) in the padded [256][72] layout (the pad slot of each
//    row keeps the fragment reads free of bank conflicts; the direct loads
//    fill it with a copy of the row's first chunk);
//  - the raw weight bytes as stored: each (panel, block) of the nibble plane
//    layout is 64 rows x 16 bytes, one 1 KiB direct load, plus the f16
//    scales of the step's 4 panels x 2 blocks.
// Each wave reads the raw bytes of its 128 columns and decodes them to f16
// in registers (the two waves of a column half decode the same weights: VALU
// work that runs beside the matrix cores).  One barrier per 64-element step
// publishes the next stage.
//
// k order.  Lane l of a fragment holds column (or row) l % 32 and 8 k
// values; lanes l < 32 take block 2s of step s and lanes l >= 32 block
// 2s+1, so MFMA group g (0..3) covers elements 8g..8g+7 of both blocks
// (activation chunks g and 4+g of the step).  A fragment holds the element
// order 0,2,4,6,1,3,5,7 of its 8 nibbles; the activations are converted in
// the same order (k_f32_to_f16 perm8).  The MFMA sums over k in any order.
constexpr int KR_NS = 3;                       // stages
constexpr int KR_SLOTS = PGLD / 8;             // 16-byte slots per activation row (8 + 1 pad)
constexpr int KR_A = PG3M * PGLD * 2;          // activation bytes per stage (36,864)
constexpr int KR_ADMA = PG3M * KR_SLOTS / 256; // activation direct loads per thread (9)
constexpr int KR_WCH = 8;                      // weight KiB per stage: 4 panels x 2 blocks
constexpr int KR_STAGE_BYTES = KR_A + (KR_WCH + 1) * 1024;  // + 1 KiB of scales
// direct loads a wave issues per stage (activations, its 2 weight chunks, the
// scales): the count kr_publish leaves outstanding per stage in flight
constexpr int KR_AFTER = KR_ADMA + KR_WCH / 4 + 1;

// the B fragment of MFMA group g from the lane's block (32 nibbles) and f16
// scale pair d: 8 f16 weights (nibble - 8) * d, each exact before one f16
// rounding (see pg_decode_w)
__device__ __forceinline__ f16x8 kr_decode(const u32x4 &q, int g, f16x2 d) {
  const f16x2 bias = f16x2{(_Float16)-1032.0f, (_Float16)-1032.0f};
  const uint32_t v = u32x4_word(q, g);
  const uint32_t lo = v & 0x0f0f0f0fu, hi = (v >> 4) & 0x0f0f0f0fu;
  const uint32_t p[4] = {__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u),
                         __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u),
                         __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u),
                         __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; i++)
    o[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, p[i]) + bias) * d);
  return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

__global__ void __launch_bounds__(256)
    k_gemm_kqr(const _Float16 *__restrict__ Xh, int ldh, int M, int K,
               const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd, int N, int B,
               float *__restrict__ Y, int ldy, const float *__restrict__ rowmul,
               int steps_per_split) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
  constexpr int WCH = KR_WCH, STAGE = KR_STAGE_BYTES;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, lh = lane >> 5, wr = wave >> 1, wc = wave & 1;
  const int n0 = blockIdx.x * PG3N, m0 = blockIdx.y * PG3M;
  const int s_begin = blockIdx.z * steps_per_split;
  const int nsteps = min((K + PGK - 1) / PGK - s_begin, steps_per_split);
  const int last_panel = (N - 1) >> 6;
  // activation slot s = (wave * KR_ADMA + i) * 64 + lane of a stage is row
  // s / 9, chunk s % 9 (the pad chunk reloads chunk 0); rows past M read
  // row M - 1 (never stored)
  uint32_t aoff[KR_ADMA];
#pragma unroll
  for (int i = 0; i < KR_ADMA; i++) {
    const int s = (wave * KR_ADMA + i) * 64 + lane, row = s / KR_SLOTS, c = s % KR_SLOTS;
    aoff[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)ldh + (uint32_t)(c < 8 ? c : 0) * 8u;
  }
  // weight chunk j = p * 2 + b of a stage: panel p of the tile (clamped to
  // the matrix's last), block 2s + b (clamped to B - 1), issued by wave
  // j / 2; the scales by every wave: lane l brings bytes 16 (l % 8) .. of
  // panel l / 16, block (l / 8) % 2
  const uint8_t *Wb = reinterpret_cast<const uint8_t *>(W);
  const uint8_t *Wdb = reinterpret_cast<const uint8_t *>(Wd);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) _Float16 *)lds;
  auto dma = [&](int t, int stage) {
    const int step = s_begin + min(t, nsteps - 1);
    const _Float16 *src = Xh + (size_t)step * PGK;
    const uint32_t sb = lds_base + (uint32_t)(stage * STAGE);
    const uint32_t wa = (uint32_t)__builtin_amdgcn_readfirstlane(wave * KR_ADMA * 1024);
#pragma unroll
    for (int i = 0; i < KR_ADMA; i++) kr_dma(src + aoff[i], sb + wa + (uint32_t)(i * 1024));
#pragma unroll
    for (int i = 0; i < WCH / 4; i++) {
      const int j = __builtin_amdgcn_readfirstlane(wave * (WCH / 4) + i);
      const int p = j >> 1, b = j & 1;
      const size_t panel = (size_t)min((n0 >> 6) + p, last_panel);
      const size_t blk = (size_t)min(2 * step + b, B - 1);
      kr_dma(Wb + (panel * B + blk) * 1024 + lane * 16, sb + (uint32_t)(KR_A + j * 1024));
    }
    {  // every wave loads the same scale bytes (no branch; identical writes)
      const int q = lane >> 3, p = q >> 1, b = q & 1;
      const size_t panel = (size_t)min((n0 >> 6) + p, last_panel);
      const size_t blk = (size_t)min(2 * step + b, B - 1);
      kr_dma(Wdb + (panel * B + blk) * 128 + (lane & 7) * 16,
             sb + (uint32_t)(KR_A + WCH * 1024));
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mt][nt][r] = 0.0f;

  const int arow = ((wr * 128 + l32) * PGLD + lh * 32) * 2;  // the lane's row, chunk 4*lh
  u32x4 q[4];     // raw nibbles of the lane's block (2s + lh) for its 4 column groups
  f16x2 dd[4];    // their f16 scales
  f16x8 fa[2][4], fb[2][4];
  // step t's raw weights, scales and MFMA group 0 operands from stage `stage`
  auto open_step = [&](int t, int stage) {
    const uint8_t *st = reinterpret_cast<const uint8_t *>(lds) + stage * STAGE;
    // all ones while block 2s + lh exists (the clamped block past the end
    // of an odd B decodes to zeros, against zero activations)
    const uint32_t dm = (uint32_t)((2 * (s_begin + t) + lh - B) >> 31) & 0xffffu;
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const int p = wc * 2 + (nt >> 1), rp = (nt & 1) * 32 + l32;
      q[nt] = *reinterpret_cast<const u32x4 *>(st + KR_A + (p * 2 + lh) * 1024 + rp * 16);
      // every scale reads as its IEEE value (QLinearQ4_0::gemm_ok)
      const uint16_t bits = *reinterpret_cast<const uint16_t *>(
                                st + KR_A + WCH * 1024 + ((p * 2 + lh) * 64 + rp) * 2) &
                            (uint16_t)dm;
      const _Float16 v = __builtin_bit_cast(_Float16, bits);
      dd[nt] = f16x2{v, v};
    }
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
      fa[0][mt] = *reinterpret_cast<const f16x8 *>(st + arow + mt * 32 * PGLD * 2);
#pragma unroll
    for (int nt = 0; nt < 4; nt++) fb[0][nt] = kr_decode(q[nt], 0, dd[nt]);
  };
  auto mma = [&](int b) {
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
      for (int nt = 0; nt < 4; nt++)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[b][mt], fb[b][nt], acc[mt][nt],
                                                             0, 0, 0);
  };

  // Step t lives in stage t % 3.  Iteration t: groups 0-2 of step t (each
  // MFMA group beside the reads and decode of the next group); the barrier
  // that publishes step t+1; the load of step t+3 into the stage step t
  // has left; step t+1's group 0 operands beside step t's last group.
  dma(0, 0);
  dma(1, 1);
  dma(2, 2);
  kr_publish<2 * KR_AFTER>();
  open_step(0, 0);
  for (int t = 0; t < nsteps; t++) {
    const int cur = t % KR_NS, nxt = cur == KR_NS - 1 ? 0 : cur + 1;
    const uint8_t *sa = reinterpret_cast<const uint8_t *>(lds) + cur * STAGE + arow;
#pragma unroll
    for (int g = 0; g < 3; g++) {
      const int b = g & 1;
#pragma unroll
      for (int mt = 0; mt < 4; mt++)
        fa[b ^ 1][mt] = *reinterpret_cast<const f16x8 *>(sa + mt * 32 * PGLD * 2 + (g + 1) * 16);
#pragma unroll
      for (int nt = 0; nt < 4; nt++) fb[b ^ 1][nt] = kr_decode(q[nt], g + 1, dd[nt]);
      mma(b);
    }
    kr_publish<KR_AFTER>();
    dma(t + 3, cur);
    // group 3 of step t runs from fa[1] / fb[1] while group 0 of step t+1
    // (a clamped, unused step after the last) fills fa[0] / fb[0]
    const f16x8 a3[4] = {fa[1][0], fa[1][1], fa[1][2], fa[1][3]};
    const f16x8 b3[4] = {fb[1][0], fb[1][1], fb[1][2], fb[1][3]};
    open_step(t + 1, nxt);
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
      for (int nt = 0; nt < 4; nt++)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a3[mt], b3[nt], acc[mt][nt], 0, 0, 0);
  }
  // the prefetches past the last step must land before the workgroup's LDS
  // can go to another workgroup
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const bool atomic = gridDim.z > 1;
#pragma unroll
  for (int mt = 0; mt < 4; mt++) {
    float rm[16];
    load_rowmul(rowmul, m0 + wr * 128 + mt * 32, lh, M, rm);
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const int n = n0 + wc * 128 + nt * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wr * 128 + mt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < M && n < N) {
          const float v = acc[mt][nt][r] * rm[r];
          if (atomic) atomicAdd(&Y[(size_t)m * ldy + n], v);
          else Y[(size_t)m * ldy + n] = v;
        }
      }
    }
  }
}

// f32 activation rows -> zero-padded f16 rows of ldh = round_up(k, PGK)
// halfs in xh (grown on demand; xh_bytes its size), each row scaled by a
// power of two whose inverse lands in *rowmul (m floats after the rows), in
// the k_gemm_kqr Q4_0 chunk order if perm8
size_t f16_rows_bytes(size_t m, size_t k) {
  return round_up(m * round_up(k, PGK) * 2, 256) + m * sizeof(float);
}
static syn_status_t to_f16_rows(size_t m, size_t k, const float *d_x, size_t ldx, DevBuf &xh,
                                size_t &xh_bytes, bool perm8, float **rowmul, hipStream_t s,
                                float *zero_y0 = nullptr, size_t ldy = 0, size_t ny = 0) {
  if (ldx % 4 || k % 8) {
    set_error("GEMM activation stride must be a multiple of 4 floats and K of 8");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  if (m > 0x7fffffffu) return SYN_ERR_INVALID_ARG;
  const size_t ldh = round_up(k, PGK);  // zero-padded to whole K steps
  const size_t need = f16_rows_bytes(m, k);
  if (xh_bytes < need) {
    SYN_HIP(hipDeviceSynchronize());
    SYN_TRY(xh.alloc(need));
    xh_bytes = need;
  }
  *rowmul = reinterpret_cast<float *>(xh.as<unsigned char>() + round_up(m * ldh * 2, 256));
  hipLaunchKernelGGL(k_f32_to_f16, dim3((unsigned)m), dim3(256), 0, s, d_x, (int)ldx,
                     xh.as<_Float16>(), (int)ldh, *rowmul, (int)k, perm8 ? 1 : 0, zero_y0,
                     (int)ldy, (int)ny);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// Y (ksplit > 1: the splits add their partial tiles into it) cleared by a
// kernel, not a memset node, so the call can sit in a captured graph
static syn_status_t zero_y(float *d_y, size_t m, size_t n, size_t ldy, hipStream_t s) {
  if (ldy % 4 || reinterpret_cast<uintptr_t>(d_y) % 16) {
    for (size_t r = 0; r < m; r++)
      SYN_TRY(launch_zero_i32(reinterpret_cast<int *>(d_y + r * ldy), n, s));
    return SYN_OK;
  }
  return launch_zero_i32(reinterpret_cast<int *>(d_y), (m - 1) * ldy + n, s);
}

template <class Kern>
static syn_status_t launch_gemm(Kern kern, bool &attr_set, dim3 grid, unsigned threads, size_t shm,
                                const _Float16 *X, size_t ldh, size_t m, size_t k,
                                const u32x4 *W, const uint16_t *Wd, size_t n, int blocks,
                                float *d_y, size_t ldy, const float *rowmul, int per,
                                hipStream_t s) {
  if (!attr_set) {  // more than the default 64 KiB of dynamic LDS
    SYN_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)shm));
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(threads), shm, s, X, (int)ldh, (int)m, (int)k, W, Wd,
                     (int)n, blocks, d_y, (int)ldy, rowmul, per);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// Y[m, n] = X[m, k] W^T for a weight matrix of format fmt in the plane
// layout (W, Wd, B blocks per row), X f32 rows converted to f16 in xh;
// exact: the weights decode with f16 products (see pg_decode_w)
static syn_status_t kq_gemm_f16(int fmt, bool exact, const u32x4 *W, const uint16_t *Wd,
                                int blocks, size_t n, size_t k, const float *d_x, size_t ldx,
                                DevBuf &xh, size_t &xh_bytes, size_t m, float *d_y, size_t ldy,
                                hipStream_t s) {
  const size_t ldh = round_up(k, PGK);
  const int steps = (int)cdiv(k, PGK);
  // dynamic-LDS attribute set per kernel: k_gemm_kq5 0-3 and 8, k_gemm_kqr
  // 10, k_gemm_kq2 11-15 (256-row tiles) and 16-20 (128-row tiles)
  static bool attr[21] = {};
  // Q4_0 on enough 256 x 256 tiles for three quarters of the CUs: the
  // direct-load kernel (measured ahead of k_gemm_kq5 there; for Q8_0 the
  // two tie, and k_gemm_kq2 leads on split-K grids)
  const int tiles256 = (int)(cdiv(n, PG3N) * cdiv(m, PG3M));
  if (fmt == SYN_HIP_FMT_Q4_0 && tiles256 >= 192 && m * ldh < (1u << 31)) {
    float *rowmul = nullptr;
    SYN_TRY(to_f16_rows(m, k, d_x, ldx, xh, xh_bytes, true, &rowmul, s));
    const int tiles_n = (int)cdiv(n, PG3N), tiles_m = (int)cdiv(m, PG3M);
    const dim3 grid((unsigned)tiles_n, (unsigned)tiles_m, 1);
    const int per = steps;
    return launch_gemm(k_gemm_kqr, attr[10], grid, 256, (size_t)KR_NS * KR_STAGE_BYTES,
                       xh.as<_Float16>(), ldh, m, k, W, Wd, n, blocks, d_y, ldy, rowmul, per,
                       s);
  }
  // Enough 256 x 256 tiles for three quarters of the CUs: the four-wave
  // kernel, one K pass per tile.  Else 256 x 128 tiles (twice as many) when
  // they cover three quarters of the CUs, one K pass (Q8_0, 2048 x 4096 x
  // 4096: 727 against 620 TF/s on 128 x 128 tiles; 1024 x 4096 x 4096, 128
  // tiles of 256 x 128: 500 against 605).  Fewer: 128 x 128 tiles (two
  // workgroups per CU), split over K into at most kMaxSplit parts towards
  // 256 workgroups.  Every split adds its partial tile into Y with f32
  // atomics, and that traffic outweighs idle CUs beyond one workgroup per
  // CU (Q8_0, 128 x 128 tiles, M = 512: q 4096 -> 4096 42.0 us in two parts,
  // 51.4 in four; k/v 4096 -> 1024 23.9 us in four, 29.0 in two, 28.3 in eight; with
  // 256 x 128 tiles in three parts 46.9 and 29.9).
  constexpr int kMaxSplit = 4;
  const bool big = cdiv(n, PG3N) * cdiv(m, PG3M) >= 192;
  const bool mid = !big && cdiv(n, PGN) * cdiv(m, PGM) >= 192;
  const int tm = big ? PG3M : mid ? PGM : 128;
  const int tiles_n = (int)cdiv(n, big ? PG3N : PGN), tiles_m = (int)cdiv(m, (size_t)tm);
  int ksplit = 1;
  if (!big && !mid)  // >= 8 steps per split
    ksplit = std::max(1, std::min(kMaxSplit, std::min((int)cdiv(256, (size_t)(tiles_n * tiles_m)),
                                                      steps / 8)));
  const int per = (int)cdiv((size_t)steps, (size_t)ksplit);
  ksplit = (int)cdiv((size_t)steps, (size_t)per);
  // a K split adds its partial tiles into Y: the conversion kernel clears Y
  // (row-aligned 16-byte rows), else a kernel of its own does
  const bool zero_in_conv =
      ksplit > 1 && ldy % 4 == 0 && reinterpret_cast<uintptr_t>(d_y) % 16 == 0 && n < (1u << 31);
  float *rowmul = nullptr;
  SYN_TRY(to_f16_rows(m, k, d_x, ldx, xh, xh_bytes, false, &rowmul, s,
                      zero_in_conv ? d_y : nullptr, ldy, n));
  const _Float16 *X = xh.as<_Float16>();
  if (ksplit > 1 && !zero_in_conv) SYN_TRY(zero_y(d_y, m, n, ldy, s));
  const dim3 grid((unsigned)tiles_n, (unsigned)tiles_m, (unsigned)ksplit);
  const size_t shm =
      2 * (size_t)(big ? PG3_STAGE : mid ? pg_stage<256>() : pg_stage<128>()) * sizeof(_Float16);
  const unsigned threads = big ? 256 : mid ? pg_threads<256>() : pg_threads<128>();
  auto launch = [&](auto kern, bool &attr_set) -> syn_status_t {
    return launch_gemm(kern, attr_set, grid, threads, shm, X, ldh, m, k, W, Wd, n, blocks, d_y,
                       ldy, rowmul, per, s);
  };
  if (big) {
    if (fmt == SYN_HIP_FMT_Q8_0 && exact) return launch(k_gemm_kq5<SYN_HIP_FMT_Q8_0, true>, attr[0]);
    if (fmt == SYN_HIP_FMT_Q8_0) return launch(k_gemm_kq5<SYN_HIP_FMT_Q8_0, false>, attr[1]);
    if (fmt == SYN_HIP_FMT_Q4_0) return launch(k_gemm_kq5<SYN_HIP_FMT_Q4_0, true>, attr[8]);
    if (fmt == SYN_HIP_FMT_Q4_K) return launch(k_gemm_kq5<SYN_HIP_FMT_Q4_K, true>, attr[2]);
    return launch(k_gemm_kq5<SYN_HIP_FMT_Q6_K, true>, attr[3]);
  }
  auto kq2 = [&](auto tmc, int a) -> syn_status_t {
    constexpr int T = decltype(tmc)::value;
    if (fmt == SYN_HIP_FMT_Q8_0 && exact) return launch(k_gemm_kq2<SYN_HIP_FMT_Q8_0, true, T>, attr[a]);
    if (fmt == SYN_HIP_FMT_Q8_0) return launch(k_gemm_kq2<SYN_HIP_FMT_Q8_0, false, T>, attr[a + 1]);
    if (fmt == SYN_HIP_FMT_Q4_0) return launch(k_gemm_kq2<SYN_HIP_FMT_Q4_0, true, T>, attr[a + 2]);
    if (fmt == SYN_HIP_FMT_Q4_K) return launch(k_gemm_kq2<SYN_HIP_FMT_Q4_K, true, T>, attr[a + 3]);
    return launch(k_gemm_kq2<SYN_HIP_FMT_Q6_K, true, T>, attr[a + 4]);
  };
  return mid ? kq2(std::integral_constant<int, 256>{}, 11)
             : kq2(std::integral_constant<int, 128>{}, 16);
}

syn_status_t QLinearKQ::gemm(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                             hipStream_t s) {
  const bool exact = fmt != SYN_HIP_FMT_Q8_0 || q8_scales_f16_exact;
  return kq_gemm_f16(fmt, exact, wq.as<u32x4>(), wd.as<uint16_t>(), blocks, n, k, d_x, ldx, xh,
                     xh_bytes, m, d_y, ldy, s);
}

// Q4_0 rows on the same GEMM (its nibble planes sit in the Q8_0 plane layout
// with one plane per block); only when every block scale, as the handle's
// loader reads it, is the IEEE value of its f16 bits (gemm_ok())
syn_status_t QLinearQ4_0::gemm(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                               hipStream_t s) {
  if (!gemm_ok()) {
    set_error("Q4_0 GEMM: halved subnormal block scales need the GEMV path");
    return SYN_ERR_INVALID_ARG;
  }
  return kq_gemm_f16(SYN_HIP_FMT_Q4_0, true, nib.as<u32x4>(), sc.as<uint16_t>(), blocks, n, k,
                     d_x, ldx, xh, xh_bytes, m, d_y, ldy, s);
}

}  // namespace syn
