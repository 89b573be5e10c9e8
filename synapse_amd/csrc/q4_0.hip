// Q4_0 path (A6/A7): Q4Linear weights (q4_linear.rs:64-121, pack_for_zig
// bytes [f16 scale | 16 nibble bytes], element 2i = low nibble, 2i+1 = high)
// times f32 activations, as q4_0GemvRow computes (qmatmul.zig:276-343).
//
// HBM layout after the one-time repack: nibble blocks in the same 64-row
// panel interleave as the INT8 path (16 bytes per block per row, one 1 KiB
// wave load per block), f16 scales in a parallel [panel][block][64] array.
// Per block the kernel forms sum_j a_j*n_j with n_j in 0..15 (f32 FMAs with a
// wave-uniform activation operand) and removes the +8 offset with the block
// sum of the activations: dot = sum a_j n_j - 8 sum a_j.  Float outputs carry
// the north star's tolerance (max_j|y-r| / max_j|r| <= 1e-3 per row).
#include <algorithm>
#include <cmath>
#include <vector>

#include "linear.hpp"
#include "split_k.hpp"

namespace syn {

__device__ __forceinline__ float nib_lo(uint32_t w, int byte) {
  return (float)((w >> (8 * byte)) & 0xfu);
}
__device__ __forceinline__ float nib_hi(uint32_t w, int byte) {
  return (float)((w >> (8 * byte + 4)) & 0xfu);
}

// 8 elements of one dword: bytes b -> elements 2b (lo), 2b+1 (hi)
__device__ __forceinline__ float dot8(uint32_t w, const float *__restrict__ a, float s) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
#pragma unroll
  for (int b = 0; b < 4; b++) {
    s = __builtin_fmaf(a[2 * b], (float)((lo >> (8 * b)) & 0xffu), s);
    s = __builtin_fmaf(a[2 * b + 1], (float)((hi >> (8 * b)) & 0xffu), s);
  }
  return s;
}


__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// A block scale as the handle's loader defines it: the Zig GEMV's IEEE
// f16ToF32 (qmatmul.zig:346-371, sub = 1), or the Rust converter of the
// GGUF path (converter.rs:12-40 via gguf.rs:294-326), which returns half
// the IEEE value for subnormal inputs (sub = 0.5; exact in f32).
__device__ __forceinline__ float q4_scale(uint32_t h, float sub) {
  const float d = f16_bits_to_f32(h);
  return (h & 0x7c00u) == 0 ? d * sub : d;
}

// grid (panels, ksplit); lane = output row, blocks [b0, b1) of this slice.
// Load order: the activation blocks whose sums this thread forms (first
// round, the waves that have any), then the first round of weight blocks,
// so that the block sums only wait for the activations and the weights'
// HBM latency overlaps them.  The dot products read the activations with
// wave-uniform addresses (scalar loads).
// A K split finishes in the same launch (split_k.hpp; skacc holds M rows
// of ksplit slices of N64 slots, skcnt a counter per panel).
template <int M, int U>
__global__ void __launch_bounds__(1024)
    k_gemv_q4_0(const u32x4 *__restrict__ nib, const uint16_t *__restrict__ sc,
                const float *__restrict__ x, int ldx, float *__restrict__ y, int ldy,
                unsigned *__restrict__ skacc, int *__restrict__ skcnt, int N, int B,
                int bs, float sub) {
  extern __shared__ __align__(16) float smem[];
  __shared__ int s_last;
  const int NT = blockDim.x;
  const int panel = blockIdx.x, ks = blockIdx.y;
  const int nw = NT >> 6;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int b0 = ks * bs, b1 = min(B, b0 + bs), nb = b1 - b0;
  float *asum = smem;            // [M][bs]
  float *red = smem + M * bs;    // [nw][M][64]
  const size_t pbase = (size_t)panel * B;
  const int nsum = M * nb;       // block sums of the slice
  const bool sum_wave = wave * 64 < nsum;
  float4 xa4[8];
  int tslot = 0;
  if (sum_wave) {
    const int t = min(tid, nsum - 1);
    const int m = M == 1 ? 0 : t / nb, bl = t - m * nb;
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)m * ldx + (size_t)(b0 + bl) * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) xa4[i] = src[i];
    tslot = m * bs + bl;
  }
  u32x4 q[U];
  uint16_t dh[U];
  auto issue = [&](int bb) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = min(bb + u * nw, b1 - 1);
      q[u] = __builtin_nontemporal_load(nib + (pbase + b) * 64 + lane);
      dh[u] = __builtin_nontemporal_load(sc + (pbase + b) * 64 + lane);
    }
  };
  int bb = b0 + wave;
  issue(min(bb, b1 - 1));
  asm volatile("" ::: "memory");
  if (sum_wave) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      s += xa4[i].x;
      s += xa4[i].y;
      s += xa4[i].z;
      s += xa4[i].w;
    }
    asum[tslot] = s;  // clamped threads store the same value again
  }
  for (int t = tid + NT; t < nsum; t += NT) {  // slices with more sums than threads
    const int m = t / nb, bl = t - m * nb;
    const float *xa = x + (size_t)m * ldx + (size_t)(b0 + bl) * 32;
    float s = 0.0f;
    for (int i = 0; i < 32; i++) s += xa[i];
    asum[m * bs + bl] = s;
  }
  __syncthreads();
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; m++) acc[m] = 0.0f;
  for (; bb < b1; bb += nw * U) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = bb + u * nw;
      if (b < b1) {
        const float d = q4_scale(dh[u], sub);
#pragma unroll
        for (int m = 0; m < M; m++) {
          const float *xa = x + (size_t)m * ldx + (size_t)b * 32;
          float s = 0.0f;
          s = dot8(q[u].x, xa, s);
          s = dot8(q[u].y, xa + 8, s);
          s = dot8(q[u].z, xa + 16, s);
          s = dot8(q[u].w, xa + 24, s);
          const float blk = s - 8.0f * asum[m * bs + (b - b0)];
          acc[m] = __builtin_fmaf(blk, d, acc[m]);
        }
      }
    }
    if (bb + nw * U < b1) issue(bb + nw * U);
  }
#pragma unroll
  for (int m = 0; m < M; m++) red[(wave * M + m) * 64 + lane] = acc[m];
  __syncthreads();
  const int N64 = gridDim.x * 64;
  if (gridDim.y > 1) {
    unsigned seen = 0;
    const int S = gridDim.y;
    for (int t = tid; t < M * 64; t += NT) {
      const int m = t >> 6, r = t & 63;
      float s = 0.0f;
      for (int w = 0; w < nw; w++) s += red[(w * M + m) * 64 + r];
      seen |= sk_put(skacc + ((size_t)m * S + blockIdx.y) * N64 + panel * 64 + r, s);
    }
    if (!sk_arrive(seen, skcnt + panel, S, &s_last)) return;
    for (int t = tid; t < M * 64; t += NT) {
      const int m = t >> 6, r = t & 63, row = panel * 64 + r;
      const float v = sk_sum(skacc + (size_t)m * S * N64 + row, N64, S);
      if (row < N) y[(size_t)m * ldy + row] = v;
    }
    sk_reset(skcnt + panel);
    return;
  }
  for (int t = tid; t < M * 64; t += NT) {
    const int m = t >> 6, r = t & 63;
    float s = 0.0f;
    for (int w = 0; w < nw; w++) s += red[(w * M + m) * 64 + r];
    const int row = panel * 64 + r;
    if (row < N) y[(size_t)m * ldy + row] = s;
  }
}

// Batch-1 form with mixed-precision FMAs.  A nibble e masked in place inside
// the low 8 bits of a 16-bit half is the f16 subnormal e * 2^-24 (positions
// 0-3) or 16e * 2^-24 (positions 4-7): exact, so each element costs one
// v_fma_mix_f32 (f16 weight operand, f32 activation and accumulator) and a
// dword of 8 nibbles one shift and four masks:
//   w & 0x000f000f -> (e0, e4)      w & 0x00f000f0 -> 16 (e1, e5)
//   (w>>8) & ...   -> (e2, e6)      (w>>8) & ...   -> 16 (e3, e7)
// Products and sums stay in f32 (activations are not rounded); the block dot
// is (s0 + s1/16) * 2^24, then Q4_0's -8 offset comes off as 8 * sum(x).
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

// A K split either writes f32 partials (part, for k_q4_reduce or the
// consumer's PartRows) or, with skacc set, finishes in the same launch
// (split_k.hpp: per-slice slots, the panel's last slice adds them in slice
// order and writes y).
template <int U>
__global__ void __launch_bounds__(512)
    k_gemv_q4_0h(const u32x4 *__restrict__ nib, const uint16_t *__restrict__ sc,
                 const float *__restrict__ x, float *__restrict__ y, float *__restrict__ part,
                 unsigned *__restrict__ skacc, int *__restrict__ skcnt, int N, int B, int bs,
                 float sub) {
  extern __shared__ __align__(16) float hsm[];
  __shared__ int s_last;
  constexpr int NT = 512, NW = NT / 64;
  const int panel = blockIdx.x, ks = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int b0 = ks * bs, b1 = min(B, b0 + bs), nb = b1 - b0;
  float *asum = hsm;        // [bs]
  float *red = hsm + bs;    // [NW][64]
  const size_t pbase = (size_t)panel * B;
  // 1. activation blocks of this thread's block sum (waves that have one)
  const bool sum_wave = wave * 64 < nb;
  float4 xa4[8];
  if (sum_wave) {
    const float4 *src =
        reinterpret_cast<const float4 *>(x + (size_t)(b0 + min(tid, nb - 1)) * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) xa4[i] = src[i];
  }
  // 2. the first round of weight blocks
  u32x4 q[U];
  uint16_t dh[U];
  auto issue = [&](int bb) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = min(bb + u * NW, b1 - 1);
      q[u] = __builtin_nontemporal_load(nib + (pbase + b) * 64 + lane);
      dh[u] = __builtin_nontemporal_load(sc + (pbase + b) * 64 + lane);
    }
  };
  int bb = b0 + wave;
  issue(min(bb, b1 - 1));
  asm volatile("" ::: "memory");
  if (sum_wave) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      s += xa4[i].x;
      s += xa4[i].y;
      s += xa4[i].z;
      s += xa4[i].w;
    }
    if (tid < nb) asum[tid] = s;
  }
  for (int t = tid + NT; t < nb; t += NT) {  // slices of more than 512 blocks
    const float *xa = x + (size_t)(b0 + t) * 32;
    float s = 0.0f;
    for (int i = 0; i < 32; i++) s += xa[i];
    asum[t] = s;
  }
  __syncthreads();
  float acc = 0.0f;
  for (; bb < b1; bb += NW * U) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = bb + u * NW;
      if (b < b1) {
        const float *xa = x + (size_t)b * 32;
        const uint32_t wd[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const uint32_t w = wd[c], w8 = wd[c] >> 8;
          const float *xc = xa + 8 * c;
          const h2_t p0 = as_h2(w & 0x000f000fu), p1 = as_h2(w & 0x00f000f0u);
          const h2_t p2 = as_h2(w8 & 0x000f000fu), p3 = as_h2(w8 & 0x00f000f0u);
          s0 = __builtin_fmaf((float)p0.x, xc[0], s0);
          s1 = __builtin_fmaf((float)p1.x, xc[1], s1);
          s0 = __builtin_fmaf((float)p2.x, xc[2], s0);
          s1 = __builtin_fmaf((float)p3.x, xc[3], s1);
          s0 = __builtin_fmaf((float)p0.y, xc[4], s0);
          s1 = __builtin_fmaf((float)p1.y, xc[5], s1);
          s0 = __builtin_fmaf((float)p2.y, xc[6], s0);
          s1 = __builtin_fmaf((float)p3.y, xc[7], s1);
        }
        const float dot = __builtin_fmaf(s1, 0.0625f, s0) * 16777216.0f;
        const float blk = dot - 8.0f * asum[b - b0];
        acc = __builtin_fmaf(blk, q4_scale(dh[u], sub), acc);
      }
    }
    if (bb + NW * U < b1) issue(bb + NW * U);
  }
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (skacc && gridDim.y > 1) {
    float v = 0.0f, tot = 0.0f;
    if (tid < 64) {
#pragma unroll
      for (int w = 0; w < NW; w++) v += red[w * 64 + tid];
    }
    if (sk_slots_last(v, skacc + panel * 64, (size_t)gridDim.x * 64, blockIdx.y, skcnt + panel,
                      gridDim.y, &tot, &s_last) &&
        tid < 64 && panel * 64 + tid < N)
      y[panel * 64 + tid] = tot;
    return;
  }
  if (tid < 64) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) s += red[w * 64 + tid];
    const int row = panel * 64 + tid;
    if (gridDim.y == 1) {
      if (row < N) y[row] = s;
    } else {
      part[(size_t)ks * gridDim.x * 64 + row] = s;
    }
  }
}

// U blocks in flight per wave: 8 with 8 waves when a slice has >= 64
// blocks (four workgroups per CU stream the matrix), else 4 with up to 16
template <int M>
static void launch_q4_m(const GemvPlan &p, const u32x4 *nib, const uint16_t *sc, const float *x,
                        int ldx, float *y, int ldy, const SplitKSlots &sk, int N, float sub,
                        hipStream_t s) {
  const bool wide = p.cs >= 64;
  const int waves = wide ? 8 : std::min(p.waves, M >= 8 ? 8 : 16);
  const size_t shm = ((size_t)M * p.cs + (size_t)waves * M * 64) * sizeof(float);
  unsigned *ska = sk.slots();
  int *skc = sk.counters();
  if (wide)
    hipLaunchKernelGGL((k_gemv_q4_0<M, 8>), dim3(p.panels, p.ksplit), dim3(64 * waves), shm, s,
                       nib, sc, x, ldx, y, ldy, ska, skc, N, p.chunks, p.cs, sub);
  else
    hipLaunchKernelGGL((k_gemv_q4_0<M, 4>), dim3(p.panels, p.ksplit), dim3(64 * waves), shm, s,
                       nib, sc, x, ldx, y, ldy, ska, skc, N, p.chunks, p.cs, sub);
}

typedef void (*q4_launcher)(const GemvPlan &, const u32x4 *, const uint16_t *, const float *,
                            int, float *, int, const SplitKSlots &, int, float, hipStream_t);
static const q4_launcher kQ4Launch[9] = {nullptr,        launch_q4_m<1>, launch_q4_m<2>,
                                         launch_q4_m<3>, launch_q4_m<4>, launch_q4_m<5>,
                                         launch_q4_m<6>, launch_q4_m<7>, launch_q4_m<8>};

syn_status_t QLinearQ4_0::gemv(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                               hipStream_t s) {
  if (m == 0 || n == 0 || k == 0) return SYN_OK;
  if (m > 16 && gemm_ok() && ldx % 4 == 0) return gemm(m, d_x, ldx, d_y, ldy, s);
  const float sub = rs_f16_scales ? 0.5f : 1.0f;
  // "chunks" here are 32-element blocks; a K slice holds whole blocks.  One
  // launch per block of up to 8 rows: a K split finishes in place (split_k.hpp)
  const GemvPlan p = make_gemv_plan(n, (size_t)blocks, false);
  if (p.ksplit > 1) SYN_TRY(sk.ensure(p.panels, 8, p.ksplit));
  for (size_t m0 = 0; m0 < m; m0 += 8) {
    const int mb = (int)std::min<size_t>(8, m - m0);
    const size_t shm_h = ((size_t)p.cs + 8 * 64) * 4;
    if (mb == 1 && shm_h <= 60 * 1024) {
      // two blocks per wave and round: measured best at the LLaMA shapes
      hipLaunchKernelGGL(k_gemv_q4_0h<2>, dim3(p.panels, p.ksplit), dim3(512), shm_h, s,
                         nib.as<u32x4>(), sc.as<uint16_t>(), d_x + m0 * ldx, d_y + m0 * ldy,
                         nullptr, sk.slots(), sk.counters(), (int)n, p.chunks,
                         p.cs, sub);
    } else {
      kQ4Launch[mb](p, nib.as<u32x4>(), sc.as<uint16_t>(), d_x + m0 * ldx, (int)ldx,
                    d_y + m0 * ldy, (int)ldy, sk, (int)n, sub, s);
    }
    SYN_LAUNCH_CHECK();
  }
  return SYN_OK;
}

syn_status_t QLinearQ4_0::gemv_parts(const float *d_x, float *d_y, PartRows *out,
                                     hipStream_t s) {
  if (!d_x || !d_y || !out) return SYN_ERR_NULL_PTR;
  if (n == 0 || k == 0) return SYN_ERR_INVALID_ARG;
  const float sub = rs_f16_scales ? 0.5f : 1.0f;
  const GemvPlan p = make_gemv_plan(n, (size_t)blocks, false);
  const size_t N64 = (size_t)p.panels * 64;
  const size_t shm_h = ((size_t)p.cs + 8 * 64) * 4;
  if (shm_h > 60 * 1024) return SYN_ERR_INVALID_ARG;  // K slice too long for this kernel
  if (p.ksplit > 1 && part_elems < (size_t)p.ksplit * N64) return SYN_ERR_INVALID_ARG;
  hipLaunchKernelGGL(k_gemv_q4_0h<2>, dim3(p.panels, p.ksplit), dim3(512), shm_h, s,
                     nib.as<u32x4>(), sc.as<uint16_t>(), d_x, d_y, part.as<float>(), nullptr,
                     nullptr, (int)n, p.chunks, p.cs, sub);
  SYN_LAUNCH_CHECK();
  if (p.ksplit > 1)
    *out = PartRows{part.as<float>(), p.ksplit, (int)N64};
  else
    *out = PartRows{d_y, 1, 0};
  return SYN_OK;
}

syn_status_t QLinearQ4_0::prepare(size_t max_m) {
  const GemvPlan p = make_gemv_plan(n, (size_t)blocks, false);
  if (p.ksplit > 1) SYN_TRY(sk.ensure(p.panels, 8, p.ksplit));
  const size_t need = (size_t)p.ksplit * std::min<size_t>(8, max_m) * (size_t)p.panels * 64;
  if (p.ksplit > 1 && part_elems < need) {
    part_elems = need;
    SYN_HIP(hipDeviceSynchronize());
    SYN_TRY(part.alloc(part_elems * sizeof(float)));
  }
  return SYN_OK;
}

syn_status_t QLinearQ4_0::upload_packed(const uint8_t *packed, size_t n_, size_t k_) {
  n = n_;
  k = k_;
  blocks = (int)(k_ / 32);
  const size_t P = cdiv(n_, 64), B = (size_t)blocks;
  std::vector<uint8_t> hn(P * B * 64 * 16, 0x88);  // padding rows: nibble 8 -> value 0
  std::vector<uint16_t> hs(P * B * 64, 0);
  has_subnormal_scale = false;
  for (size_t row = 0; row < n_; row++) {
    const size_t p = row / 64, r = row % 64;
    for (size_t b = 0; b < B; b++) {
      const uint8_t *src = packed + (row * B + b) * 18;
      const uint16_t d = (uint16_t)(src[0] | (src[1] << 8));
      hs[(p * B + b) * 64 + r] = d;
      if ((d & 0x7c00u) == 0 && (d & 0x3ffu) != 0) has_subnormal_scale = true;
      std::memcpy(&hn[((p * B + b) * 64 + r) * 16], src + 2, 16);
    }
  }
  SYN_TRY(nib.alloc(hn.size()));
  SYN_TRY(sc.alloc(hs.size() * 2));
  SYN_HIP(hipMemcpy(nib.p, hn.data(), hn.size(), hipMemcpyHostToDevice));
  SYN_HIP(hipMemcpy(sc.p, hs.data(), hs.size() * 2, hipMemcpyHostToDevice));
  return SYN_OK;
}

// q4_linear.rs:64-121
void host_q4_pack(const float *w, size_t n, size_t k, uint8_t *packed) {
  const size_t bpr = (k + 31) / 32;
  for (size_t row = 0; row < n; row++)
    for (size_t b = 0; b < bpr; b++) {
      float vals[32];
      for (int i = 0; i < 32; i++) {
        const size_t col = b * 32 + (size_t)i;
        vals[i] = col < k ? w[row * k + col] : 0.0f;
      }
      float mx = 0.0f;
      for (int i = 0; i < 32; i++) mx = std::fmax(mx, std::fabs(vals[i]));
      const float scale = (mx == 0.0f) ? 0.0f : mx / 7.0f;
      const float inv = (scale == 0.0f) ? 0.0f : 1.0f / scale;
      uint8_t *blk = packed + (row * bpr + b) * 18;
      const uint16_t h = f32_to_f16_trunc(scale);
      blk[0] = (uint8_t)(h & 0xff);
      blk[1] = (uint8_t)(h >> 8);
      for (int i = 0; i < 16; i++) {
        float r0 = std::round(vals[2 * i] * inv), r1 = std::round(vals[2 * i + 1] * inv);
        r0 = std::min(7.0f, std::max(-8.0f, r0));
        r1 = std::min(7.0f, std::max(-8.0f, r1));
        const int v0 = (int)r0, v1 = (int)r1;
        blk[2 + i] = (uint8_t)((uint8_t)(v0 + 8) | (uint8_t)((v1 + 8) << 4));
      }
    }
}

syn_status_t QLinearQ4_0::from_f32(const float *w_nk, size_t n_, size_t k_) {
  std::vector<uint8_t> packed(n_ * ((k_ + 31) / 32) * 18);
  host_q4_pack(w_nk, n_, k_, packed.data());
  return upload_packed(packed.data(), n_, k_);
}

}  // namespace syn

using namespace syn;

extern "C" syn_status_t syn_q4_0_gemv(size_t n, size_t k, const float *a, const uint8_t *b_q4,
                                      float *c) {
  if (!a || !b_q4 || !c) return SYN_ERR_NULL_PTR;
  if (n == 0 || k == 0) return SYN_OK;
  if (k % 32 != 0) return SYN_ERR_SHAPE_MISMATCH;  // exports.zig:1625
  SYN_TRY(ensure_init());
  hipStream_t s = default_stream();
  QLinearQ4_0 L;
  SYN_TRY(L.upload_packed(b_q4, n, k));
  DevBuf dx, dy;
  SYN_TRY(dx.alloc(k * 4));
  SYN_TRY(dy.alloc(n * 4));
  SYN_HIP(hipMemcpyAsync(dx.p, a, k * 4, hipMemcpyHostToDevice, s));
  SYN_TRY(L.gemv(1, dx.as<float>(), k, dy.as<float>(), n, s));
  SYN_HIP(hipMemcpyAsync(c, dy.p, n * 4, hipMemcpyDeviceToHost, s));
  SYN_HIP(hipStreamSynchronize(s));
  return SYN_OK;
}
