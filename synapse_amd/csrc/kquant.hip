// GGUF-block formats Q8_0 / Q4_K / Q6_K (A9-A12): load-time encoder and
// repack, and the decode GEMV over f32 activations.
//
// The reference dequantizes these formats to f32 at load
// (weight_loading/gguf.rs:217-237) and runs f32 matmul_t (ops/matmul.rs:55-79
// -> f32GemvRow, matmul.zig:223-305).  Values are therefore defined by its
// dequantizers, which this file decodes in registers instead:
//   Q8_0  (gguf.rs:255-288)  34 B / 32:  [d f16][32 x i8]          v = d*q
//   Q4_K  (gguf.rs:375-431) 144 B / 256: [d][dmin][12 B scales][128 B nibbles]
//         sub-block s (32): v = n*(d*sc[s]) - dmin*mn[s], element 32s+2i is the
//         low nibble of byte 16s+i, 32s+2i+1 the high nibble
//   Q6_K  (gguf.rs:440-487) 210 B / 256: [ql 128][qh 64][sc i8 16][d f16]
//         q(idx) = ql nibble idx%2 of byte idx/2 | (qh byte idx/4 >> 2*(idx%4) & 3)<<4,
//         v = (q-32) * (sc[idx/16]*d)
// with f16 decoded by the Rust converter (converter.rs:12-40; subnormals halve).
// Float outputs carry the north star's 1e-3 per-row tolerance.
//
// HBM layout: blocks of 64 output rows (panels) are interleaved in 16-byte
// planes, plane p of a block holding bytes 16p..16p+15 of every row's block:
//   Q8_0  2 planes (the 32 quants) + f16 d in a [panel][block][64] array
//   Q4_K  9 planes (the whole 144-byte superblock)
//   Q6_K 13 planes (ql, qh, sc) + f16 d in a [panel][block][64] array
// so every wave64 load (lane = row) is one contiguous 1 KiB.
#include <algorithm>
#include <type_traits>
#include <cmath>
#include <vector>

#include "kq_unit.hpp"
#include "kquant.hpp"
#include "split_k.hpp"

namespace syn {

// ------------------------------------------------------------------ host f16
static float h2f_rs(uint16_t h) {  // converter.rs:12-40
  uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, out;
  if (exp == 0) {
    if (mant == 0) {
      out = sign << 31;
    } else {
      uint32_t e = 1, m = mant;
      while ((m & 0x400u) == 0) { m <<= 1; e++; }
      out = (sign << 31) | ((127u - 15u + 1u - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    out = (sign << 31) | (0xffu << 23) | (mant << 13);
  } else {
    out = (sign << 31) | ((exp + 127u - 15u) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

// f32 -> f16, round to nearest even (encoder side; normal range only is used)
static uint16_t f2h_rne(float v) {
  uint32_t x;
  std::memcpy(&x, &v, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  x &= 0x7fffffffu;
  if (x >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);       // overflow -> inf
  if (x < 0x38800000u) {                                         // below f16 normal range
    float f;
    std::memcpy(&f, &x, 4);
    const float q = f * 16777216.0f;                             // units of 2^-24
    return (uint16_t)(sign | (uint32_t)std::nearbyint(q));
  }
  const uint32_t e = ((x >> 23) - 112u) << 10, m = (x >> 13) & 0x3ffu, rest = x & 0x1fffu;
  uint32_t h = e | m;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

// A super-block scale >= v that decodes to a normal f16 (the reference's
// converter halves subnormals, so the encoder stays out of that range).
static uint16_t enc_scale(float v, float *decoded) {
  uint16_t h = f2h_rne(std::fmax(v, 6.103515625e-05f));  // 2^-14, smallest normal
  while (h2f_rs(h) < v && (h & 0x7fffu) < 0x7bffu) h++;
  *decoded = h2f_rs(h);
  return h;
}

float f16_to_f32_reference(uint16_t h) { return h2f_rs(h); }

// gguf.rs:255-288 (Q8_0), 375-431 (Q4_K), 440-487 (Q6_K), in their order
void kq_dequant(int fmt, const uint8_t *b, size_t nblocks, float *out) {
  for (size_t blk = 0; blk < nblocks; blk++) {
    if (fmt == SYN_HIP_FMT_Q8_0) {
      const uint8_t *p = b + blk * 34;
      const float d = h2f_rs((uint16_t)(p[0] | (p[1] << 8)));
      for (int i = 0; i < 32; i++) out[blk * 32 + i] = d * (float)(int8_t)p[2 + i];
    } else if (fmt == SYN_HIP_FMT_Q4_K) {
      const uint8_t *p = b + blk * 144;
      const float d = h2f_rs((uint16_t)(p[0] | (p[1] << 8)));
      const float dmin = h2f_rs((uint16_t)(p[2] | (p[3] << 8)));
      const uint8_t *sc = p + 4, *qs = p + 16;
      uint8_t scales[8], mins[8];
      for (int i = 0; i < 4; i++) {
        scales[i] = sc[i] & 63;
        scales[i + 4] = (uint8_t)((sc[i + 4] & 15) | ((sc[i] >> 6) << 4));
        mins[i] = (uint8_t)((sc[i + 4] >> 4) | ((sc[i + 8] & 15) << 4));
        mins[i + 4] = (uint8_t)((sc[i + 8] >> 4) | (((sc[i] >> 4) & 12) << 4));
      }
      for (int s = 0; s < 8; s++) {
        const float scf = d * (float)scales[s], mf = dmin * (float)mins[s];
        for (int i = 0; i < 16; i++) {
          const uint8_t byte = qs[16 * s + i];
          out[blk * 256 + 32 * s + 2 * i] = (float)(byte & 15) * scf - mf;
          out[blk * 256 + 32 * s + 2 * i + 1] = (float)(byte >> 4) * scf - mf;
        }
      }
    } else {
      const uint8_t *p = b + blk * 210;
      const uint8_t *ql = p, *qh = p + 128;
      const int8_t *sc = reinterpret_cast<const int8_t *>(p + 192);
      const float d = h2f_rs((uint16_t)(p[208] | (p[209] << 8)));
      for (int idx = 0; idx < 256; idx++) {
        const uint8_t qlb = ql[idx / 2];
        const uint32_t lo = (idx % 2) ? (qlb >> 4) : (qlb & 15u);
        const uint32_t hi = (qh[idx / 4] >> (2 * (idx % 4))) & 3u;
        const float q = (float)((int)(lo | (hi << 4)) - 32);
        out[blk * 256 + idx] = q * ((float)sc[idx / 16] * d);
      }
    }
  }
}

size_t kq_block_bytes(int fmt) {
  return fmt == SYN_HIP_FMT_Q8_0 ? 34 : fmt == SYN_HIP_FMT_Q4_K ? 144 : 210;
}
size_t kq_block_elems(int fmt) { return fmt == SYN_HIP_FMT_Q8_0 ? 32 : 256; }

// ------------------------------------------------------------------ encoders
// The reference ships dequantizers only; these encoders produce bytes in its
// formats (any encoder is valid: the dequantizer defines the values).
static void enc_q8_0(const float *x, uint8_t *b) {
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[i]));
  float d;
  const uint16_t h = enc_scale(amax / 127.0f, &d);
  b[0] = (uint8_t)(h & 0xff);
  b[1] = (uint8_t)(h >> 8);
  for (int i = 0; i < 32; i++) {
    float q = d > 0.0f ? std::round(x[i] / d) : 0.0f;
    q = std::min(127.0f, std::max(-127.0f, q));
    b[2 + i] = (uint8_t)(int8_t)q;
  }
}

// Sub-blocks 0-3 get 6-bit scales and 8-bit mins; in the reference's field
// layout (gguf.rs:405-410) the top two bits of sc[4..7] are also bits 6-7 of
// mn[4..7], so sub-blocks 4-7 are encoded with 4-bit scales and mins.
static void enc_q4_k(const float *x, uint8_t *b) {
  float scale[8], mneg[8];
  for (int s = 0; s < 8; s++) {
    float lo = 0.0f, hi = 0.0f;
    for (int i = 0; i < 32; i++) {
      lo = std::fmin(lo, x[32 * s + i]);
      hi = std::fmax(hi, x[32 * s + i]);
    }
    scale[s] = (hi - lo) / 15.0f;
    mneg[s] = -lo;
  }
  float dmax = 0.0f, mmax = 0.0f;
  for (int s = 0; s < 8; s++) {
    dmax = std::fmax(dmax, scale[s] / (s < 4 ? 63.0f : 15.0f));
    mmax = std::fmax(mmax, mneg[s] / (s < 4 ? 255.0f : 15.0f));
  }
  float d, dmin;
  const uint16_t dh = enc_scale(dmax, &d), mh = enc_scale(mmax, &dmin);
  int sc[8], mn[8];
  for (int s = 0; s < 8; s++) {
    const int smax = s < 4 ? 63 : 15, mmx = s < 4 ? 255 : 15;
    sc[s] = d > 0.0f ? (int)std::lround(scale[s] / d) : 0;
    mn[s] = dmin > 0.0f ? (int)std::lround(mneg[s] / dmin) : 0;
    sc[s] = std::min(smax, std::max(0, sc[s]));
    mn[s] = std::min(mmx, std::max(0, mn[s]));
  }
  std::memset(b, 0, 144);
  b[0] = (uint8_t)(dh & 0xff);
  b[1] = (uint8_t)(dh >> 8);
  b[2] = (uint8_t)(mh & 0xff);
  b[3] = (uint8_t)(mh >> 8);
  uint8_t *sb = b + 4;
  for (int i = 0; i < 4; i++) {
    sb[i] = (uint8_t)(sc[i] | ((sc[i + 4] >> 4) << 6));
    sb[i + 4] = (uint8_t)((sc[i + 4] & 0xf) | ((mn[i] & 0xf) << 4));
    sb[i + 8] = (uint8_t)((mn[i] >> 4) | ((mn[i + 4] & 0xf) << 4));
  }
  for (int s = 0; s < 8; s++) {
    const float scv = d * (float)sc[s], m = dmin * (float)mn[s];
    for (int i = 0; i < 16; i++) {
      int n0 = 0, n1 = 0;
      if (scv > 0.0f) {
        n0 = (int)std::lround((x[32 * s + 2 * i] + m) / scv);
        n1 = (int)std::lround((x[32 * s + 2 * i + 1] + m) / scv);
      }
      n0 = std::min(15, std::max(0, n0));
      n1 = std::min(15, std::max(0, n1));
      b[16 + 16 * s + i] = (uint8_t)(n0 | (n1 << 4));
    }
  }
}

static void enc_q6_k(const float *x, uint8_t *b) {
  float sscale[16];
  float smax = 0.0f;
  for (int s = 0; s < 16; s++) {
    float amax = 0.0f;
    for (int i = 0; i < 16; i++) amax = std::fmax(amax, std::fabs(x[16 * s + i]));
    sscale[s] = amax / 31.0f;
    smax = std::fmax(smax, sscale[s]);
  }
  float d;
  const uint16_t dh = enc_scale(smax / 127.0f, &d);
  std::memset(b, 0, 210);
  for (int s = 0; s < 16; s++) {
    int sc = d > 0.0f ? (int)std::lround(sscale[s] / d) : 0;
    sc = std::min(127, std::max(-127, sc));
    b[192 + s] = (uint8_t)(int8_t)sc;
    const float scale = (float)sc * d;
    for (int i = 0; i < 16; i++) {
      const int idx = 16 * s + i;
      int q = scale > 0.0f ? (int)std::lround(x[idx] / scale) + 32 : 32;
      q = std::min(63, std::max(0, q));
      b[idx / 2] |= (uint8_t)((q & 0xf) << (4 * (idx % 2)));
      b[128 + idx / 4] |= (uint8_t)((q >> 4) << (2 * (idx % 4)));
    }
  }
  b[208] = (uint8_t)(dh & 0xff);
  b[209] = (uint8_t)(dh >> 8);
}

void kq_encode(int fmt, const float *w, size_t n, size_t k, uint8_t *out) {
  const size_t be = kq_block_elems(fmt), bb = kq_block_bytes(fmt), nb = k / be;
  for (size_t r = 0; r < n; r++)
    for (size_t j = 0; j < nb; j++) {
      const float *x = w + r * k + j * be;
      uint8_t *b = out + (r * nb + j) * bb;
      if (fmt == SYN_HIP_FMT_Q8_0) enc_q8_0(x, b);
      else if (fmt == SYN_HIP_FMT_Q4_K) enc_q4_k(x, b);
      else enc_q6_k(x, b);
    }
}

// ------------------------------------------------------------------ repack
static int kq_planes(int fmt) {
  return fmt == SYN_HIP_FMT_Q8_0 ? 2 : fmt == SYN_HIP_FMT_Q4_K ? 9 : 13;
}

syn_status_t QLinearKQ::upload(int fmt_, const uint8_t *gguf, size_t n_, size_t k_) {
  fmt = fmt_;
  n = n_;
  k = k_;
  q8_scales_f16_exact = true;
  const size_t be = kq_block_elems(fmt), bb = kq_block_bytes(fmt);
  blocks = (int)(k / be);
  planes = kq_planes(fmt);
  const size_t P = cdiv(n, 64), B = (size_t)blocks, NP = (size_t)planes;
  std::vector<uint8_t> hp(P * B * NP * 64 * 16, 0);
  std::vector<uint16_t> hd;
  const bool sep_d = fmt != SYN_HIP_FMT_Q4_K;
  if (sep_d) hd.assign(P * B * 64, 0);
  // padding rows decode to zero: Q8_0 d = 0, Q4_K d = dmin = 0, Q6_K d = 0
  for (size_t row = 0; row < n; row++) {
    const size_t p = row / 64, r = row % 64;
    for (size_t b = 0; b < B; b++) {
      const uint8_t *src = gguf + (row * B + b) * bb;
      const uint8_t *qsrc = src;
      if (fmt == SYN_HIP_FMT_Q8_0) {
        const uint16_t d = (uint16_t)(src[0] | (src[1] << 8));
        hd[(p * B + b) * 64 + r] = d;
        qsrc = src + 2;
        // converter.rs:12-40 halves subnormals: an odd subnormal mantissa
        // then falls between f16 values, and a NaN is no f16 value either
        const uint32_t e = (d >> 10) & 0x1fu, m = d & 0x3ffu;
        if ((e == 0 && (m & 1u)) || (e == 31 && m)) q8_scales_f16_exact = false;
      } else if (fmt == SYN_HIP_FMT_Q6_K) {
        hd[(p * B + b) * 64 + r] = (uint16_t)(src[208] | (src[209] << 8));
      }
      for (size_t pl = 0; pl < NP; pl++)
        std::memcpy(&hp[(((p * B + b) * NP + pl) * 64 + r) * 16], qsrc + pl * 16, 16);
    }
  }
  SYN_TRY(wq.alloc(hp.size()));
  SYN_HIP(hipMemcpy(wq.p, hp.data(), hp.size(), hipMemcpyHostToDevice));
  if (sep_d) {
    SYN_TRY(wd.alloc(hd.size() * 2));
    SYN_HIP(hipMemcpy(wd.p, hd.data(), hd.size() * 2, hipMemcpyHostToDevice));
  }
  return SYN_OK;
}

syn_status_t QLinearKQ::from_f32(int fmt_, const float *w, size_t n_, size_t k_) {
  std::vector<uint8_t> bytes(n_ * (k_ / kq_block_elems(fmt_)) * kq_block_bytes(fmt_));
  kq_encode(fmt_, w, n_, k_, bytes.data());
  return upload(fmt_, bytes.data(), n_, k_);
}

size_t QLinearKQ::weight_bytes() const { return n * (size_t)blocks * kq_block_bytes(fmt); }

// ------------------------------------------------------------------ GEMV kernels
// 8 elements of one dword of low/high nibble pairs: bytes b -> (2b lo, 2b+1 hi)
__device__ __forceinline__ float kq_dot8_nib(uint32_t w, const float *__restrict__ a, float s) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
#pragma unroll
  for (int b = 0; b < 4; b++) {
    s = __builtin_fmaf(a[2 * b], (float)((lo >> (8 * b)) & 0xffu), s);
    s = __builtin_fmaf(a[2 * b + 1], (float)((hi >> (8 * b)) & 0xffu), s);
  }
  return s;
}

__device__ __forceinline__ float kq_dot4_i8(uint32_t w, const float *__restrict__ a, float s) {
#pragma unroll
  for (int b = 0; b < 4; b++) s = __builtin_fmaf(a[b], (float)(int8_t)(w >> (8 * b)), s);
  return s;
}

// activation block sums (per `grp` elements) of this workgroup's K range into LDS
template <int M>
__device__ __forceinline__ void kq_asums(const float *__restrict__ x, int ldx, int e0, int ne,
                                         int grp, float *asum, int stride) {
  for (int t = threadIdx.x; t < M * (ne / grp); t += blockDim.x) {
    const int m = t / (ne / grp), g = t - m * (ne / grp);
    const float *xa = x + (size_t)m * ldx + e0 + g * grp;
    float s = 0.0f;
    for (int i = 0; i < grp; i++) s += xa[i];
    asum[m * stride + g] = s;
  }
}

// grid (panels, ksplit); lane = output row; blocks [b0, b1) of this slice.
// WPU waves share each Q4_K / Q6_K block (wave part p decodes sub-blocks /
// groups [p, p + 1) * 8 / WPU or 16 / WPU from only the planes they read),
// so more waves per SIMD hide the activations' scalar-load latency: at eight
// rows a block is ~2,800 VALU ops per lane.
// A K split finishes in the same launch (split_k.hpp; skacc holds M rows of
// ksplit slices of N64 slots, skcnt a counter per panel).
template <int FMT, int M, int WPU>
__global__ void __launch_bounds__(1024)
    k_gemv_kq(const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd,
              const float *__restrict__ x, int ldx, float *__restrict__ y, int ldy,
              unsigned *__restrict__ skacc, int *__restrict__ skcnt, int N, int B,
              int bs) {
  static_assert(WPU == 1 || FMT != SYN_HIP_FMT_Q8_0, "Q8_0 blocks are not split");
  __shared__ int s_last;
  constexpr int NP = FMT == SYN_HIP_FMT_Q8_0 ? 2 : FMT == SYN_HIP_FMT_Q4_K ? 9 : 13;
  constexpr int BE = FMT == SYN_HIP_FMT_Q8_0 ? 32 : 256;
  constexpr int GRP = FMT == SYN_HIP_FMT_Q4_K ? 32 : 16;  // asum group (unused for Q8_0)
  constexpr int GPB = BE / GRP;
  extern __shared__ float smem[];
  const int panel = blockIdx.x, ks = blockIdx.y;
  const int nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int b0 = ks * bs, b1 = min(B, b0 + bs), nb = b1 - b0;
  float *asum = smem;                                   // [M][bs*GPB]
  float *red = smem + (FMT == SYN_HIP_FMT_Q8_0 ? 0 : M * bs * GPB);  // [nw][M][64]
  if (FMT != SYN_HIP_FMT_Q8_0) {
    kq_asums<M>(x, ldx, b0 * BE, nb * BE, GRP, asum, bs * GPB);
    __syncthreads();
  }
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; m++) acc[m] = 0.0f;
  const size_t pbase = (size_t)panel * B;
  // Q4_K sub-blocks [S0, S0 + 8 / WPU) of block b
  auto q4k_part = [&](auto S0c, int b) {
    constexpr int S0 = decltype(S0c)::value, NS = 8 / WPU;
    const u32x4 *Wb = W + ((pbase + b) * NP) * 64 + lane;
    u32x4 pl[9];
    pl[0] = __builtin_nontemporal_load(Wb);
#pragma unroll
    for (int sb = S0; sb < S0 + NS; sb++) pl[1 + sb] = __builtin_nontemporal_load(Wb + (1 + sb) * 64);
    const float d = syn_f16_to_f32_rs(pl[0].x & 0xffffu);
    const float dmin = syn_f16_to_f32_rs(pl[0].x >> 16);
    if constexpr (true) {
      // the in-place f16 subnormal decode of kq_unit.hpp (one v_fma_mix per
      // element and row; the masks are shared by the rows): per Q4_K block
      // ~7 % fewer VALU ops than extract + convert + FMA at eight rows, ~27 %
      // at one (gate 8192 x 3072: 7.69 against 8.0 us at one row, 15.4
      // against 16.1 at eight)
#pragma unroll
      for (int sb = S0; sb < S0 + NS; sb++)
#pragma unroll
        for (int m = 0; m < M; m++)
          kq4_stage(pl, sb, d, dmin, x + (size_t)m * ldx + (size_t)b * 256 + sb * 32,
                    asum[m * bs * GPB + (b - b0) * GPB + sb], acc[m]);
      return;
    }
    // 12 scale bytes = bytes 4..15 of plane 0 (gguf.rs:405-410, u8 arithmetic)
    uint32_t sbw[3] = {pl[0].y, pl[0].z, pl[0].w};
    auto SB = [&](int i) -> uint32_t { return (sbw[i >> 2] >> (8 * (i & 3))) & 0xffu; };
#pragma unroll
    for (int sb = S0; sb < S0 + NS; sb++) {
      uint32_t sc, mn;
      if (sb < 4) {
        sc = SB(sb) & 63u;
        mn = ((SB(sb + 4) >> 4) | ((SB(sb + 8) & 15u) << 4)) & 0xffu;
      } else {
        sc = (SB(sb) & 15u) | ((SB(sb - 4) >> 6) << 4);
        mn = ((SB(sb + 4) >> 4) | (((SB(sb - 4) >> 4) & 12u) << 4)) & 0xffu;
      }
      const float scf = d * (float)sc;
      const float mf = dmin * (float)mn;
      const u32x4 q = pl[1 + sb];
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float *xa = x + (size_t)m * ldx + (size_t)b * 256 + sb * 32;
        float t = 0.0f;
        t = kq_dot8_nib(q.x, xa, t);
        t = kq_dot8_nib(q.y, xa + 8, t);
        t = kq_dot8_nib(q.z, xa + 16, t);
        t = kq_dot8_nib(q.w, xa + 24, t);
        const float as = asum[m * bs * GPB + (b - b0) * GPB + sb];
        acc[m] = __builtin_fmaf(scf, t, acc[m]);
        acc[m] = __builtin_fmaf(-mf, as, acc[m]);
      }
    }
  };
  // Q6_K groups [G0, G0 + 16 / WPU) of block b
  auto q6k_part = [&](auto G0c, int b) {
    constexpr int G0 = decltype(G0c)::value, NG = 16 / WPU;
    const u32x4 *Wb = W + ((pbase + b) * NP) * 64 + lane;
    u32x4 pl[13];
#pragma unroll
    for (int g = G0; g < G0 + NG; g++) {
      if (g == G0 || (g & 1) == 0) pl[g >> 1] = __builtin_nontemporal_load(Wb + (g >> 1) * 64);
      if (g == G0 || (g & 3) == 0)
        pl[8 + (g >> 2)] = __builtin_nontemporal_load(Wb + (8 + (g >> 2)) * 64);
    }
    pl[12] = __builtin_nontemporal_load(Wb + 12 * 64);
    const float d = syn_f16_to_f32_rs(Wd[(pbase + b) * 64 + lane]);
    if constexpr (true) {
      // the in-place six-bit decode of kq_unit.hpp (one v_fma_mix per element
      // and row, the masks shared by the rows; down 8192 -> 3072: 8.9, 10.0
      // and 23.0 us at one, two and eight rows against 9.2, 10.8 and 23.3
      // with two bit classes per element, 10.7, 10.8 and 23.3 with extract +
      // convert + FMA)
#pragma unroll
      for (int g = G0; g < G0 + NG; g++)
#pragma unroll
        for (int m = 0; m < M; m++)
          kq6_group(pl, g, d, x + (size_t)m * ldx + (size_t)b * 256 + g * 16,
                    asum[m * bs * GPB + (b - b0) * GPB + g], acc[m]);
      return;
    }
    const uint32_t scw[4] = {pl[12].x, pl[12].y, pl[12].z, pl[12].w};
#pragma unroll
    for (int g = G0; g < G0 + NG; g++) {
      // ql bytes 8g..8g+7: plane g/2, dwords 2*(g%2), 2*(g%2)+1
      const u32x4 qp = pl[g >> 1];
      const uint32_t lo0 = (g & 1) ? qp.z : qp.x, lo1 = (g & 1) ? qp.w : qp.y;
      // qh bytes 4g..4g+3: plane 8 + g/4, dword g%4
      const u32x4 hp = pl[8 + (g >> 2)];
      const uint32_t hi = (g & 3) == 0 ? hp.x : (g & 3) == 1 ? hp.y : (g & 3) == 2 ? hp.z : hp.w;
      const float scale = (float)(int8_t)(scw[g >> 2] >> (8 * (g & 3))) * d;
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float *xa = x + (size_t)m * ldx + (size_t)b * 256 + g * 16;
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const uint32_t lo = ((i < 8 ? lo0 : lo1) >> (4 * (i & 7))) & 15u;
          const uint32_t h2 = (hi >> (2 * i)) & 3u;
          t = __builtin_fmaf(xa[i], (float)(lo | (h2 << 4)), t);
        }
        const float as = asum[m * bs * GPB + (b - b0) * GPB + g];
        const float v = t - 32.0f * as;
        acc[m] = __builtin_fmaf(v, scale, acc[m]);
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  for (int t = wave; t < nb * WPU; t += nw) {
    const int b = b0 + t / WPU, part = t % WPU;
    if constexpr (FMT == SYN_HIP_FMT_Q8_0) {
      const u32x4 *Wb = W + ((pbase + b) * NP) * 64 + lane;
      const u32x4 q0 = __builtin_nontemporal_load(Wb);
      const u32x4 q1 = __builtin_nontemporal_load(Wb + 64);
      const float d = syn_f16_to_f32_rs(Wd[(pbase + b) * 64 + lane]);
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float *xa = x + (size_t)m * ldx + (size_t)b * 32;
        float s = 0.0f;
        s = kq_dot4_i8(q0.x, xa, s);
        s = kq_dot4_i8(q0.y, xa + 4, s);
        s = kq_dot4_i8(q0.z, xa + 8, s);
        s = kq_dot4_i8(q0.w, xa + 12, s);
        s = kq_dot4_i8(q1.x, xa + 16, s);
        s = kq_dot4_i8(q1.y, xa + 20, s);
        s = kq_dot4_i8(q1.z, xa + 24, s);
        s = kq_dot4_i8(q1.w, xa + 28, s);
        acc[m] = __builtin_fmaf(s, d, acc[m]);
      }
    } else if constexpr (WPU == 1) {
      if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(I0{}, b);
      else q6k_part(I0{}, b);
    } else if constexpr (WPU == 2) {
      if (part == 0) {
        if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(I0{}, b);
        else q6k_part(I0{}, b);
      } else {
        if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(std::integral_constant<int, 4>{}, b);
        else q6k_part(std::integral_constant<int, 8>{}, b);
      }
    } else {  // WPU == 4
      if (part == 0) {
        if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(I0{}, b);
        else q6k_part(I0{}, b);
      } else if (part == 1) {
        if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(std::integral_constant<int, 2>{}, b);
        else q6k_part(std::integral_constant<int, 4>{}, b);
      } else if (part == 2) {
        if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(std::integral_constant<int, 4>{}, b);
        else q6k_part(std::integral_constant<int, 8>{}, b);
      } else {
        if constexpr (FMT == SYN_HIP_FMT_Q4_K) q4k_part(std::integral_constant<int, 6>{}, b);
        else q6k_part(std::integral_constant<int, 12>{}, b);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++) red[(wave * M + m) * 64 + lane] = acc[m];
  __syncthreads();
  const int N64 = gridDim.x * 64;
  if (gridDim.y > 1) {
    unsigned seen = 0;
    const int S = gridDim.y;
    for (int t = threadIdx.x; t < M * 64; t += blockDim.x) {
      const int m = t >> 6, r = t & 63;
      float s = 0.0f;
      for (int w = 0; w < nw; w++) s += red[(w * M + m) * 64 + r];
      seen |= sk_put(skacc + ((size_t)m * S + blockIdx.y) * N64 + panel * 64 + r, s);
    }
    if (!sk_arrive(seen, skcnt + panel, S, &s_last)) return;
    for (int t = threadIdx.x; t < M * 64; t += blockDim.x) {
      const int m = t >> 6, r = t & 63, row = panel * 64 + r;
      const float v = sk_sum(skacc + (size_t)m * S * N64 + row, N64, S);
      if (row < N) y[(size_t)m * ldy + row] = v;
    }
    sk_reset(skcnt + panel);
    return;
  }
  for (int t = threadIdx.x; t < M * 64; t += blockDim.x) {
    const int m = t >> 6, r = t & 63;
    float s = 0.0f;
    for (int w = 0; w < nw; w++) s += red[(w * M + m) * 64 + r];
    const int row = panel * 64 + r;
    if (row < N) y[(size_t)m * ldy + row] = s;
  }
}

// ------------------------------------------------------------------ batch-1 GEMV
// Q4_K / Q6_K at M = 1 on grids without a K split (lm_head-sized N): one lane
// per row, the unit decoders of kq_unit.hpp.
// A K split finishes in the same launch (split_k.hpp).
template <int FMT, int NW, int U>
__global__ void __launch_bounds__(NW * 64)
    k_gemv_kqh(const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd,
               const float *__restrict__ x, float *__restrict__ y,
               unsigned *__restrict__ skacc, int *__restrict__ skcnt, int N, int B,
               int bs) {
  __shared__ int s_last;
  constexpr int NT = NW * 64;
  constexpr int NP = FMT == SYN_HIP_FMT_Q4_K ? 9 : 13;
  constexpr int GRP = FMT == SYN_HIP_FMT_Q4_K ? 32 : 16;  // elements per sub-block sum
  constexpr int GPB = 256 / GRP;
  extern __shared__ __align__(16) float ksm[];
  const int panel = blockIdx.x, ks = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int b0 = ks * bs, b1 = min(B, b0 + bs), nb = b1 - b0;
  float *asum = ksm;             // [bs * GPB]
  float *red = ksm + bs * GPB;   // [NW][64]
  const size_t pbase = (size_t)panel * B;
  const float *xb = x + (size_t)b0 * 256;
  const int nsum = nb * GPB;
  // 1. activations of this thread's sub-block sum (waves that have one)
  const bool sum_wave = wave * 64 < nsum;
  float4 xa4[GRP / 4];
  if (sum_wave) {
    const float4 *src = reinterpret_cast<const float4 *>(xb + (size_t)min(tid, nsum - 1) * GRP);
#pragma unroll
    for (int i = 0; i < GRP / 4; i++) xa4[i] = src[i];
  }
  // 2. the first round of superblocks
  u32x4 pl[U][NP];
  uint16_t dh[U];
  auto issue = [&](int bb) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = min(bb + u * NW, b1 - 1);
      const u32x4 *Wb = W + ((pbase + b) * NP) * 64 + lane;
#pragma unroll
      for (int p = 0; p < NP; p++) pl[u][p] = __builtin_nontemporal_load(Wb + p * 64);
      if (FMT == SYN_HIP_FMT_Q6_K) dh[u] = __builtin_nontemporal_load(Wd + (pbase + b) * 64 + lane);
    }
  };
  int bb = b0 + wave;
  issue(min(bb, b1 - 1));
  asm volatile("" ::: "memory");
  if (sum_wave) {
    float sm = 0.0f;
#pragma unroll
    for (int i = 0; i < GRP / 4; i++) {
      sm += xa4[i].x;
      sm += xa4[i].y;
      sm += xa4[i].z;
      sm += xa4[i].w;
    }
    if (tid < nsum) asum[tid] = sm;
  }
  for (int t = tid + NT; t < nsum; t += NT) {
    const float *xa = xb + (size_t)t * GRP;
    float sm = 0.0f;
    for (int i = 0; i < GRP; i++) sm += xa[i];
    asum[t] = sm;
  }
  __syncthreads();
  float acc = 0.0f;
  for (; bb < b1; bb += NW * U) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = bb + u * NW;
      if (b < b1) {
        const float *xs = x + (size_t)b * 256;
        const float *as = asum + (b - b0) * GPB;
        if constexpr (FMT == SYN_HIP_FMT_Q4_K)
          kq4_unit(pl[u], xs, as, acc);
        else
          kq6_unit(pl[u], dh[u], xs, as, acc);
      }
    }
    if (bb + NW * U < b1) issue(bb + NW * U);
  }
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (gridDim.y > 1) {
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
    float sm = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) sm += red[w * 64 + tid];
    const int row = panel * 64 + tid;
    if (row < N) y[row] = sm;
  }
}

// Q4_K / Q6_K: four waves per block (LLaMA-3B shapes, eight rows: gate
// 8192 x 3072 16.2 us against 16.7 with two and 24.4 with one, q 11.8
// against 13.8 and 21.9, down 23.2 against 30.1 and 28.5)
template <int FMT, int M>
static void launch_kq(const GemvPlan &p, const void *W, const uint16_t *Wd, const float *x,
                      int ldx, float *y, int ldy, const SplitKSlots &sk, int N, hipStream_t s) {
  constexpr int BE = FMT == SYN_HIP_FMT_Q8_0 ? 32 : 256;
  constexpr int GRP = FMT == SYN_HIP_FMT_Q4_K ? 32 : 16;
  constexpr int WPU = FMT == SYN_HIP_FMT_Q8_0 ? 1 : 4;
  const int waves = WPU == 1 ? std::min(p.waves, M >= 4 ? 8 : 16) : std::min(16, p.cs * WPU);
  const size_t as = FMT == SYN_HIP_FMT_Q8_0 ? 0 : (size_t)M * p.cs * (BE / GRP);
  const size_t shm = (as + (size_t)waves * M * 64) * sizeof(float);
  hipLaunchKernelGGL((k_gemv_kq<FMT, M, WPU>), dim3(p.panels, p.ksplit), dim3(64 * waves), shm, s,
                     (const u32x4 *)W, Wd, x, ldx, y, ldy, sk.slots(),
                     sk.counters(), N, p.chunks, p.cs);
}

template <int FMT>
static void launch_kq_m(int m, const GemvPlan &p, const void *W, const uint16_t *Wd,
                        const float *x, int ldx, float *y, int ldy, const SplitKSlots &sk, int N,
                        hipStream_t s) {
  switch (m) {
    case 1: launch_kq<FMT, 1>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    case 2: launch_kq<FMT, 2>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    case 3: launch_kq<FMT, 3>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    case 4: launch_kq<FMT, 4>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    case 5: launch_kq<FMT, 5>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    case 6: launch_kq<FMT, 6>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    case 7: launch_kq<FMT, 7>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
    default: launch_kq<FMT, 8>(p, W, Wd, x, ldx, y, ldy, sk, N, s); break;
  }
}

// Batch-1 launch shape (measured at the LLaMA-3.2-3B shapes): Q6_K, and Q4_K
// slices of 8 or more superblocks, run 4 waves of 2 superblocks per round
// (more workgroups per CU); shorter Q4_K slices 8 waves of one.
template <int FMT>
static syn_status_t launch_kqh(const GemvPlan &p, const u32x4 *W, const uint16_t *Wd,
                               const float *x, float *y, const SplitKSlots &sk, int N, size_t shm,
                               hipStream_t s) {
  unsigned *ska = sk.slots();
  int *skc = sk.counters();
  if (FMT == SYN_HIP_FMT_Q6_K || p.cs >= 8)
    hipLaunchKernelGGL((k_gemv_kqh<FMT, 4, 2>), dim3(p.panels, p.ksplit), dim3(256), shm, s, W,
                       Wd, x, y, ska, skc, N, p.chunks, p.cs);
  else
    hipLaunchKernelGGL((k_gemv_kqh<FMT, 8, 1>), dim3(p.panels, p.ksplit), dim3(512), shm, s, W,
                       Wd, x, y, ska, skc, N, p.chunks, p.cs);
  return SYN_OK;
}

syn_status_t QLinearKQ::gemv(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                             hipStream_t s) {
  if (m == 0 || n == 0 || k == 0) return SYN_OK;
  if (m > 8) return gemm(m, d_x, ldx, d_y, ldy, s);
  const GemvPlan p = make_gemv_plan(n, (size_t)blocks, false);
  // one launch for all (up to 8) rows: the weights stream once, and a K
  // split finishes in place (split_k.hpp)
  if (p.ksplit > 1) SYN_TRY(sk.ensure(p.panels, 8, p.ksplit));
  const uint16_t *Wd = wd.as<uint16_t>();
  for (size_t m0 = 0; m0 < m; m0 += 8) {
    const int mb = (int)std::min<size_t>(8, m - m0);
    const float *xm = d_x + m0 * ldx;
    float *ym = d_y + m0 * ldy;
    const size_t gpb = fmt == SYN_HIP_FMT_Q4_K ? 8 : 16;
    const size_t shm_h = ((size_t)p.cs * gpb + 16 * 64) * sizeof(float);
    // one row: the one-lane-per-row kernel on grids without a K split (the
    // lm_head, 128256 x 3072 Q6_K: 60.6 us against 70.4 for the split
    // blocks); split grids take the split blocks (LLaMA-3B q 6.42 against
    // 7.18 us, gate 8.02 against 8.49, down 10.74 against 13.64)
    if (mb == 1 && fmt != SYN_HIP_FMT_Q8_0 && p.ksplit == 1 && shm_h <= 60 * 1024) {
      if (fmt == SYN_HIP_FMT_Q4_K)
        SYN_TRY(launch_kqh<SYN_HIP_FMT_Q4_K>(p, wq.as<u32x4>(), Wd, xm, ym, sk, (int)n, shm_h, s));
      else
        SYN_TRY(launch_kqh<SYN_HIP_FMT_Q6_K>(p, wq.as<u32x4>(), Wd, xm, ym, sk, (int)n, shm_h, s));
    } else if (fmt == SYN_HIP_FMT_Q8_0) {
      launch_kq_m<SYN_HIP_FMT_Q8_0>(mb, p, wq.p, Wd, xm, (int)ldx, ym, (int)ldy, sk, (int)n, s);
    } else if (fmt == SYN_HIP_FMT_Q4_K) {
      launch_kq_m<SYN_HIP_FMT_Q4_K>(mb, p, wq.p, Wd, xm, (int)ldx, ym, (int)ldy, sk, (int)n, s);
    } else {
      launch_kq_m<SYN_HIP_FMT_Q6_K>(mb, p, wq.p, Wd, xm, (int)ldx, ym, (int)ldy, sk, (int)n, s);
    }
    SYN_LAUNCH_CHECK();
  }
  return SYN_OK;
}

syn_status_t QLinearKQ::prepare(size_t max_m) {
  if (max_m > 8 && xh_bytes < f16_rows_bytes(max_m, k)) {
    SYN_TRY(xh.alloc(f16_rows_bytes(max_m, k)));
    xh_bytes = f16_rows_bytes(max_m, k);
  }
  const GemvPlan p = make_gemv_plan(n, (size_t)blocks, false);
  return p.ksplit > 1 ? sk.ensure(p.panels, 8, p.ksplit) : SYN_OK;
}

}  // namespace syn

extern "C" syn_status_t syn_hip_kquant_encode(int fmt, size_t n, size_t k, const float *host_w,
                                              uint8_t *host_out) {
  using namespace syn;
  if (!host_w || !host_out) return SYN_ERR_NULL_PTR;
  if (fmt != SYN_HIP_FMT_Q8_0 && fmt != SYN_HIP_FMT_Q4_K && fmt != SYN_HIP_FMT_Q6_K)
    return SYN_ERR_INVALID_ARG;
  if (n == 0 || k == 0) return SYN_ERR_INVALID_ARG;
  if (k % kq_block_elems(fmt)) return SYN_ERR_SHAPE_MISMATCH;
  kq_encode(fmt, host_w, n, k, host_out);
  return SYN_OK;
}

extern "C" syn_status_t syn_hip_kquant_decode(int fmt, size_t nblocks, const uint8_t *host_blocks,
                                              float *host_out) {
  using namespace syn;
  if (!host_blocks || !host_out) return SYN_ERR_NULL_PTR;
  if (fmt != SYN_HIP_FMT_Q8_0 && fmt != SYN_HIP_FMT_Q4_K && fmt != SYN_HIP_FMT_Q6_K)
    return SYN_ERR_INVALID_ARG;
  kq_dequant(fmt, host_blocks, nblocks, host_out);
  return SYN_OK;
}
