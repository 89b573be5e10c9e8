/*
 * CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference (eren23/synapse) algorithms.  Each
 * function names the reference file:line it restates; paths are relative to
 * the reference's `synapse/` directory.  It is the parity checker for the HIP
 * library and the timed "cpu_simd port" baseline; the product never links it.
 *
 * Floating-point contract: built with -ffp-contract=off, so every `a*b + c`
 * written here rounds twice, as the reference's Zig (strict float mode) and
 * Rust (no contraction) code does; fmaf() marks the places where the
 * reference uses @mulAdd.  libm calls (expf, powf, cosf, sinf, sqrtf) go to
 * glibc, which is what Rust's f32 methods call on Linux.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   - quantizer KATs from zig/tests/test_quantize.zig:143-170, 225-246
 *   - qgemm KATs from crates/synapse-core/src/lib.rs:1541-1567
 *   - GGUF KATs from weight_loading/gguf.rs:700-721, 789-820
 *   - f16 conversions checked exhaustively against IEEE (numpy float16)
 *   - integer GEMM checked against brute force in int64
 *   - the three decoders (INT8 Qwen3-style, f32 CausalLM over Q8_0, INT8
 *     Mamba) against independent float64 numpy forwards, with planted wiring
 *     mistakes shown to fail; conv1d_step by its impulse response; the fused
 *     SwiGLU against numpy
 * Parity unpinned (no reference test, no runnable reference here):
 *   - Q4_K / Q6_K dequant beyond the restated source text (self-made KATs only)
 *   - exact order of Zig's @reduce(.Add) (taken as sequential, LLVM's ordered
 *     vector.reduce.fadd) and whether Zig contracts `a*b + c` (taken as no)
 *   - libm bit patterns of exp/pow/cos/sin on the reference's own host
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * Harness input spec: SplitMix64 + Box-Muller (f64, cast to f32).
 * Not a reference algorithm — the synthetic-data contract shared with the
 * HIP library's own generator.
 * ==================================================================== */
static uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

void orc_fill_normal(float *dst, size_t n, uint64_t seed, float stddev) {
  uint64_t s = seed;
  const double two_pi = 6.283185307179586476925286766559;
  const double sd = (double)stddev;
  size_t i = 0;
  while (i < n) {
    double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    double r = sqrt(-2.0 * log(u1));
    double z0 = r * cos(two_pi * u2);
    double z1 = r * sin(two_pi * u2);
    dst[i++] = (float)(z0 * sd);
    if (i < n) dst[i++] = (float)(z1 * sd);
  }
}

void orc_fill_token_ids(uint32_t *dst, size_t n, uint64_t seed, uint32_t vocab) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; i++) dst[i] = (uint32_t)(splitmix64(&s) % (uint64_t)vocab);
}

/* ======================================================================
 * f16 conversions
 * ==================================================================== */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* q4_linear.rs:9-33 — truncating f32->f16; subnormal/underflow -> signed 0 */
uint16_t orc_f32_to_f16_trunc(float val) {
  uint32_t bits = f2u(val);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
  uint32_t man = bits & 0x7FFFFFu;
  if (exp == 0) return (uint16_t)sign;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man != 0 ? 0x200u : 0u));
  int32_t new_exp = exp - 127 + 15;
  if (new_exp >= 31) return (uint16_t)(sign | 0x7C00u);
  if (new_exp <= 0) return (uint16_t)sign;
  return (uint16_t)(sign | ((uint32_t)new_exp << 10) | (man >> 13));
}

/* qmatmul.zig:346-371 — IEEE-exact f16->f32 (used by the Q4_0 GEMV) */
float orc_f16_to_f32_zig(uint16_t bits) {
  uint32_t sign = ((uint32_t)(bits >> 15)) << 31;
  uint32_t exp5 = (bits >> 10) & 0x1Fu;
  uint32_t mant = bits & 0x3FFu;
  if (exp5 == 0) {
    if (mant == 0) return u2f(sign);
    uint32_t m = mant, e = 0;
    while ((m & 0x400u) == 0) { m <<= 1; e += 1; }
    m &= 0x3FFu;
    uint32_t exp32 = (127u - 15u + 1u - e) << 23;
    return u2f(sign | exp32 | (m << 13));
  } else if (exp5 == 31) {
    return u2f(sign | 0x7F800000u | (mant << 13));
  }
  return u2f(sign | ((exp5 + 127u - 15u) << 23) | (mant << 13));
}

/* weight_loading/converter.rs:12-40 — used by every GGUF dequantizer.
 * The subnormal branch starts its shift counter at 1, so subnormal inputs
 * come out at half their IEEE value; restated as written. */
float orc_f16_to_f32_rs(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t mant = h & 0x3FFu;
  if (exp == 0) {
    if (mant == 0) return u2f(sign << 31);
    uint32_t e = 1, m = mant;
    while ((m & 0x400u) == 0) { m <<= 1; e += 1; }
    m = (m & 0x3FFu) << 13;
    e = 127u - 15u + 1u - e;
    return u2f((sign << 31) | (e << 23) | m);
  } else if (exp == 31) {
    return u2f((sign << 31) | (0xFFu << 23) | (mant << 13));
  }
  return u2f((sign << 31) | ((exp + 127u - 15u) << 23) | (mant << 13));
}

/* ======================================================================
 * A1 — zig/src/ops/quantize.zig:12-47 via ffi/exports.zig:1275-1288
 * ==================================================================== */
int orc_quantize_per_channel_int8(const float *data, size_t channels, size_t channel_size,
                                  int8_t *out, float *scales) {
  if (!data || !out || !scales) return ORC_ERR_NULL_PTR;
  if (channels == 0 || channel_size == 0) return ORC_ERR_INVALID_ARG; /* exports.zig:1284 */
  for (size_t c = 0; c < channels; c++) {
    const float *row = data + c * channel_size;
    int8_t *orow = out + c * channel_size;
    float max_abs = 0.0f;
    for (size_t j = 0; j < channel_size; j++) {
      float a = fabsf(row[j]);
      if (a > max_abs) max_abs = a;
    }
    if (max_abs == 0.0f) {
      scales[c] = 1.0f;
      memset(orow, 0, channel_size);
      continue;
    }
    scales[c] = max_abs / 127.0f;
    float inv_scale = 127.0f / max_abs;
    for (size_t j = 0; j < channel_size; j++) {
      float r = roundf(row[j] * inv_scale); /* @round: half away from zero */
      if (r > 127.0f) r = 127.0f;
      if (r < -127.0f) r = -127.0f;
      orow[j] = (int8_t)r;
    }
  }
  return ORC_OK;
}

/* ======================================================================
 * A2 — quantization/primitives/calibration.rs:11-24 and
 *      int8_linear.rs:35-70 (from_f32_with_scales + transpose_i8)
 * ==================================================================== */
void orc_minmax_scales(const float *w, size_t channels, size_t channel_size, float *scales) {
  for (size_t ch = 0; ch < channels; ch++) {
    const float *row = w + ch * channel_size;
    float max_abs = 0.0f;
    for (size_t j = 0; j < channel_size; j++) max_abs = fmaxf(max_abs, fabsf(row[j]));
    scales[ch] = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
  }
}

/* out_kn is the reference's GEMM-ready transposed layout [in_features, out_features]. */
void orc_quantize_weights_int8(const float *w, const float *scales, size_t out_features,
                               size_t in_features, int8_t *out_kn) {
  for (size_t ch = 0; ch < out_features; ch++) {
    float s = scales[ch];
    if (s == 0.0f) {
      for (size_t j = 0; j < in_features; j++) out_kn[j * out_features + ch] = 0;
      continue;
    }
    float inv_s = 1.0f / s;
    for (size_t j = 0; j < in_features; j++) {
      float v = roundf(w[ch * in_features + j] * inv_s);
      if (v < -128.0f) v = -128.0f;
      if (v > 127.0f) v = 127.0f;
      out_kn[j * out_features + ch] = (int8_t)v;
    }
  }
}

/* ======================================================================
 * A3/A4 — zig/src/ops/qmatmul.zig:37-99 (int8GemmTiled), :171-256
 * (int8GemvRow), :442-548 (macro/micro kernels) via exports.zig:1313-1350
 * ==================================================================== */
#define ORC_KC 512
static void int8_gemv_row(size_t n, size_t k, const int8_t *a, const int8_t *b, size_t ldb,
                          float *c, float sa, const float *sb) {
  size_t j = 0;
  /* 64-column blocks: i32 accumulators, then (f32(acc)*sa)*sb (qmatmul.zig:187-225) */
  for (; j + 64 <= n; j += 64) {
    int32_t acc[64];
    memset(acc, 0, sizeof(acc));
    for (size_t p = 0; p < k; p++) {
      const int32_t av = a[p];
      const int8_t *bp = b + p * ldb + j;
      for (int v = 0; v < 64; v++) acc[v] += av * (int32_t)bp[v];
    }
    for (int v = 0; v < 64; v++) c[j + v] = (float)acc[v] * sa * sb[j + v];
  }
  /* 8-column blocks (:228-246) */
  for (; j + 8 <= n; j += 8) {
    int32_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t p = 0; p < k; p++) {
      const int32_t av = a[p];
      const int8_t *bp = b + p * ldb + j;
      for (int v = 0; v < 8; v++) acc[v] += av * (int32_t)bp[v];
    }
    for (int v = 0; v < 8; v++) c[j + v] = (float)acc[v] * sa * sb[j + v];
  }
  /* scalar tail (:249-255) */
  for (; j < n; j++) {
    int32_t acc = 0;
    for (size_t p = 0; p < k; p++) acc += (int32_t)a[p] * (int32_t)b[p * ldb + j];
    c[j] = (float)acc * sa * sb[j];
  }
}

int orc_qgemm_int8(size_t m, size_t n, size_t k, const int8_t *a, size_t lda, const int8_t *b,
                   size_t ldb, float *c, size_t ldc, const float *scales_a,
                   const float *scales_b) {
  if (!a || !b || !c || !scales_a || !scales_b) return ORC_ERR_NULL_PTR;
  if (m == 0 || n == 0 || k == 0) return ORC_OK; /* exports.zig:1331 */
  if (m <= 16) {                                  /* qmatmul.zig:54-66 */
    for (size_t i = 0; i < m; i++)
      int8_gemv_row(n, k, a + i * lda, b, ldb, c + i * ldc, scales_a[i], scales_b);
    return ORC_OK;
  }
  /* M > 16: C zeroed, then for each KC=512 chunk (in order) the exact i32
   * partial is converted and added: C += (f32(acc_chunk)*sa)*sb.  Packing and
   * MR/NR tiling do not change any value, so the restatement walks chunks. */
  for (size_t i = 0; i < m; i++) memset(c + i * ldc, 0, n * sizeof(float));
  int32_t *acc = (int32_t *)malloc(n * sizeof(int32_t));
  if (!acc) return ORC_ERR_OUT_OF_MEMORY;
  for (size_t pc = 0; pc < k; pc += ORC_KC) {
    size_t kc = (k - pc < ORC_KC) ? (k - pc) : ORC_KC;
    for (size_t i = 0; i < m; i++) {
      memset(acc, 0, n * sizeof(int32_t));
      const int8_t *ar = a + i * lda + pc;
      for (size_t p = 0; p < kc; p++) {
        const int32_t av = ar[p];
        const int8_t *bp = b + (pc + p) * ldb;
        for (size_t j = 0; j < n; j++) acc[j] += av * (int32_t)bp[j];
      }
      float *cr = c + i * ldc;
      const float sa = scales_a[i];
      for (size_t j = 0; j < n; j++) cr[j] = cr[j] + (float)acc[j] * sa * scales_b[j];
    }
  }
  free(acc);
  return ORC_OK;
}

/* qmatmul.zig:106-128 */
void orc_naive_int8_gemm(size_t m, size_t n, size_t k, const int8_t *a, size_t lda,
                         const int8_t *b, size_t ldb, float *c, size_t ldc,
                         const float *scales_a, const float *scales_b) {
  for (size_t i = 0; i < m; i++)
    for (size_t j = 0; j < n; j++) {
      int32_t acc = 0;
      for (size_t p = 0; p < k; p++) acc += (int32_t)a[i * lda + p] * (int32_t)b[p * ldb + j];
      c[i * ldc + j] = (float)acc * scales_a[i] * scales_b[j];
    }
}

/* ======================================================================
 * A6 — quantization/primitives/q4_linear.rs:64-100 (from_f32) and
 *      :106-121 (pack_for_zig): [f16 scale (truncated) | 16 nibble bytes]
 * ==================================================================== */
size_t orc_q4_packed_bytes(size_t out_features, size_t in_features) {
  return out_features * ((in_features + 31) / 32) * 18;
}

void orc_q4_from_f32_packed(const float *w, size_t out_features, size_t in_features,
                            uint8_t *packed) {
  size_t bpr = (in_features + 31) / 32;
  for (size_t row = 0; row < out_features; row++) {
    for (size_t b = 0; b < bpr; b++) {
      float vals[32];
      for (int i = 0; i < 32; i++) {
        size_t col = b * 32 + (size_t)i;
        vals[i] = col < in_features ? w[row * in_features + col] : 0.0f;
      }
      float max_abs = 0.0f;
      for (int i = 0; i < 32; i++) max_abs = fmaxf(max_abs, fabsf(vals[i]));
      float scale = (max_abs == 0.0f) ? 0.0f : max_abs / 7.0f;
      float inv = (scale == 0.0f) ? 0.0f : 1.0f / scale;
      uint8_t *blk = packed + (row * bpr + b) * 18;
      uint16_t h = orc_f32_to_f16_trunc(scale);
      blk[0] = (uint8_t)(h & 0xFF);
      blk[1] = (uint8_t)(h >> 8);
      for (int i = 0; i < 16; i++) {
        float r0 = roundf(vals[2 * i] * inv), r1 = roundf(vals[2 * i + 1] * inv);
        r0 = r0 < -8.0f ? -8.0f : (r0 > 7.0f ? 7.0f : r0);
        r1 = r1 < -8.0f ? -8.0f : (r1 > 7.0f ? 7.0f : r1);
        int v0 = (int)r0, v1 = (int)r1;
        blk[2 + i] = (uint8_t)((uint8_t)(v0 + 8) | (uint8_t)((v1 + 8) << 4));
      }
    }
  }
}

/* A7 — qmatmul.zig:276-343 via exports.zig:1614-1628 */
int orc_q4_0_gemv(size_t n, size_t k, const float *a, const uint8_t *b_q4, float *c) {
  if (!a || !b_q4 || !c) return ORC_ERR_NULL_PTR;
  if (n == 0 || k == 0) return ORC_OK;
  if (k % 32 != 0) return ORC_ERR_SHAPE_MISMATCH;
  const size_t bpr = k / 32, row_bytes = bpr * 18;
  size_t j = 0;
  for (; j + 4 <= n; j += 4) { /* 4 rows at a time (:288-319) */
    float sums[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t blk = 0; blk < bpr; blk++) {
      const size_t a_off = blk * 32;
      for (int r = 0; r < 4; r++) {
        const uint8_t *bs = b_q4 + (j + r) * row_bytes + blk * 18;
        float scale = orc_f16_to_f32_zig((uint16_t)(bs[0] | (bs[1] << 8)));
        float block_sum = 0.0f;
        for (int i = 0; i < 16; i++) {
          uint8_t byte = bs[2 + i];
          float lo = (float)((int)(byte & 0x0F) - 8);
          float hi = (float)((int)(byte >> 4) - 8);
          block_sum += a[a_off + 2 * i] * lo + a[a_off + 2 * i + 1] * hi;
        }
        sums[r] += block_sum * scale;
      }
    }
    for (int r = 0; r < 4; r++) c[j + r] = sums[r];
  }
  for (; j < n; j++) { /* scalar tail (:322-342): scale applied per pair */
    float sum = 0.0f;
    for (size_t blk = 0; blk < bpr; blk++) {
      const size_t a_off = blk * 32;
      const uint8_t *bs = b_q4 + j * row_bytes + blk * 18;
      float scale = orc_f16_to_f32_zig((uint16_t)(bs[0] | (bs[1] << 8)));
      for (int i = 0; i < 16; i++) {
        uint8_t byte = bs[2 + i];
        float lo = (float)((int)(byte & 0x0F) - 8);
        float hi = (float)((int)(byte >> 4) - 8);
        sum += (a[a_off + 2 * i] * lo + a[a_off + 2 * i + 1] * hi) * scale;
      }
    }
    c[j] = sum;
  }
  return ORC_OK;
}

/* ======================================================================
 * A8..A11 — weight_loading/gguf.rs:255-487 (values via converter.rs)
 * ==================================================================== */
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* gguf.rs:294-326 */
int orc_dequant_q4_0(const uint8_t *data, size_t numel, float *out) {
  if (numel % 32) return ORC_ERR_SHAPE_MISMATCH;
  for (size_t b = 0; b < numel / 32; b++) {
    const uint8_t *bs = data + b * 18;
    float delta = orc_f16_to_f32_rs(rd16(bs));
    for (int i = 0; i < 16; i++) {
      uint8_t byte = bs[2 + i];
      out[b * 32 + 2 * i] = delta * (float)((int)(byte & 0x0F) - 8);
      out[b * 32 + 2 * i + 1] = delta * (float)((int)((byte >> 4) & 0x0F) - 8);
    }
  }
  return ORC_OK;
}

/* gguf.rs:255-288 */
int orc_dequant_q8_0(const uint8_t *data, size_t numel, float *out) {
  if (numel % 32) return ORC_ERR_SHAPE_MISMATCH;
  for (size_t b = 0; b < numel / 32; b++) {
    const uint8_t *bs = data + b * 34;
    float scale = orc_f16_to_f32_rs(rd16(bs));
    for (int i = 0; i < 32; i++) out[b * 32 + i] = scale * (float)(int8_t)bs[2 + i];
  }
  return ORC_OK;
}

/* gguf.rs:375-431 — u8 arithmetic exactly as written (6-bit/8-bit fields) */
int orc_dequant_q4_k(const uint8_t *data, size_t numel, float *out) {
  if (numel % 256) return ORC_ERR_SHAPE_MISMATCH;
  for (size_t blk = 0; blk < numel / 256; blk++) {
    const uint8_t *bs = data + blk * 144;
    float d = orc_f16_to_f32_rs(rd16(bs));
    float dmin = orc_f16_to_f32_rs(rd16(bs + 2));
    const uint8_t *sb = bs + 4;
    uint8_t sc[8], mn[8];
    for (int i = 0; i < 4; i++) {
      sc[i] = (uint8_t)(sb[i] & 0x3F);
      sc[i + 4] = (uint8_t)((sb[i + 4] & 0x0F) | (uint8_t)((sb[i] >> 6) << 4));
      mn[i] = (uint8_t)((sb[i + 4] >> 4) | (uint8_t)((sb[i + 8] & 0x0F) << 4));
      mn[i + 4] = (uint8_t)((sb[i + 8] >> 4) | (uint8_t)(((sb[i] >> 4) & 0x0C) << 4));
    }
    const uint8_t *q = bs + 16;
    float *o = out + blk * 256;
    for (int s = 0; s < 8; s++) {
      float scv = d * (float)sc[s];
      float m = dmin * (float)mn[s];
      for (int i = 0; i < 16; i++) {
        uint8_t byte = q[s * 16 + i];
        o[s * 32 + 2 * i] = (float)(byte & 0x0F) * scv - m;
        o[s * 32 + 2 * i + 1] = (float)((byte >> 4) & 0x0F) * scv - m;
      }
    }
  }
  return ORC_OK;
}

/* gguf.rs:440-487 */
int orc_dequant_q6_k(const uint8_t *data, size_t numel, float *out) {
  if (numel % 256) return ORC_ERR_SHAPE_MISMATCH;
  for (size_t blk = 0; blk < numel / 256; blk++) {
    const uint8_t *bs = data + blk * 210;
    const uint8_t *ql = bs, *qh = bs + 128, *sc = bs + 192;
    float d = orc_f16_to_f32_rs(rd16(bs + 208));
    float *o = out + blk * 256;
    for (int sub = 0; sub < 16; sub++) {
      float scale = (float)(int8_t)sc[sub] * d;
      for (int i = 0; i < 16; i++) {
        int idx = sub * 16 + i;
        uint8_t qlb = ql[idx / 2];
        uint8_t lo = (idx % 2 == 0) ? (uint8_t)(qlb & 0x0F) : (uint8_t)(qlb >> 4);
        uint8_t hi = (uint8_t)((qh[idx / 4] >> ((idx % 4) * 2)) & 0x03);
        float qv = (float)((int)(lo | (hi << 4)) - 32);
        o[idx] = qv * scale;
      }
    }
  }
  return ORC_OK;
}

/* ======================================================================
 * A12 — zig/src/ops/matmul.zig:125-184 (sgemmTiled), :223-347 (f32GemvRow),
 *       :454-515 (micro kernels) via exports.zig:725-761
 * ==================================================================== */
static void f32_gemv_row(size_t n, size_t k, const float *a, const float *b, size_t ldb,
                         int trans_b, float *c) {
  /* every output column is its own chain, so the columns are spread over
   * OpenMP threads for large matrices (the values do not depend on it) */
  const int par = (double)n * (double)k > 1048576.0;
  if (trans_b) {
    /* 32-wide and 8-wide column blocks: per column a sequential @mulAdd chain */
    const long n32 = (long)(n - n % 32);
    const long n8 = n32 + (long)((n - (size_t)n32) / 8 * 8);
#pragma omp parallel for schedule(static) if (par)
    for (long j = 0; j < n8; j++) {
      float acc = 0.0f;
      const float *br = b + (size_t)j * ldb;
      for (size_t p = 0; p < k; p++) acc = fmaf(a[p], br[p], acc);
      c[j] = acc;
    }
    for (size_t j = (size_t)n8; j < n; j++) { /* scalar tail: unfused */
      float sum = 0.0f;
      const float *br = b + j * ldb;
      for (size_t p = 0; p < k; p++) sum += a[p] * br[p];
      c[j] = sum;
    }
  } else {
    const long n32 = (long)(n - n % 32);
#pragma omp parallel for schedule(static) if (par)
    for (long j = 0; j < n32; j++) {
      float acc = 0.0f;
      for (size_t p = 0; p < k; p++) acc = fmaf(a[p], b[p * ldb + (size_t)j], acc);
      c[j] = acc;
    }
    for (size_t j = (size_t)n32; j < n; j++) {
      float sum = 0.0f;
      for (size_t p = 0; p < k; p++) sum += a[p] * b[p * ldb + j];
      c[j] = sum;
    }
  }
}

int orc_sgemm(size_t m, size_t n, size_t k, const float *a, size_t lda, int trans_a,
              const float *b, size_t ldb, int trans_b, float *c, size_t ldc) {
  if (!a || !b || !c) return ORC_ERR_NULL_PTR;
  if (m == 0 || n == 0 || k == 0) return ORC_OK;
  if (m <= 16 && !trans_a) { /* matmul.zig:142-155: GEMV per row, C overwritten */
    for (size_t i = 0; i < m; i++) f32_gemv_row(n, k, a + i * lda, b, ldb, trans_b, c + i * ldc);
    return ORC_OK;
  }
  /* GOTO path (:157-183): C accumulates; per element a sequential chain over
   * p = 0..k-1 starting from C's value — fused (@mulAdd) inside full 8x8
   * micro-tiles, unfused in edge tiles (rows of a partial MR panel within an
   * MC=256 block, or columns of a partial NR panel within an NC=4096 block). */
  const int par = (double)m * (double)n * (double)k > 4194304.0;
#pragma omp parallel for schedule(dynamic) if (par)
  for (long ii = 0; ii < (long)m; ii++) {
    const size_t i = (size_t)ii;
    size_t ic = i / 256 * 256, mc = (m - ic < 256) ? m - ic : 256;
    size_t ir = (i - ic) / 8 * 8;
    int row_full = (mc - ir) >= 8;
    for (size_t j = 0; j < n; j++) {
      size_t jc = j / 4096 * 4096, nc = (n - jc < 4096) ? n - jc : 4096;
      size_t jr = (j - jc) / 8 * 8;
      int col_full = (nc - jr) >= 8;
      float acc = c[i * ldc + j];
      if (row_full && col_full) {
        for (size_t p = 0; p < k; p++) {
          float av = trans_a ? a[p * lda + i] : a[i * lda + p];
          float bv = trans_b ? b[j * ldb + p] : b[p * ldb + j];
          acc = fmaf(av, bv, acc);
        }
      } else {
        for (size_t p = 0; p < k; p++) {
          float av = trans_a ? a[p * lda + i] : a[i * lda + p];
          float bv = trans_b ? b[j * ldb + p] : b[p * ldb + j];
          acc += av * bv;
        }
      }
      c[i * ldc + j] = acc;
    }
  }
  return ORC_OK;
}

/* OpenMP threads for the large f32 products (the values do not depend on
 * it); 1 reproduces the reference's single-threaded timing */
#include <omp.h>
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int orc_get_threads(void) { return omp_get_max_threads(); }

/* ======================================================================
 * A14 — per-layer ops
 * ==================================================================== */
/* ops/norm.rs:8-38 with syn_vmul (exports.zig:366-375) and syn_vreduce_sum
 * (vecHsum, exports.zig:503-514: four lane accumulators over i%4, reduced
 * in lane order, then the tail). */
void orc_rmsnorm(const float *x, const float *w, float eps, size_t rows, size_t hidden,
                 float *out) {
  for (size_t r = 0; r < rows; r++) {
    const float *xr = x + r * hidden;
    float *o = out + r * hidden;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    size_t i = 0;
    for (; i + 4 <= hidden; i += 4)
      for (int l = 0; l < 4; l++) acc[l] += xr[i + l] * xr[i + l];
    float s = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    for (; i < hidden; i++) s += xr[i] * xr[i];
    float scale = 1.0f / sqrtf(s / (float)hidden + eps);
    for (size_t j = 0; j < hidden; j++) {
      float t = xr[j] * w[j];
      o[j] = t * scale;
    }
  }
}

/* models/lm/builder.rs:88-133 (no scaling): freq = 1/powf(base, 2i/hd) */
void orc_rope_tables(size_t max_pos, size_t head_dim, double base, float *cos_t,
                     float *sin_t) {
  size_t half = head_dim / 2;
  float fb = (float)base;
  for (size_t pos = 0; pos < max_pos; pos++)
    for (size_t i = 0; i < half; i++) {
      float freq = 1.0f / powf(fb, 2.0f * (float)i / (float)head_dim);
      float scaled = freq / 1.0f;
      float angle = (float)pos * scaled;
      cos_t[pos * half + i] = cosf(angle);
      sin_t[pos * half + i] = sinf(angle);
    }
}

/* ops/rope.rs:13-60 (RotateHalf) */
void orc_rope_apply(float *qk, const float *cos_t, const float *sin_t, size_t seq_len,
                    size_t num_heads, size_t head_dim, size_t pos_offset) {
  size_t half = head_dim / 2, total = num_heads * head_dim;
  for (size_t t = 0; t < seq_len; t++) {
    size_t row = (pos_offset + t) * half;
    for (size_t h = 0; h < num_heads; h++) {
      size_t base = t * total + h * head_dim;
      for (size_t i = 0; i < half; i++) {
        float cv = cos_t[row + i], sv = sin_t[row + i];
        float x1 = qk[base + i], x2 = qk[base + half + i];
        qk[base + i] = x1 * cv - x2 * sv;
        qk[base + half + i] = x2 * cv + x1 * sv;
      }
    }
  }
}

/* Rust f32::exp on Linux = glibc expf (used by silu, softmax_slice) */
float orc_expf(float x) { return expf(x); }

/* ops/activation.rs:30-32 */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops/activation.rs:117-129 */
void orc_softmax_slice(float *x, size_t n) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  if (sum > 0.0f)
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* generation/sampler.rs:217-224 — Iterator::max_by keeps the LAST maximum */
uint32_t orc_argmax(const float *logits, size_t n) {
  if (n == 0) return 0;
  size_t best = 0;
  for (size_t i = 1; i < n; i++)
    if (!(logits[i] < logits[best])) best = i;
  return (uint32_t)best;
}

/* ops/attention.rs:24-147 (no sliding window): scores, softmax, weighted V.
 * len >= 64 takes the gather + matmul_t / matmul_nn route (f32GemvRow),
 * shorter lengths the scalar loops. */
void orc_attention_decode(const float *q, const float *kcache, const float *vcache,
                          size_t seq_len, size_t num_heads, size_t num_kv_heads,
                          size_t head_dim, float *out) {
  size_t kv_dim = num_kv_heads * head_dim, groups = num_heads / num_kv_heads;
  float scale = 1.0f / sqrtf((float)head_dim);
  float *scores = (float *)malloc(seq_len * sizeof(float));
  if (seq_len >= 64) {
    float *kb = (float *)malloc(seq_len * head_dim * sizeof(float));
    float *vb = (float *)malloc(seq_len * head_dim * sizeof(float));
    for (size_t h = 0; h < num_heads; h++) {
      size_t kvh = h / groups;
      for (size_t s = 0; s < seq_len; s++) {
        memcpy(kb + s * head_dim, kcache + s * kv_dim + kvh * head_dim, head_dim * 4);
        memcpy(vb + s * head_dim, vcache + s * kv_dim + kvh * head_dim, head_dim * 4);
      }
      f32_gemv_row(seq_len, head_dim, q + h * head_dim, kb, head_dim, 1, scores);
      for (size_t s = 0; s < seq_len; s++) scores[s] *= scale;
      orc_softmax_slice(scores, seq_len);
      f32_gemv_row(head_dim, seq_len, scores, vb, head_dim, 0, out + h * head_dim);
    }
    free(kb);
    free(vb);
  } else {
    for (size_t h = 0; h < num_heads; h++) {
      size_t kvh = h / groups;
      for (size_t s = 0; s < seq_len; s++) {
        float dot = 0.0f;
        for (size_t d = 0; d < head_dim; d++)
          dot += q[h * head_dim + d] * kcache[s * kv_dim + kvh * head_dim + d];
        scores[s] = dot * scale;
      }
      orc_softmax_slice(scores, seq_len);
      for (size_t d = 0; d < head_dim; d++) {
        float sum = 0.0f;
        for (size_t s = 0; s < seq_len; s++)
          sum += scores[s] * vcache[s * kv_dim + kvh * head_dim + d];
        out[h * head_dim + d] = sum;
      }
    }
  }
  free(scores);
}

/* ffi/exports.zig:1364-1478 — single-head causal attention, TILE_Q=32
 * (zig/src/ops/attention.zig:25), online max/sum then normalise. */
int orc_fused_attention(size_t seq_q, size_t seq_k, size_t d_head, const float *q,
                        const float *k, const float *v, float *out) {
  if (!q || !k || !v || !out) return ORC_ERR_NULL_PTR;
  if (seq_q == 0 || seq_k == 0 || d_head == 0) return ORC_OK;
  const size_t TQ = 32;
  float *s_tile = (float *)malloc(TQ * seq_k * sizeof(float));
  if (!s_tile) return ORC_ERR_OUT_OF_MEMORY;
  float scale = 1.0f / sqrtf((float)d_head);
  for (size_t tq = 0; tq < seq_q; tq += TQ) {
    size_t tqs = (seq_q - tq < TQ) ? seq_q - tq : TQ;
    memset(s_tile, 0, tqs * seq_k * sizeof(float));
    orc_sgemm(tqs, seq_k, d_head, q + tq * d_head, d_head, 0, k, d_head, 1, s_tile, seq_k);
    for (size_t i = 0; i < tqs * seq_k; i++) s_tile[i] *= scale;
    for (size_t i = 0; i < tqs; i++) {
      size_t ms = tq + i + 1;
      for (size_t j = ms; j < seq_k; j++) s_tile[i * seq_k + j] = -INFINITY;
    }
    for (size_t i = 0; i < tqs; i++) {
      float *row = s_tile + i * seq_k;
      float mx = -INFINITY, se = 0.0f;
      for (size_t j = 0; j < seq_k; j++) {
        float x = row[j];
        if (x > mx) {
          se = se * expf(mx - x) + 1.0f;
          mx = x;
        } else {
          se += expf(x - mx);
        }
      }
      float inv = 1.0f / se;
      for (size_t j = 0; j < seq_k; j++) row[j] = expf(row[j] - mx) * inv;
    }
    for (size_t i = 0; i < tqs; i++) memset(out + (tq + i) * d_head, 0, d_head * sizeof(float));
    orc_sgemm(tqs, d_head, seq_k, s_tile, seq_k, 0, v, d_head, 0, out + tq * d_head, d_head);
  }
  free(s_tile);
  return ORC_OK;
}

/* ======================================================================
 * A15 — quantization/lm/int8.rs:78-709 (quantize_model, QuantizedCausalLM),
 *       ops/attention.rs:24-247, generation/pipeline.rs:197-278
 * ==================================================================== */
typedef struct {
  int8_t *w; /* [K,N] reference layout */
  float *s;  /* [N] */
  size_t n, k;
} orc_qlin;

struct orc_qlm {
  orc_lm_cfg c;
  float *embed; /* [vocab, h] f32 (tied) */
  orc_qlin *lin; /* per layer: q,k,v,o,gate,up,down */
  orc_qlin lm_head;
  /* RMSNorm gains, 1.0 until set: attention / FFN [L][h], q / k head norms
     [L][hd], final [h] (int8.rs:33-56) */
  float *attn_norm, *ffn_norm, *q_norm, *k_norm, *final_norm;
  int qk_norm;      /* 0: no head norms (empty weights skip it, norm.rs:86-88) */
  float *lm_head_f; /* untied lm_head f32 [vocab, h], or NULL (tied) */
  float *rope_cos, *rope_sin;
  float *kc, *vc; /* per layer [max_seq, kv_dim] */
  size_t cur;
};

static int qlin_from_f32(orc_qlin *q, const float *w, size_t n, size_t k) {
  q->n = n;
  q->k = k;
  q->w = (int8_t *)malloc(n * k);
  q->s = (float *)malloc(n * sizeof(float));
  if (!q->w || !q->s) return ORC_ERR_OUT_OF_MEMORY;
  orc_minmax_scales(w, n, k, q->s);
  orc_quantize_weights_int8(w, q->s, n, k, q->w);
  return ORC_OK;
}

/* QuantizedLinear::forward (int8_linear.rs:87-117): quantize rows, qgemm */
static void qlin_forward(const orc_qlin *q, const float *x, size_t m, float *y, int8_t *xq,
                         float *sx) {
  orc_quantize_per_channel_int8(x, m, q->k, xq, sx);
  orc_qgemm_int8(m, q->n, q->k, xq, q->k, q->w, q->n, y, q->n, sx, q->s);
}
static void qlin_forward_pre(const orc_qlin *q, const int8_t *xq, const float *sx, size_t m,
                             float *y) {
  orc_qgemm_int8(m, q->n, q->k, xq, q->k, q->w, q->n, y, q->n, sx, q->s);
}

orc_qlm *orc_qlm_create(const orc_lm_cfg *cfg) {
  orc_qlm *m = (orc_qlm *)calloc(1, sizeof(orc_qlm));
  if (!m) return NULL;
  m->c = *cfg;
  size_t h = cfg->hidden, hd = cfg->head_dim, L = cfg->n_layers;
  size_t kv = cfg->n_kv_heads * hd;
  m->lin = (orc_qlin *)calloc(L * 7, sizeof(orc_qlin));
  m->attn_norm = (float *)malloc(L * h * 4);
  m->ffn_norm = (float *)malloc(L * h * 4);
  m->final_norm = (float *)malloc(h * 4);
  m->q_norm = (float *)malloc(L * hd * 4);
  m->k_norm = (float *)malloc(L * hd * 4);
  for (size_t i = 0; i < L * h; i++) m->attn_norm[i] = m->ffn_norm[i] = 1.0f;
  for (size_t i = 0; i < h; i++) m->final_norm[i] = 1.0f;
  for (size_t i = 0; i < L * hd; i++) m->q_norm[i] = m->k_norm[i] = 1.0f;
  m->qk_norm = 1;
  m->rope_cos = (float *)malloc(cfg->max_seq * (hd / 2) * 4);
  m->rope_sin = (float *)malloc(cfg->max_seq * (hd / 2) * 4);
  orc_rope_tables(cfg->max_seq, hd, cfg->rope_theta, m->rope_cos, m->rope_sin);
  m->kc = (float *)calloc(L * cfg->max_seq * kv, 4);
  m->vc = (float *)calloc(L * cfg->max_seq * kv, 4);
  return m;
}

void orc_qlm_destroy(orc_qlm *m) {
  if (!m) return;
  for (size_t i = 0; i < m->c.n_layers * 7; i++) {
    free(m->lin[i].w);
    free(m->lin[i].s);
  }
  free(m->lin);
  free(m->lm_head.w);
  free(m->lm_head.s);
  free(m->embed);
  free(m->attn_norm);
  free(m->ffn_norm);
  free(m->final_norm);
  free(m->q_norm);
  free(m->k_norm);
  free(m->lm_head_f);
  free(m->rope_cos);
  free(m->rope_sin);
  free(m->kc);
  free(m->vc);
  free(m);
}

int orc_qlm_set_embed(orc_qlm *m, const float *embed) {
  size_t bytes = m->c.vocab * m->c.hidden * sizeof(float);
  m->embed = (float *)malloc(bytes);
  if (!m->embed) return ORC_ERR_OUT_OF_MEMORY;
  memcpy(m->embed, embed, bytes);
  return ORC_OK;
}

/* quantize_model per-layer step (int8.rs:85-101) */
int orc_qlm_set_layer(orc_qlm *m, size_t l, const float *wq, const float *wk, const float *wv,
                      const float *wo, const float *wg, const float *wu, const float *wd) {
  const orc_lm_cfg *c = &m->c;
  size_t h = c->hidden, qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
  orc_qlin *L = m->lin + l * 7;
  int rc = 0;
  rc |= qlin_from_f32(&L[0], wq, qd, h);
  rc |= qlin_from_f32(&L[1], wk, kvd, h);
  rc |= qlin_from_f32(&L[2], wv, kvd, h);
  rc |= qlin_from_f32(&L[3], wo, h, qd);
  rc |= qlin_from_f32(&L[4], wg, c->inter, h);
  rc |= qlin_from_f32(&L[5], wu, c->inter, h);
  rc |= qlin_from_f32(&L[6], wd, h, c->inter);
  return rc ? ORC_ERR_OUT_OF_MEMORY : ORC_OK;
}

/* Pair p of a normal stream uses draws 2p, 2p+1: a chunk starting at even
 * element e starts from state seed + e*gamma, so chunks fill in parallel. */
static void fill_normal_par(float *dst, size_t n, uint64_t seed, float stddev) {
  const size_t chunk = (size_t)1 << 20; /* even */
  long nch = (long)((n + chunk - 1) / chunk);
#pragma omp parallel for schedule(dynamic)
  for (long c = 0; c < nch; c++) {
    size_t b = (size_t)c * chunk, e = b + chunk < n ? b + chunk : n;
    orc_fill_normal(dst + b, e - b, seed + (uint64_t)b * 0x9E3779B97F4A7C15ULL, stddev);
  }
}

/* Synthetic weights: tensor id 0 = embed, 1 + 8*l + {0..6} = q,k,v,o,gate,up,down */
int orc_qlm_init_synthetic(orc_qlm *m, uint64_t seed_base, float stddev) {
  const orc_lm_cfg *c = &m->c;
  size_t h = c->hidden, qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
  m->embed = (float *)malloc(c->vocab * h * sizeof(float));
  if (!m->embed) return ORC_ERR_OUT_OF_MEMORY;
  fill_normal_par(m->embed, c->vocab * h, seed_base + 0, stddev);
  const size_t rows[7] = {qd, kvd, kvd, h, c->inter, c->inter, h};
  const size_t cols[7] = {h, h, h, qd, h, h, c->inter};
  int bad = 0;
  long total = (long)(c->n_layers * 7);
#pragma omp parallel for schedule(dynamic) reduction(| : bad)
  for (long idx = 0; idx < total; idx++) {
    size_t l = (size_t)idx / 7;
    int t = (int)(idx % 7);
    float *tmp = (float *)malloc(rows[t] * cols[t] * sizeof(float));
    if (!tmp) { bad |= 1; continue; }
    orc_fill_normal(tmp, rows[t] * cols[t], seed_base + 1 + 8 * l + (uint64_t)t, stddev);
    bad |= qlin_from_f32(&m->lin[l * 7 + t], tmp, rows[t], cols[t]) != ORC_OK;
    free(tmp);
  }
  return bad ? ORC_ERR_OUT_OF_MEMORY : ORC_OK;
}

int orc_qlm_set_norms(orc_qlm *m, size_t l, const float *attn, const float *ffn,
                      const float *q, const float *k) {
  size_t h = m->c.hidden, hd = m->c.head_dim;
  if (l >= m->c.n_layers) return ORC_ERR_INVALID_ARG;
  if (attn) memcpy(m->attn_norm + l * h, attn, h * 4);
  if (ffn) memcpy(m->ffn_norm + l * h, ffn, h * 4);
  if (q) memcpy(m->q_norm + l * hd, q, hd * 4);
  if (k) memcpy(m->k_norm + l * hd, k, hd * 4);
  return ORC_OK;
}

int orc_qlm_set_final_norm(orc_qlm *m, const float *w) {
  memcpy(m->final_norm, w, m->c.hidden * 4);
  return ORC_OK;
}

void orc_qlm_set_qk_norm(orc_qlm *m, int enabled) { m->qk_norm = enabled != 0; }

int orc_qlm_set_lm_head(orc_qlm *m, const float *w) {
  size_t bytes = m->c.vocab * m->c.hidden * 4;
  free(m->lm_head_f);
  m->lm_head_f = (float *)malloc(bytes);
  if (!m->lm_head_f) return ORC_ERR_OUT_OF_MEMORY;
  memcpy(m->lm_head_f, w, bytes);
  return ORC_OK;
}

/* lm_head quantized from its own weight, else tied to embed_tokens
   (int8.rs:125-139) */
int orc_qlm_finalize(orc_qlm *m) {
  if (!m->embed) return ORC_ERR_NULL_PTR;
  return qlin_from_f32(&m->lm_head, m->lm_head_f ? m->lm_head_f : m->embed, m->c.vocab,
                       m->c.hidden);
}

void orc_qlm_reset(orc_qlm *m) { m->cur = 0; }
size_t orc_qlm_cur_len(const orc_qlm *m) { return m->cur; }
const int8_t *orc_qlm_lm_head_weights(const orc_qlm *m) { return m->lm_head.w; }
const float *orc_qlm_lm_head_scales(const orc_qlm *m) { return m->lm_head.s; }

static void embed_rows(const orc_qlm *m, const uint32_t *ids, size_t n, float *x) {
  size_t h = m->c.hidden;
  for (size_t t = 0; t < n; t++) {
    if (ids[t] < m->c.vocab)
      memcpy(x + t * h, m->embed + (size_t)ids[t] * h, h * 4);
    else
      memset(x + t * h, 0, h * 4);
  }
}

/* FFN sub-layer, SwiGLU (int8.rs:480-505) */
static void ffn_swiglu(const orc_qlm *m, const orc_qlin *L, const float *x, size_t t, float *out,
                       int8_t *xq, float *sx, float *g, float *u) {
  size_t inter = m->c.inter;
  orc_quantize_per_channel_int8(x, t, m->c.hidden, xq, sx);
  qlin_forward_pre(&L[4], xq, sx, t, g);
  qlin_forward_pre(&L[5], xq, sx, t, u);
  for (size_t i = 0; i < t * inter; i++) g[i] = orc_silu(g[i]) * u[i];
  qlin_forward(&L[6], g, t, out, xq, sx);
}

/* Decoder layer, prefill (int8.rs:194-216, 379-426) or decode (int8.rs:242-282, 429-478).
 * prefill==1: t tokens rotated at positions 0..t-1 and appended at cache rows
 * m->cur.. (cached_attention_prefill, ops/attention.rs:173-198), attending among
 * themselves (:200-244); prefill==0: one token at position m->cur. */
static void layer_forward(orc_qlm *m, size_t l, float *x, size_t t, int prefill) {
  const orc_lm_cfg *c = &m->c;
  size_t h = c->hidden, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
  size_t qd = nh * hd, kvd = nkv * hd, inter = c->inter;
  const orc_qlin *L = m->lin + l * 7;
  size_t big = (inter > qd ? inter : qd);
  if (big < h) big = h;
  float *normed = (float *)malloc(t * h * 4);
  int8_t *xq = (int8_t *)malloc(t * big);
  float *sx = (float *)malloc(t * 4);
  float *q = (float *)malloc(t * qd * 4), *k = (float *)malloc(t * kvd * 4);
  float *v = (float *)malloc(t * kvd * 4), *attn = (float *)malloc(t * qd * 4);
  float *o = (float *)malloc(t * h * 4);
  float *g = (float *)malloc(t * inter * 4), *u = (float *)malloc(t * inter * 4);
  float *kcl = m->kc + l * c->max_seq * kvd, *vcl = m->vc + l * c->max_seq * kvd;

  orc_rmsnorm(x, m->attn_norm + l * h, c->eps, t, h, normed);
  orc_quantize_per_channel_int8(normed, t, h, xq, sx);
  qlin_forward_pre(&L[0], xq, sx, t, q);
  qlin_forward_pre(&L[1], xq, sx, t, k);
  qlin_forward_pre(&L[2], xq, sx, t, v);
  /* headwise q/k RMSNorm (norm.rs:78-93), RoPE, cache append */
  if (m->qk_norm) {
    orc_rmsnorm(q, m->q_norm + l * hd, c->eps, t * nh, hd, q);
    orc_rmsnorm(k, m->k_norm + l * hd, c->eps, t * nkv, hd, k);
  }
  size_t pos0 = prefill ? 0 : m->cur, row0 = m->cur;
  orc_rope_apply(q, m->rope_cos, m->rope_sin, t, nh, hd, pos0);
  orc_rope_apply(k, m->rope_cos, m->rope_sin, t, nkv, hd, pos0);
  memcpy(kcl + row0 * kvd, k, t * kvd * 4);
  memcpy(vcl + row0 * kvd, v, t * kvd * 4);
  if (prefill) {
    size_t groups = nh / nkv;
    float *qh = (float *)malloc(t * hd * 4), *kh = (float *)malloc(t * hd * 4);
    float *vh = (float *)malloc(t * hd * 4), *oh = (float *)malloc(t * hd * 4);
    for (size_t head = 0; head < nh; head++) {
      size_t kvh = head / groups;
      for (size_t s = 0; s < t; s++) {
        memcpy(qh + s * hd, q + s * qd + head * hd, hd * 4);
        memcpy(kh + s * hd, k + s * kvd + kvh * hd, hd * 4);
        memcpy(vh + s * hd, v + s * kvd + kvh * hd, hd * 4);
      }
      orc_fused_attention(t, t, hd, qh, kh, vh, oh);
      for (size_t s = 0; s < t; s++) memcpy(attn + s * qd + head * hd, oh + s * hd, hd * 4);
    }
    free(qh);
    free(kh);
    free(vh);
    free(oh);
  } else {
    orc_attention_decode(q, kcl, vcl, row0 + 1, nh, nkv, hd, attn);
  }
  qlin_forward(&L[3], attn, t, o, xq, sx);
  for (size_t i = 0; i < t * h; i++) x[i] = x[i] + o[i];
  orc_rmsnorm(x, m->ffn_norm + l * h, c->eps, t, h, normed);
  ffn_swiglu(m, L, normed, t, o, xq, sx, g, u);
  for (size_t i = 0; i < t * h; i++) x[i] += o[i];
  free(normed); free(xq); free(sx); free(q); free(k); free(v);
  free(attn); free(o); free(g); free(u);
}

static void lm_head_logits(orc_qlm *m, const float *xlast, float *logits) {
  size_t h = m->c.hidden;
  float *normed = (float *)malloc(h * 4);
  int8_t *xq = (int8_t *)malloc(h);
  float sx;
  orc_rmsnorm(xlast, m->final_norm, m->c.eps, 1, h, normed);
  qlin_forward(&m->lm_head, normed, 1, logits, xq, &sx);
  free(normed);
  free(xq);
}

/* QuantizedCausalLM::forward_prefill (int8.rs:593-635) into the cache as it
 * stands: the n rows go after the m->cur cached ones */
int orc_qlm_prefill_append(orc_qlm *m, const uint32_t *ids, size_t n, float *logits) {
  if (n == 0 || m->cur + n > m->c.max_seq) return ORC_ERR_INVALID_ARG;
  size_t h = m->c.hidden;
  float *x = (float *)malloc(n * h * 4);
  embed_rows(m, ids, n, x);
  for (size_t l = 0; l < m->c.n_layers; l++) layer_forward(m, l, x, n, 1);
  m->cur += n;
  lm_head_logits(m, x + (n - 1) * h, logits);
  free(x);
  return ORC_OK;
}

/* forward_prefill on a fresh ModelState (empty cache) */
int orc_qlm_prefill(orc_qlm *m, const uint32_t *ids, size_t n, float *logits) {
  if (n == 0 || n > m->c.max_seq) return ORC_ERR_INVALID_ARG;
  m->cur = 0;
  return orc_qlm_prefill_append(m, ids, n, logits);
}

/* KvCache.truncateTo (kvcache.zig:109-113) on every layer: only a shorter
 * length applies, contents are kept */
void orc_qlm_truncate(orc_qlm *m, size_t new_len) {
  if (new_len < m->cur) m->cur = new_len;
}

/* QuantizedCausalLM::forward_one (int8.rs:638-709) */
int orc_qlm_forward_one(orc_qlm *m, uint32_t token, float *logits) {
  if (m->cur >= m->c.max_seq) return ORC_ERR_INVALID_ARG;
  size_t h = m->c.hidden;
  float *x = (float *)malloc(h * 4);
  embed_rows(m, &token, 1, x);
  for (size_t l = 0; l < m->c.n_layers; l++) layer_forward(m, l, x, 1, 0);
  m->cur += 1;
  lm_head_logits(m, x, logits);
  free(x);
  return ORC_OK;
}

/* generate_cached greedy loop (pipeline.rs:197-278, stopping.rs:39-42):
 * max_new tokens from one prefill + (max_new-1) forward_one calls.
 * margins[i] = top1 - top2 logit at step i (NULL to skip). */
static float top2_margin(const float *lg, size_t n, uint32_t best) {
  float second = -INFINITY;
  for (size_t i = 0; i < n; i++)
    if (i != best && lg[i] > second) second = lg[i];
  return lg[best] - second;
}

int orc_qlm_generate(orc_qlm *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                     uint32_t *out_tokens, float *margins) {
  if (max_new == 0) return ORC_OK;
  float *logits = (float *)malloc(m->c.vocab * 4);
  int rc = orc_qlm_prefill(m, prompt, n_prompt, logits);
  if (rc) { free(logits); return rc; }
  uint32_t tok = orc_argmax(logits, m->c.vocab);
  out_tokens[0] = tok;
  if (margins) margins[0] = top2_margin(logits, m->c.vocab, tok);
  for (size_t i = 1; i < max_new; i++) {
    rc = orc_qlm_forward_one(m, tok, logits);
    if (rc) break;
    tok = orc_argmax(logits, m->c.vocab);
    out_tokens[i] = tok;
    if (margins) margins[i] = top2_margin(logits, m->c.vocab, tok);
  }
  free(logits);
  return rc;
}

/* ======================================================================
 * f32 CausalLM (models/lm/causal_lm.rs:195-278, decoder_layer.rs:51-138,
 * 590-730): weights dequantized at load (gguf.rs:217-237), every projection
 * through matmul_t (orc_sgemm with trans_b), SwiGLU through Zig swigluFused.
 * ==================================================================== */
/* zig/src/ops/silu.zig:85-114: vector part (i < n - n%4) computes
 * sig = 1/(1+exp(-g)); dst = (g*sig)*u; the scalar tail (g/(1+exp(-g)))*u */
void orc_swiglu_fused(float *dst, const float *gate, const float *up, size_t n) {
  size_t n4 = n - n % 4;
  for (size_t i = 0; i < n4; i++) {
    float g = gate[i];
    float sig = 1.0f / (1.0f + expf(-g));
    float t = g * sig;
    dst[i] = t * up[i];
  }
  for (size_t i = n4; i < n; i++) {
    float g = gate[i];
    float t = g / (1.0f + expf(-g));
    dst[i] = t * up[i];
  }
}

struct orc_flm {
  orc_lm_cfg c;
  int qk_norm;
  float *embed;
  float **w;        /* [L*7] f32 [N,K] */
  float *lm_head;   /* f32 [vocab, h] */
  /* RMSNorm gains, 1.0 until set: attention / FFN [L][h], q / k head norms
     [L][hd], final [h] (decoder_layer.rs:590-730, causal_lm.rs:267-268) */
  float *attn_nw, *ffn_nw, *q_nw, *k_nw, *final_nw;
  float *rope_cos, *rope_sin;
  float *kc, *vc;
  size_t cur;
};

static int dequant_fmt(int fmt, const uint8_t *b, size_t numel, float *out) {
  if (fmt == ORC_FMT_Q8_0) return orc_dequant_q8_0(b, numel, out);
  if (fmt == ORC_FMT_Q4_K) return orc_dequant_q4_k(b, numel, out);
  if (fmt == ORC_FMT_Q6_K) return orc_dequant_q6_k(b, numel, out);
  return ORC_ERR_INVALID_ARG;
}

orc_flm *orc_flm_create(const orc_lm_cfg *cfg, int qk_norm) {
  orc_flm *m = (orc_flm *)calloc(1, sizeof(orc_flm));
  if (!m) return NULL;
  m->c = *cfg;
  m->qk_norm = qk_norm;
  size_t h = cfg->hidden, hd = cfg->head_dim, kv = cfg->n_kv_heads * hd;
  m->w = (float **)calloc(cfg->n_layers * 7, sizeof(float *));
  size_t L = cfg->n_layers;
  m->attn_nw = (float *)malloc(L * h * 4);
  m->ffn_nw = (float *)malloc(L * h * 4);
  m->q_nw = (float *)malloc(L * hd * 4);
  m->k_nw = (float *)malloc(L * hd * 4);
  m->final_nw = (float *)malloc(h * 4);
  for (size_t i = 0; i < L * h; i++) m->attn_nw[i] = m->ffn_nw[i] = 1.0f;
  for (size_t i = 0; i < L * hd; i++) m->q_nw[i] = m->k_nw[i] = 1.0f;
  for (size_t i = 0; i < h; i++) m->final_nw[i] = 1.0f;
  m->rope_cos = (float *)malloc(cfg->max_seq * (hd / 2) * 4);
  m->rope_sin = (float *)malloc(cfg->max_seq * (hd / 2) * 4);
  orc_rope_tables(cfg->max_seq, hd, cfg->rope_theta, m->rope_cos, m->rope_sin);
  m->kc = (float *)calloc(cfg->n_layers * cfg->max_seq * kv, 4);
  m->vc = (float *)calloc(cfg->n_layers * cfg->max_seq * kv, 4);
  return m;
}

void orc_flm_destroy(orc_flm *m) {
  if (!m) return;
  for (size_t i = 0; i < m->c.n_layers * 7; i++) free(m->w[i]);
  free(m->w);
  free(m->embed);
  free(m->lm_head);
  free(m->attn_nw);
  free(m->ffn_nw);
  free(m->q_nw);
  free(m->k_nw);
  free(m->final_nw);
  free(m->rope_cos);
  free(m->rope_sin);
  free(m->kc);
  free(m->vc);
  free(m);
}

int orc_flm_set_embed(orc_flm *m, const float *embed) {
  size_t bytes = m->c.vocab * m->c.hidden * 4;
  m->embed = (float *)malloc(bytes);
  if (!m->embed) return ORC_ERR_OUT_OF_MEMORY;
  memcpy(m->embed, embed, bytes);
  return ORC_OK;
}

static void flm_proj_shape(const orc_flm *m, int proj, size_t *n, size_t *k) {
  const orc_lm_cfg *c = &m->c;
  size_t h = c->hidden, qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
  const size_t rows[7] = {qd, kvd, kvd, h, c->inter, c->inter, h};
  const size_t cols[7] = {h, h, h, qd, h, h, c->inter};
  *n = rows[proj];
  *k = cols[proj];
}

int orc_flm_set_proj(orc_flm *m, size_t layer, int proj, int fmt, const uint8_t *bytes) {
  if (layer >= m->c.n_layers || proj < 0 || proj > 6) return ORC_ERR_INVALID_ARG;
  size_t n, k;
  flm_proj_shape(m, proj, &n, &k);
  float *w = (float *)malloc(n * k * 4);
  if (!w) return ORC_ERR_OUT_OF_MEMORY;
  int rc = dequant_fmt(fmt, bytes, n * k, w);
  if (rc) { free(w); return rc; }
  free(m->w[layer * 7 + proj]);
  m->w[layer * 7 + proj] = w;
  return ORC_OK;
}

int orc_flm_set_lm_head(orc_flm *m, int fmt, const uint8_t *bytes) {
  size_t n = m->c.vocab * m->c.hidden;
  m->lm_head = (float *)malloc(n * 4);
  if (!m->lm_head) return ORC_ERR_OUT_OF_MEMORY;
  return dequant_fmt(fmt, bytes, n, m->lm_head);
}

int orc_flm_set_norms(orc_flm *m, size_t layer, const float *attn, const float *ffn,
                      const float *q, const float *k) {
  size_t h = m->c.hidden, hd = m->c.head_dim;
  if (layer >= m->c.n_layers) return ORC_ERR_INVALID_ARG;
  if (attn) memcpy(m->attn_nw + layer * h, attn, h * 4);
  if (ffn) memcpy(m->ffn_nw + layer * h, ffn, h * 4);
  if (q) memcpy(m->q_nw + layer * hd, q, hd * 4);
  if (k) memcpy(m->k_nw + layer * hd, k, hd * 4);
  return ORC_OK;
}

int orc_flm_set_final_norm(orc_flm *m, const float *w) {
  memcpy(m->final_nw, w, m->c.hidden * 4);
  return ORC_OK;
}

void orc_flm_reset(orc_flm *m) { m->cur = 0; }

static void flm_matmul_t(const float *x, const float *w, size_t m, size_t k, size_t n, float *y) {
  memset(y, 0, m * n * 4);
  orc_sgemm(m, n, k, x, k, 0, w, k, 1, y, n);
}

static void flm_layer(orc_flm *m, size_t l, float *x, size_t t, int prefill) {
  const orc_lm_cfg *c = &m->c;
  size_t h = c->hidden, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
  size_t qd = nh * hd, kvd = nkv * hd, inter = c->inter;
  float **W = m->w + l * 7;
  float *normed = (float *)malloc(t * h * 4);
  float *q = (float *)malloc(t * qd * 4), *k = (float *)malloc(t * kvd * 4);
  float *v = (float *)malloc(t * kvd * 4), *attn = (float *)malloc(t * qd * 4);
  float *o = (float *)malloc(t * h * 4);
  float *g = (float *)malloc(t * inter * 4), *u = (float *)malloc(t * inter * 4);
  float *hb = (float *)malloc(t * inter * 4);
  float *kcl = m->kc + l * c->max_seq * kvd, *vcl = m->vc + l * c->max_seq * kvd;

  orc_rmsnorm(x, m->attn_nw + l * h, c->eps, t, h, normed);
  flm_matmul_t(normed, W[0], t, h, qd, q);
  flm_matmul_t(normed, W[1], t, h, kvd, k);
  flm_matmul_t(normed, W[2], t, h, kvd, v);
  if (m->qk_norm) {
    orc_rmsnorm(q, m->q_nw + l * hd, c->eps, t * nh, hd, q);
    orc_rmsnorm(k, m->k_nw + l * hd, c->eps, t * nkv, hd, k);
  }
  /* prefill: rotated at 0..t-1, appended at rows m->cur.. (as the INT8 layer) */
  size_t pos0 = prefill ? 0 : m->cur, row0 = m->cur;
  orc_rope_apply(q, m->rope_cos, m->rope_sin, t, nh, hd, pos0);
  orc_rope_apply(k, m->rope_cos, m->rope_sin, t, nkv, hd, pos0);
  memcpy(kcl + row0 * kvd, k, t * kvd * 4);
  memcpy(vcl + row0 * kvd, v, t * kvd * 4);
  if (prefill) {
    size_t groups = nh / nkv;
    float *qh = (float *)malloc(t * hd * 4), *kh = (float *)malloc(t * hd * 4);
    float *vh = (float *)malloc(t * hd * 4), *oh = (float *)malloc(t * hd * 4);
    for (size_t head = 0; head < nh; head++) {
      size_t kvh = head / groups;
      for (size_t s = 0; s < t; s++) {
        memcpy(qh + s * hd, q + s * qd + head * hd, hd * 4);
        memcpy(kh + s * hd, k + s * kvd + kvh * hd, hd * 4);
        memcpy(vh + s * hd, v + s * kvd + kvh * hd, hd * 4);
      }
      orc_fused_attention(t, t, hd, qh, kh, vh, oh);
      for (size_t s = 0; s < t; s++) memcpy(attn + s * qd + head * hd, oh + s * hd, hd * 4);
    }
    free(qh); free(kh); free(vh); free(oh);
  } else {
    orc_attention_decode(q, kcl, vcl, row0 + 1, nh, nkv, hd, attn);
  }
  flm_matmul_t(attn, W[3], t, qd, h, o);
  for (size_t i = 0; i < t * h; i++) x[i] = x[i] + o[i];
  orc_rmsnorm(x, m->ffn_nw + l * h, c->eps, t, h, normed);
  flm_matmul_t(normed, W[4], t, h, inter, g);
  flm_matmul_t(normed, W[5], t, h, inter, u);
  orc_swiglu_fused(hb, g, u, t * inter);
  flm_matmul_t(hb, W[6], t, inter, h, o);
  for (size_t i = 0; i < t * h; i++) x[i] += o[i];
  free(normed); free(q); free(k); free(v); free(attn); free(o); free(g); free(u); free(hb);
}

static void flm_head(orc_flm *m, const float *xlast, float *logits) {
  size_t h = m->c.hidden;
  float *normed = (float *)malloc(h * 4);
  orc_rmsnorm(xlast, m->final_nw, m->c.eps, 1, h, normed);
  flm_matmul_t(normed, m->lm_head, 1, h, m->c.vocab, logits);
  free(normed);
}

/* CausalLM::forward_prefill (causal_lm.rs:195-239) into the cache as it
 * stands: rows appended after the m->cur cached ones */
int orc_flm_prefill_append(orc_flm *m, const uint32_t *ids, size_t n, float *logits) {
  if (n == 0 || m->cur + n > m->c.max_seq) return ORC_ERR_INVALID_ARG;
  size_t h = m->c.hidden;
  float *x = (float *)malloc(n * h * 4);
  for (size_t t = 0; t < n; t++) {
    if (ids[t] < m->c.vocab) memcpy(x + t * h, m->embed + (size_t)ids[t] * h, h * 4);
    else memset(x + t * h, 0, h * 4);
  }
  for (size_t l = 0; l < m->c.n_layers; l++) flm_layer(m, l, x, n, 1);
  m->cur += n;
  flm_head(m, x + (n - 1) * h, logits);
  free(x);
  return ORC_OK;
}

void orc_flm_truncate(orc_flm *m, size_t new_len) {
  if (new_len < m->cur) m->cur = new_len;  /* kvcache.zig:109-113 */
}

size_t orc_flm_cur_len(const orc_flm *m) { return m->cur; }

/* CausalLM::forward_one_draft (causal_lm.rs:283-323): the first n_draft
 * layers, zero K and V rows appended to the others, final norm, lm_head */
int orc_flm_forward_one_draft(orc_flm *m, uint32_t token, size_t n_draft, float *logits) {
  if (m->cur >= m->c.max_seq) return ORC_ERR_INVALID_ARG;
  size_t h = m->c.hidden, kvd = m->c.n_kv_heads * m->c.head_dim;
  size_t n = n_draft < m->c.n_layers ? n_draft : m->c.n_layers;
  float *x = (float *)malloc(h * 4);
  if (token < m->c.vocab) memcpy(x, m->embed + (size_t)token * h, h * 4);
  else memset(x, 0, h * 4);
  for (size_t l = 0; l < n; l++) flm_layer(m, l, x, 1, 0);
  for (size_t l = n; l < m->c.n_layers; l++) {
    memset(m->kc + (l * m->c.max_seq + m->cur) * kvd, 0, kvd * 4);
    memset(m->vc + (l * m->c.max_seq + m->cur) * kvd, 0, kvd * 4);
  }
  m->cur += 1;
  flm_head(m, x, logits);
  free(x);
  return ORC_OK;
}

int orc_flm_prefill(orc_flm *m, const uint32_t *ids, size_t n, float *logits) {
  if (n == 0 || n > m->c.max_seq) return ORC_ERR_INVALID_ARG;
  m->cur = 0;
  return orc_flm_prefill_append(m, ids, n, logits);
}

int orc_flm_forward_one(orc_flm *m, uint32_t token, float *logits) {
  if (m->cur >= m->c.max_seq) return ORC_ERR_INVALID_ARG;
  size_t h = m->c.hidden;
  float *x = (float *)malloc(h * 4);
  if (token < m->c.vocab) memcpy(x, m->embed + (size_t)token * h, h * 4);
  else memset(x, 0, h * 4);
  for (size_t l = 0; l < m->c.n_layers; l++) flm_layer(m, l, x, 1, 0);
  m->cur += 1;
  flm_head(m, x, logits);
  free(x);
  return ORC_OK;
}

int orc_flm_generate(orc_flm *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                     uint32_t *out_tokens, float *margins) {
  if (max_new == 0) return ORC_OK;
  float *logits = (float *)malloc(m->c.vocab * 4);
  int rc = orc_flm_prefill(m, prompt, n_prompt, logits);
  if (rc) { free(logits); return rc; }
  uint32_t tok = orc_argmax(logits, m->c.vocab);
  out_tokens[0] = tok;
  if (margins) margins[0] = top2_margin(logits, m->c.vocab, tok);
  for (size_t i = 1; i < max_new; i++) {
    rc = orc_flm_forward_one(m, tok, logits);
    if (rc) break;
    tok = orc_argmax(logits, m->c.vocab);
    out_tokens[i] = tok;
    if (margins) margins[i] = top2_margin(logits, m->c.vocab, tok);
  }
  free(logits);
  return rc;
}

/* ======================================================================
 * INT8 Mamba (quantization/ssm/int8_mamba.rs:21-224)
 * ==================================================================== */
/* ops/activation.rs:88-90 */
float orc_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

/* ops/pure_rust_ops.rs:96-112: one sequential sum of squares */
void orc_rmsnorm_seq(const float *x, const float *w, float eps, size_t hidden, float *out) {
  float s = 0.0f;
  for (size_t i = 0; i < hidden; i++) {
    float t = x[i] * x[i];
    s = s + t;
  }
  float scale = 1.0f / sqrtf(s / (float)hidden + eps);
  for (size_t j = 0; j < hidden; j++) {
    float t = x[j] * w[j];
    out[j] = t * scale;
  }
}

/* zig/src/ops/selective_scan.zig:30-90 */
void orc_selective_scan_step(const float *x, const float *delta, const float *a_log,
                             const float *b, const float *c, const float *d, float *state,
                             float *y, size_t d_inner, size_t d_state) {
  for (size_t i = 0; i < d_inner; i++) {
    float dt = delta[i], xi = x[i];
    float dt_x = dt * xi;
    float yi = 0.0f;
    float *h = state + i * d_state;
    const float *al = a_log + i * d_state;
    size_t j = 0;
    for (; j + 4 <= d_state; j += 4) {
      float contrib[4];
      for (int l = 0; l < 4; l++) {
        float e = expf(al[j + l]);
        float ad = expf(-dt * e);
        float p1 = ad * h[j + l], p2 = dt_x * b[j + l];
        float hn = p1 + p2;
        h[j + l] = hn;
        contrib[l] = c[j + l] * hn;
      }
      yi += ((contrib[0] + contrib[1]) + contrib[2]) + contrib[3];
    }
    for (; j < d_state; j++) {
      float a = -expf(al[j]);
      float ad = expf(dt * a);
      float hn = ad * h[j] + dt * b[j] * xi;
      h[j] = hn;
      yi += c[j] * hn;
    }
    y[i] = yi + d[i] * xi;
  }
}

typedef struct {
  orc_qlin in_proj, out_proj;            /* [2*d_inner, d_model], [d_model, d_inner] */
  float *conv_w, *conv_b;                /* [d_inner, d_conv], [d_inner] */
  float *x_proj, *dt_proj, *dt_bias;     /* [dt_rank+2*d_state, d_inner], [d_inner, dt_rank], [d_inner] */
  float *a_log, *d_param, *norm_w;       /* [d_inner, d_state], [d_inner], [d_model] */
  float *conv_state, *ssm_state;         /* [d_inner, d_conv], [d_inner, d_state] */
  orc_qlin x_i8, dt_i8;                  /* INT8 x_proj / dt_proj (int8_xdt variant) */
} orc_mblock;

struct orc_mamba {
  orc_mamba_cfg c;
  float *embed, *final_norm;
  orc_qlin lm_dummy;
  orc_mblock *blk;
  int int8_xdt; /* x_proj and dt_proj as QuantizedLinear */
};

orc_mamba *orc_mamba_create(const orc_mamba_cfg *cfg) {
  orc_mamba *m = (orc_mamba *)calloc(1, sizeof(orc_mamba));
  if (!m) return NULL;
  m->c = *cfg;
  m->blk = (orc_mblock *)calloc(cfg->n_layers, sizeof(orc_mblock));
  return m;
}

void orc_mamba_destroy(orc_mamba *m) {
  if (!m) return;
  for (size_t l = 0; l < m->c.n_layers; l++) {
    orc_mblock *b = &m->blk[l];
    free(b->in_proj.w); free(b->in_proj.s); free(b->out_proj.w); free(b->out_proj.s);
    free(b->conv_w); free(b->conv_b); free(b->x_proj); free(b->dt_proj); free(b->dt_bias);
    free(b->a_log); free(b->d_param); free(b->norm_w); free(b->conv_state); free(b->ssm_state);
    free(b->x_i8.w); free(b->x_i8.s); free(b->dt_i8.w); free(b->dt_i8.s);
  }
  free(m->blk);
  free(m->embed);
  free(m->final_norm);
  free(m);
}

/* Synthetic weights (harness spec): embed (tied lm_head) id 0, block l:
 * 1+16l+{0 in_proj, 1 conv1d, 2 x_proj, 3 dt_proj, 4 out_proj} ~ N(0, 0.02);
 * conv bias 0, dt bias log(expm1(0.01)), a_log[i][s] = log(s+1), D = 1, norms 1. */
int orc_mamba_init_synthetic(orc_mamba *m, uint64_t seed_base) {
  return orc_mamba_init_synthetic_std(m, seed_base, 0.02f);
}

/* the same seed spec with `std` for the projections and the conv taps (the
   embedding keeps 0.02) */
int orc_mamba_init_synthetic_std(orc_mamba *m, uint64_t seed_base, float std) {
  const orc_mamba_cfg *c = &m->c;
  size_t dm = c->d_model, di = c->d_inner, ds = c->d_state, dc = c->d_conv, dr = c->dt_rank;
  m->embed = (float *)malloc(c->vocab * dm * 4);
  m->final_norm = (float *)malloc(dm * 4);
  if (!m->embed || !m->final_norm) return ORC_ERR_OUT_OF_MEMORY;
  fill_normal_par(m->embed, c->vocab * dm, seed_base, 0.02f);
  for (size_t i = 0; i < dm; i++) m->final_norm[i] = 1.0f;
  const float dt_bias = logf(expm1f(0.01f));
  int bad = 0;
#pragma omp parallel for schedule(dynamic) reduction(| : bad)
  for (long ll = 0; ll < (long)c->n_layers; ll++) {
    size_t l = (size_t)ll;
    orc_mblock *b = &m->blk[l];
    uint64_t sb = seed_base + 1 + 16 * l;
    float *w = (float *)malloc(2 * di * dm * 4);
    orc_fill_normal(w, 2 * di * dm, sb + 0, std);
    bad |= qlin_from_f32(&b->in_proj, w, 2 * di, dm);
    orc_fill_normal(w, dm * di, sb + 4, std);
    bad |= qlin_from_f32(&b->out_proj, w, dm, di);
    free(w);
    b->conv_w = (float *)malloc(di * dc * 4);
    orc_fill_normal(b->conv_w, di * dc, sb + 1, std);
    b->conv_b = (float *)calloc(di, 4);
    b->x_proj = (float *)malloc((dr + 2 * ds) * di * 4);
    orc_fill_normal(b->x_proj, (dr + 2 * ds) * di, sb + 2, std);
    b->dt_proj = (float *)malloc(di * dr * 4);
    orc_fill_normal(b->dt_proj, di * dr, sb + 3, std);
    b->dt_bias = (float *)malloc(di * 4);
    b->a_log = (float *)malloc(di * ds * 4);
    b->d_param = (float *)malloc(di * 4);
    b->norm_w = (float *)malloc(dm * 4);
    for (size_t i = 0; i < di; i++) {
      b->dt_bias[i] = dt_bias;
      b->d_param[i] = 1.0f;
      for (size_t s2 = 0; s2 < ds; s2++) b->a_log[i * ds + s2] = logf((float)(s2 + 1));
    }
    for (size_t i = 0; i < dm; i++) b->norm_w[i] = 1.0f;
    b->conv_state = (float *)calloc(di * dc, 4);
    b->ssm_state = (float *)calloc(di * ds, 4);
  }
  return bad ? ORC_ERR_OUT_OF_MEMORY : ORC_OK;
}

/* The config-5 variant: x_proj and dt_proj become W8A8 QuantizedLinears of
   their f32 weights, built with the same from_f32 as in_proj/out_proj
   (int8_mamba.rs:136-171 -> int8_linear.rs:35-70), and run through the same
   forward (int8_linear.rs:87-117: A1 row quantizer, exact i32 products,
   (f32(acc)*sx)*sw).  dt_proj's input is the dt_rank head of x_proj's
   output, as in ssm_forward_step (int8_mamba.rs:59-75).  The reference keeps
   these two projections f32 (:33-34); this is the variant the benchmark
   config names.  Call after init; idempotent. */
int orc_mamba_set_int8_xdt(orc_mamba *m) {
  const orc_mamba_cfg *c = &m->c;
  size_t di = c->d_inner, ds = c->d_state, dr = c->dt_rank;
  if (m->int8_xdt) return ORC_OK;
  for (size_t l = 0; l < c->n_layers; l++) {
    orc_mblock *b = &m->blk[l];
    if (!b->x_proj || !b->dt_proj) return ORC_ERR_INVALID_ARG;
    if (qlin_from_f32(&b->x_i8, b->x_proj, dr + 2 * ds, di)) return ORC_ERR_OUT_OF_MEMORY;
    if (qlin_from_f32(&b->dt_i8, b->dt_proj, di, dr)) return ORC_ERR_OUT_OF_MEMORY;
  }
  m->int8_xdt = 1;
  return ORC_OK;
}

void orc_mamba_reset(orc_mamba *m) {
  for (size_t l = 0; l < m->c.n_layers; l++) {
    memset(m->blk[l].conv_state, 0, m->c.d_inner * m->c.d_conv * 4);
    memset(m->blk[l].ssm_state, 0, m->c.d_inner * m->c.d_state * 4);
  }
}

/* QuantizedMambaBlock::conv1d_step (int8_mamba.rs:43-56): per channel the
   d_conv-long window shifts left by one, the new sample enters at the end,
   and out = sum_k window[k] * w[k] (in k order) + bias */
void orc_conv1d_step(const float *x, const float *w, const float *bias, float *state,
                     size_t d_inner, size_t d_conv, float *out) {
  for (size_t i = 0; i < d_inner; i++) {
    float *buf = state + i * d_conv;
    memmove(buf, buf + 1, (d_conv - 1) * 4);
    buf[d_conv - 1] = x[i];
    const float *wi = w + i * d_conv;
    float sum = 0.0f;
    for (size_t k = 0; k < d_conv; k++) {
      float t = buf[k] * wi[k];
      sum = sum + t;
    }
    out[i] = sum + bias[i];
  }
}

/* QuantizedMambaBlock::forward_one (int8_mamba.rs:78-109) */
static void mamba_block_one(const orc_mamba *m, orc_mblock *b, const float *hid, float *out) {
  const orc_mamba_cfg *c = &m->c;
  size_t dm = c->d_model, di = c->d_inner, ds = c->d_state, dc = c->d_conv, dr = c->dt_rank;
  float *normed = (float *)malloc(dm * 4), *proj = (float *)malloc(2 * di * 4);
  float *xc = (float *)malloc(di * 4), *xp = (float *)malloc((dr + 2 * ds) * 4);
  float *dtp = (float *)malloc(di * 4), *delta = (float *)malloc(di * 4);
  float *y = (float *)malloc(di * 4), *g = (float *)malloc(di * 4), *o = (float *)malloc(dm * 4);
  size_t xqn = 2 * di > dm ? 2 * di : dm;
  int8_t *xq = (int8_t *)malloc(xqn > dr + 2 * ds ? xqn : dr + 2 * ds);
  float sx;
  orc_rmsnorm_seq(hid, b->norm_w, c->eps, dm, normed);
  qlin_forward(&b->in_proj, normed, 1, proj, xq, &sx);
  orc_conv1d_step(proj, b->conv_w, b->conv_b, b->conv_state, di, dc, xc);
  for (size_t i = 0; i < di; i++) xc[i] = orc_silu(xc[i]);
  if (m->int8_xdt) {
    /* config-5 variant: both projections through QuantizedLinear::forward */
    qlin_forward(&b->x_i8, xc, 1, xp, xq, &sx);
    qlin_forward(&b->dt_i8, xp, 1, dtp, xq, &sx);
  } else {
    /* ssm_forward_step :59-75: x_proj and dt_proj are f32 matmul_t */
    memset(xp, 0, (dr + 2 * ds) * 4);
    orc_sgemm(1, dr + 2 * ds, di, xc, di, 0, b->x_proj, di, 1, xp, dr + 2 * ds);
    memset(dtp, 0, di * 4);
    orc_sgemm(1, di, dr, xp, dr, 0, b->dt_proj, dr, 1, dtp, di);
  }
  for (size_t i = 0; i < di; i++) delta[i] = orc_softplus(dtp[i] + b->dt_bias[i]);
  orc_selective_scan_step(xc, delta, b->a_log, xp + dr, xp + dr + ds, b->d_param, b->ssm_state, y,
                          di, ds);
  for (size_t i = 0; i < di; i++) g[i] = orc_silu(proj[di + i]) * y[i];
  qlin_forward(&b->out_proj, g, 1, o, xq, &sx);
  for (size_t i = 0; i < dm; i++) out[i] = o[i] + hid[i];
  free(normed); free(proj); free(xc); free(xp); free(dtp); free(delta); free(y); free(g);
  free(o); free(xq);
}

static void mamba_token(orc_mamba *m, uint32_t token, float *hid) {
  size_t dm = m->c.d_model;
  float *tmp = (float *)malloc(dm * 4);
  if (token < m->c.vocab) memcpy(hid, m->embed + (size_t)token * dm, dm * 4);
  else memset(hid, 0, dm * 4);
  for (size_t l = 0; l < m->c.n_layers; l++) {
    mamba_block_one(m, &m->blk[l], hid, tmp);
    memcpy(hid, tmp, dm * 4);
  }
  free(tmp);
}

static void mamba_logits(orc_mamba *m, const float *hid, float *logits) {
  size_t dm = m->c.d_model;
  float *normed = (float *)malloc(dm * 4);
  orc_rmsnorm_seq(hid, m->final_norm, m->c.eps, dm, normed);
  memset(logits, 0, m->c.vocab * 4);
  orc_sgemm(1, m->c.vocab, dm, normed, dm, 0, m->embed, dm, 1, logits, m->c.vocab);
  free(normed);
}

/* prefill :177-203 (per-token loop inside each block = token-major order) */
int orc_mamba_prefill(orc_mamba *m, const uint32_t *ids, size_t n, float *logits) {
  if (n == 0) return ORC_ERR_INVALID_ARG;
  float *hid = (float *)malloc(m->c.d_model * 4);
  for (size_t t = 0; t < n; t++) mamba_token(m, ids[t], hid);
  mamba_logits(m, hid, logits);
  free(hid);
  return ORC_OK;
}

int orc_mamba_decode_one(orc_mamba *m, uint32_t token, float *logits) {
  float *hid = (float *)malloc(m->c.d_model * 4);
  mamba_token(m, token, hid);
  mamba_logits(m, hid, logits);
  free(hid);
  return ORC_OK;
}

int orc_mamba_generate(orc_mamba *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                       uint32_t *out_tokens, float *margins) {
  if (max_new == 0) return ORC_OK;
  float *logits = (float *)malloc(m->c.vocab * 4);
  int rc = orc_mamba_prefill(m, prompt, n_prompt, logits);
  if (rc) { free(logits); return rc; }
  uint32_t tok = orc_argmax(logits, m->c.vocab);
  out_tokens[0] = tok;
  if (margins) margins[0] = top2_margin(logits, m->c.vocab, tok);
  for (size_t i = 1; i < max_new; i++) {
    orc_mamba_decode_one(m, tok, logits);
    tok = orc_argmax(logits, m->c.vocab);
    out_tokens[i] = tok;
    if (margins) margins[i] = top2_margin(logits, m->c.vocab, tok);
  }
  free(logits);
  return ORC_OK;
}

/* ======================================================================
 * Sampling (generation/sampler.rs) and the random stream that feeds it.
 * ====================================================================== */

/* RepetitionPenalty::apply (sampler.rs:130-149): every occurrence in the
 * history divides a positive logit by the penalty or multiplies a
 * non-positive one, in history order. */
void orc_repetition_penalty(float *logits, size_t n, const uint32_t *hist, size_t nh,
                            float penalty) {
  if (fabsf(penalty - 1.0f) < FLT_EPSILON) return;
  for (size_t i = 0; i < nh; i++) {
    const size_t idx = hist[i];
    if (idx < n) {
      if (logits[idx] > 0.0f) logits[idx] /= penalty;
      else logits[idx] *= penalty;
    }
  }
}

/* f32::max fold from -inf (sampler.rs:234, 275-278): NaN-ignoring */
static float max_fold(const float *x, size_t n) {
  float m = -INFINITY;
  for (size_t i = 0; i < n; i++) m = fmaxf(m, x[i]);
  return m;
}

/* softmax_inplace (sampler.rs:233-245): exp(l - max), sequential sum in index
 * order, division when the sum is positive */
void orc_softmax_inplace(float *x, size_t n) {
  const float mx = max_fold(x, n);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  if (sum > 0.0f)
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

static int cmp_desc_f32(const void *a, const void *b) {
  const float x = *(const float *)a, y = *(const float *)b;
  return x > y ? -1 : x < y ? 1 : 0;
}

/* top_k_filter (sampler.rs:262-276): the k-th largest value is the
 * threshold, every logit below it becomes -inf */
void orc_top_k_filter(float *logits, size_t n, size_t k) {
  if (k > n) k = n;
  if (k == 0) return;
  float *s = (float *)malloc(n * sizeof(float));
  memcpy(s, logits, n * sizeof(float));
  qsort(s, n, sizeof(float), cmp_desc_f32);
  const float thr = s[k - 1];
  free(s);
  for (size_t i = 0; i < n; i++)
    if (logits[i] < thr) logits[i] = -INFINITY;
}

typedef struct {
  float p;
  uint32_t i;
} orc_prob_idx;

/* probabilities descending; equal probabilities by index ascending (the
 * reference's unstable sort leaves their order unspecified) */
static int cmp_prob_desc(const void *a, const void *b) {
  const orc_prob_idx *x = (const orc_prob_idx *)a, *y = (const orc_prob_idx *)b;
  if (x->p > y->p) return -1;
  if (x->p < y->p) return 1;
  return x->i < y->i ? -1 : x->i > y->i ? 1 : 0;
}

/* top_p_filter (sampler.rs:279-319): softmax, sort by probability
 * descending, keep tokens until the cumulative probability reaches p */
void orc_top_p_filter(float *logits, size_t n, float p) {
  orc_prob_idx *pr = (orc_prob_idx *)malloc(n * sizeof(orc_prob_idx));
  float *v = (float *)malloc(n * sizeof(float));
  memcpy(v, logits, n * sizeof(float));
  orc_softmax_inplace(v, n);
  for (size_t i = 0; i < n; i++) {
    pr[i].p = v[i];
    pr[i].i = (uint32_t)i;
  }
  qsort(pr, n, sizeof(orc_prob_idx), cmp_prob_desc);
  unsigned char *keep = (unsigned char *)calloc(n, 1);
  float cum = 0.0f;
  for (size_t j = 0; j < n; j++) {
    keep[pr[j].i] = 1;
    cum += pr[j].p;
    if (cum >= p) break;
  }
  for (size_t i = 0; i < n; i++)
    if (!keep[i]) logits[i] = -INFINITY;
  free(keep);
  free(v);
  free(pr);
}

/* categorical_sample (sampler.rs:248-259) with the uniform draw u given */
static uint32_t categorical(const float *probs, size_t n, float u) {
  float cum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    cum += probs[i];
    if (u < cum) return (uint32_t)i;
  }
  return (uint32_t)(n - 1);
}

/* CombinedSampler::sample_with_history (sampler.rs:161-201): repetition
 * penalty -> temperature -> top-k -> top-p -> softmax + categorical draw.
 * logits are modified in place as in the reference; u is the draw
 * rng.gen::<f32>() the reference would take (used only on the sampling
 * route). */
uint32_t orc_sample_combined(float *logits, size_t n, const uint32_t *hist, size_t nh,
                             float temperature, size_t top_k, float top_p, float rep_penalty,
                             float u) {
  if (fabsf(rep_penalty - 1.0f) > FLT_EPSILON)
    orc_repetition_penalty(logits, n, hist, nh, rep_penalty);
  if (temperature <= 0.0f) return orc_argmax(logits, n);
  const float inv_t = 1.0f / temperature;
  for (size_t i = 0; i < n; i++) logits[i] *= inv_t;
  if (top_k > 0 && top_k < n) {
    if (top_k == 1) return orc_argmax(logits, n);
    orc_top_k_filter(logits, n, top_k);
  }
  if (top_p > 0.0f && top_p < 1.0f) orc_top_p_filter(logits, n, top_p);
  orc_softmax_inplace(logits, n);
  return categorical(logits, n, u);
}

/* ---- the random stream: rand 0.8.5 StdRng = rand_chacha 0.3.1 ChaCha12Rng,
 * seeded by rand_core 0.6.4 SeedableRng::seed_from_u64 (third-party crates,
 * not vendored in the reference; restated from their published algorithms,
 * parity unpinned beyond the ChaCha block test vector of RFC 8439 and
 * PCG32's demo stream) ---- */

static uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

/* one ChaCha block with a 64-bit block counter (words 12-13) and a 64-bit
 * stream id (words 14-15), `rounds` rounds (20 for ChaCha20, 12 for
 * ChaCha12) */
void orc_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds,
                      uint32_t out[16]) {
  uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                    key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                    (uint32_t)counter, (uint32_t)(counter >> 32),
                    (uint32_t)stream, (uint32_t)(stream >> 32)};
  uint32_t x[16];
  memcpy(x, s, sizeof(x));
#define QR(a, b, c, d)                 \
  x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 16); \
  x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 12); \
  x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 8);  \
  x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 7);
  for (int r = 0; r < rounds; r += 2) {
    QR(0, 4, 8, 12) QR(1, 5, 9, 13) QR(2, 6, 10, 14) QR(3, 7, 11, 15)
    QR(0, 5, 10, 15) QR(1, 6, 11, 12) QR(2, 7, 8, 13) QR(3, 4, 9, 14)
  }
#undef QR
  for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

/* PCG32's LCG step (multiplier 6364136223846793005, increment inc) and its
 * XSH-RR output function (O'Neill's pcg32_random_r), exported so that the
 * tests can pin both against the PCG reference implementation's published
 * demo stream */
uint64_t orc_pcg32_step(uint64_t state, uint64_t inc) {
  return state * 6364136223846793005ull + inc;
}
uint32_t orc_pcg32_xsh_rr(uint64_t state) {
  const uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
  const uint32_t rot = (uint32_t)(state >> 59);
  return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

/* seed_from_u64: the 32-byte seed from a PCG32 sequence (state advanced
 * first, then the XSH-RR output of the new state), little-endian words */
static void seed_from_u64(uint64_t state, uint32_t key[8]) {
  const uint64_t INC = 11634580027462260723ull;
  for (int i = 0; i < 8; i++) {
    state = orc_pcg32_step(state, INC);
    key[i] = orc_pcg32_xsh_rr(state);
  }
}

/* the first n draws of StdRng::seed_from_u64(seed).gen::<f32>():
 * next_u32 walks the 64-word buffer of four consecutive ChaCha12 blocks
 * (counter from 0, stream 0), and each draw is (u32 >> 8) * 2^-24 */
void orc_stdrng_f32(uint64_t seed, size_t n, float *out) {
  uint32_t key[8], buf[64];
  seed_from_u64(seed, key);
  uint64_t ctr = 0;
  size_t idx = 64;
  for (size_t i = 0; i < n; i++) {
    if (idx >= 64) {
      for (int b = 0; b < 4; b++) orc_chacha_block(key, ctr + (uint64_t)b, 0, 12, buf + 16 * b);
      ctr += 4;
      idx = 0;
    }
    out[i] = (float)(buf[idx++] >> 8) * (1.0f / 16777216.0f);
  }
}

/* ======================================================================
 * Ternary linear (quantization/primitives/ternary_linear.rs)
 * ====================================================================== */

/* TernaryLinear::from_f32 (ternary_linear.rs:100-161): per row, threshold
 * 0.5 * mean|w| (sequential sum), codes +1 / -1 / 0, scale = mean |w| of
 * the non-zero codes (or mean|w| when there are none); blocks of 16 weights
 * = f32 scale + 4 code bytes (0b00 -1, 0b01 0, 0b10 +1; weight 4b+j at bits
 * 2j of byte b); K padded with zero codes to a multiple of 16. */
void orc_ternary_from_f32(const float *w, size_t n, size_t k, uint8_t *blocks) {
  const size_t bpr = (k + 15) / 16;
  for (size_t r = 0; r < n; r++) {
    const float *row = w + r * k;
    float s = 0.0f;
    for (size_t i = 0; i < k; i++) s += fabsf(row[i]);
    const float mean_abs = k ? s / (float)k : 0.0f;
    const float thr = 0.5f * mean_abs;
    float nz_sum = 0.0f;
    size_t nz = 0;
    for (size_t i = 0; i < k; i++) {
      if (row[i] > thr || row[i] < -thr) {
        nz_sum += fabsf(row[i]);
        nz++;
      }
    }
    const float scale = nz ? nz_sum / (float)nz : mean_abs;
    for (size_t b = 0; b < bpr; b++) {
      uint8_t *blk = blocks + (r * bpr + b) * 8;
      memcpy(blk, &scale, 4);
      for (int byte = 0; byte < 4; byte++) {
        uint8_t v = 0;
        for (int j = 0; j < 4; j++) {
          const size_t col = b * 16 + (size_t)byte * 4 + (size_t)j;
          uint8_t code = 1;  /* zero (and the padding) */
          if (col < k) {
            if (row[col] > thr) code = 2;
            else if (row[col] < -thr) code = 0;
          }
          v |= (uint8_t)(code << (2 * j));
        }
        blk[4 + byte] = v;
      }
    }
  }
}

/* TernaryLinear::forward (ternary_linear.rs:179-215): per block the codes add
 * or subtract x in column order (zero and reserved codes skip), then
 * acc += block_acc * scale, blocks in order; columns >= k are skipped. */
void orc_ternary_forward(const uint8_t *blocks, size_t n, size_t k, const float *x, size_t m,
                         float *y) {
  const size_t bpr = (k + 15) / 16;
  for (size_t i = 0; i < m; i++) {
    const float *xr = x + i * k;
    for (size_t j = 0; j < n; j++) {
      float acc = 0.0f;
      for (size_t b = 0; b < bpr; b++) {
        const uint8_t *blk = blocks + (j * bpr + b) * 8;
        float scale;
        memcpy(&scale, blk, 4);
        float bacc = 0.0f;
        for (int wi = 0; wi < 16; wi++) {
          const size_t col = b * 16 + (size_t)wi;
          if (col >= k) continue;
          const int code = (blk[4 + wi / 4] >> (2 * (wi % 4))) & 3;
          if (code == 2) bacc += xr[col];
          else if (code == 0) bacc -= xr[col];
        }
        acc += bacc * scale;
      }
      y[i * n + j] = acc;
    }
  }
}

/* ---- Hybrid LFM2.5 decoder, Q4 decode path (models/ssm/hybrid/{layer,model}.rs):
 * LIV conv and GQA layers with every projection a Q4Linear GEMV
 * (q4_0GemvRow after quantize_for_decode, layer.rs:570-581, 832-846), the
 * tied f32 lm_head as matmul_t (model.rs:240-290). ---- */
struct orc_hlm {
  orc_hlm_cfg c;
  size_t qd, kvd, nq4;
  float *embed, *final_nw, *rope_cos, *rope_sin;
  float **attn_nw, **ffn_nw, **conv_w, **conv_b, **q_nw, **k_nw;
  uint8_t **w_in, **w_out, **w_q, **w_k, **w_v, **w_o, **w_gate, **w_up, **w_down;
  float **conv_state, **kc, **vc;
  size_t pos;
};

orc_hlm *orc_hlm_create(const orc_hlm_cfg *cfg) {
  if (!cfg || cfg->n_layers == 0 || cfg->n_layers > 64 || cfg->hidden % 32 ||
      cfg->inner % 32 || cfg->inter % 32 || cfg->n_kv_heads == 0 ||
      cfg->n_heads % cfg->n_kv_heads || cfg->head_dim % 2 || cfg->conv_kernel == 0)
    return NULL;
  orc_hlm *m = (orc_hlm *)calloc(1, sizeof(orc_hlm));
  m->c = *cfg;
  m->qd = cfg->n_heads * cfg->head_dim;
  m->kvd = cfg->n_kv_heads * cfg->head_dim;
  size_t L = cfg->n_layers;
#define HLM_ARR(f, T) m->f = (T *)calloc(L, sizeof(T))
  HLM_ARR(attn_nw, float *); HLM_ARR(ffn_nw, float *); HLM_ARR(conv_w, float *);
  HLM_ARR(conv_b, float *); HLM_ARR(q_nw, float *); HLM_ARR(k_nw, float *);
  HLM_ARR(w_in, uint8_t *); HLM_ARR(w_out, uint8_t *); HLM_ARR(w_q, uint8_t *);
  HLM_ARR(w_k, uint8_t *); HLM_ARR(w_v, uint8_t *); HLM_ARR(w_o, uint8_t *);
  HLM_ARR(w_gate, uint8_t *); HLM_ARR(w_up, uint8_t *); HLM_ARR(w_down, uint8_t *);
  HLM_ARR(conv_state, float *); HLM_ARR(kc, float *); HLM_ARR(vc, float *);
#undef HLM_ARR
  size_t half = cfg->head_dim / 2;
  m->rope_cos = (float *)malloc(cfg->max_seq * half * 4);
  m->rope_sin = (float *)malloc(cfg->max_seq * half * 4);
  /* model.rs:708-720: freq = 1 / theta^(2i/hd), angle = pos * freq (f32) */
  orc_rope_tables(cfg->max_seq, cfg->head_dim, cfg->rope_theta, m->rope_cos, m->rope_sin);
  return m;
}

void orc_hlm_destroy(orc_hlm *m) {
  if (!m) return;
  for (size_t l = 0; l < m->c.n_layers; l++) {
    free(m->attn_nw[l]); free(m->ffn_nw[l]); free(m->conv_w[l]); free(m->conv_b[l]);
    free(m->q_nw[l]); free(m->k_nw[l]); free(m->w_in[l]); free(m->w_out[l]);
    free(m->w_q[l]); free(m->w_k[l]); free(m->w_v[l]); free(m->w_o[l]);
    free(m->w_gate[l]); free(m->w_up[l]); free(m->w_down[l]);
    free(m->conv_state[l]); free(m->kc[l]); free(m->vc[l]);
  }
  free(m->attn_nw); free(m->ffn_nw); free(m->conv_w); free(m->conv_b); free(m->q_nw);
  free(m->k_nw); free(m->w_in); free(m->w_out); free(m->w_q); free(m->w_k); free(m->w_v);
  free(m->w_o); free(m->w_gate); free(m->w_up); free(m->w_down); free(m->conv_state);
  free(m->kc); free(m->vc);
  free(m->embed); free(m->final_nw); free(m->rope_cos); free(m->rope_sin);
  free(m);
}

/* Q4Linear::from_f32 + pack_for_zig of an N(0, std) [n][k] tensor */
static uint8_t *hlm_q4(size_t n, size_t k, uint64_t seed, float std) {
  float *w = (float *)malloc(n * k * 4);
  orc_fill_normal(w, n * k, seed, std);
  uint8_t *p = (uint8_t *)malloc(orc_q4_packed_bytes(n, k));
  orc_q4_from_f32_packed(w, n, k, p);
  free(w);
  return p;
}

/* norm gains 1 + N(0, 0.1) */
static float *hlm_gain(size_t n, uint64_t seed) {
  float *g = (float *)malloc(n * 4);
  orc_fill_normal(g, n, seed, 0.1f);
  for (size_t i = 0; i < n; i++) g[i] = 1.0f + g[i];
  return g;
}

/* Synthetic weights (harness spec, shared with the device):
 * embed (= tied lm_head) tensor 0 ~ N(0, std); layer l, seeds s = seed_base
 * + 1 + 16 l: conv: in_proj s+0, conv taps s+1, out_proj s+2, conv bias
 * s+3 (if enabled); GQA: q s+0, k s+1, v s+2, o s+3, q/k norm gains s+6,
 * s+7; both: attn/ffn norm gains s+8, s+9, gate s+10, up s+11, down s+12
 * (projections ~ N(0, std), Q4-quantized; gains 1 + N(0, 0.1)); final norm
 * gain seed_base + 1 + 16 L. */
int orc_hlm_init_synthetic(orc_hlm *m, uint64_t seed_base, float std) {
  const orc_hlm_cfg *c = &m->c;
  size_t H = c->hidden, I = c->inner, ck = c->conv_kernel, F = c->inter;
  m->embed = (float *)malloc(c->vocab * H * 4);
  orc_fill_normal(m->embed, c->vocab * H, seed_base, std);
  for (size_t l = 0; l < c->n_layers; l++) {
    uint64_t s = seed_base + 1 + 16 * l;
    if (c->layer_kinds[l] == 0) {
      m->w_in[l] = hlm_q4(3 * I, H, s + 0, std);
      m->conv_w[l] = (float *)malloc(I * ck * 4);
      orc_fill_normal(m->conv_w[l], I * ck, s + 1, std);
      m->w_out[l] = hlm_q4(H, I, s + 2, std);
      if (c->conv_bias) {
        m->conv_b[l] = (float *)malloc(I * 4);
        orc_fill_normal(m->conv_b[l], I, s + 3, std);
      }
      m->conv_state[l] = (float *)calloc(I * ck, 4);
    } else {
      m->w_q[l] = hlm_q4(m->qd, H, s + 0, std);
      m->w_k[l] = hlm_q4(m->kvd, H, s + 1, std);
      m->w_v[l] = hlm_q4(m->kvd, H, s + 2, std);
      m->w_o[l] = hlm_q4(H, m->qd, s + 3, std);
      m->q_nw[l] = hlm_gain(c->head_dim, s + 6);
      m->k_nw[l] = hlm_gain(c->head_dim, s + 7);
      m->kc[l] = (float *)calloc(c->max_seq * m->kvd, 4);
      m->vc[l] = (float *)calloc(c->max_seq * m->kvd, 4);
    }
    m->attn_nw[l] = hlm_gain(H, s + 8);
    m->ffn_nw[l] = hlm_gain(H, s + 9);
    m->w_gate[l] = hlm_q4(F, H, s + 10, std);
    m->w_up[l] = hlm_q4(F, H, s + 11, std);
    m->w_down[l] = hlm_q4(H, F, s + 12, std);
  }
  m->final_nw = hlm_gain(H, seed_base + 1 + 16 * c->n_layers);
  m->pos = 0;
  return ORC_OK;
}

void orc_hlm_reset(orc_hlm *m) {
  for (size_t l = 0; l < m->c.n_layers; l++)
    if (m->conv_state[l]) memset(m->conv_state[l], 0, m->c.inner * m->c.conv_kernel * 4);
  m->pos = 0;
}
size_t orc_hlm_pos(const orc_hlm *m) { return m->pos; }

/* layer.rs:25-42 conv1d_step_single over every channel of the double-gated
 * LIV conv (layer.rs:609-627): proj = [B | C | x], conv input B*x, output
 * C * (sum_j buf[j] w[j] (+ bias)).  The state row of a channel holds its
 * last `ck` inputs, oldest first. */
void orc_hlm_conv_step(const float *proj, size_t inner, size_t ck, float *state,
                       const float *w, const float *bias, float *out) {
  for (size_t i = 0; i < inner; i++) {
    float b_gate = proj[i], c_gate = proj[inner + i], x_sig = proj[2 * inner + i];
    float bx = b_gate * x_sig;
    float *buf = state + i * ck;
    memmove(buf, buf + 1, (ck - 1) * 4);
    buf[ck - 1] = bx;
    /* Iterator::sum of f32 folds from -0.0 */
    float sum = -0.0f;
    for (size_t j = 0; j < ck; j++) {
      float t = buf[j] * w[i * ck + j];
      sum = sum + t;
    }
    float cv = bias ? sum + bias[i] : sum;
    out[i] = c_gate * cv;
  }
}

/* layer.rs:865-876: per head, scale = 1/sqrt(sum x^2 / hd + eps), x *= w * scale */
static void hlm_head_norm(float *data, const float *w, size_t heads, size_t hd, float eps) {
  for (size_t h = 0; h < heads; h++) {
    float *d = data + h * hd;
    float s = -0.0f;
    for (size_t j = 0; j < hd; j++) {
      float t = d[j] * d[j];
      s = s + t;
    }
    float scale = 1.0f / sqrtf(s / (float)hd + eps);
    for (size_t j = 0; j < hd; j++) d[j] = d[j] * (w[j] * scale);
  }
}

/* residual add (layer.rs:640-641, 1068-1069: h + a) */
static void hlm_add(float *x, const float *d, size_t n) {
  for (size_t i = 0; i < n; i++) x[i] = x[i] + d[i];
}

/* layer.rs:80-101 swiglu_ffn_forward_q4 with m = 1 */
static void hlm_ffn(orc_hlm *m, size_t l, const float *x, float *out) {
  size_t H = m->c.hidden, F = m->c.inter;
  float *normed = (float *)malloc(H * 4), *g = (float *)malloc(F * 4), *u = (float *)malloc(F * 4);
  orc_rmsnorm_seq(x, m->ffn_nw[l], m->c.eps, H, normed);
  orc_q4_0_gemv(F, H, normed, m->w_gate[l], g);
  orc_q4_0_gemv(F, H, normed, m->w_up[l], u);
  for (size_t i = 0; i < F; i++) g[i] = orc_silu(g[i]) * u[i];
  orc_q4_0_gemv(H, F, g, m->w_down[l], out);
  free(normed); free(g); free(u);
}

/* layer.rs:593-654 LivConvDecoderLayer::forward_one (double-gated) */
static void hlm_conv_layer(orc_hlm *m, size_t l, float *x) {
  size_t H = m->c.hidden, I = m->c.inner;
  float *normed = (float *)malloc(H * 4), *proj = (float *)malloc(3 * I * 4);
  float *co = (float *)malloc(I * 4), *o = (float *)malloc(H * 4);
  orc_rmsnorm_seq(x, m->attn_nw[l], m->c.eps, H, normed);
  orc_q4_0_gemv(3 * I, H, normed, m->w_in[l], proj);
  orc_hlm_conv_step(proj, I, m->c.conv_kernel, m->conv_state[l], m->conv_w[l], m->conv_b[l], co);
  orc_q4_0_gemv(H, I, co, m->w_out[l], o);
  hlm_add(x, o, H);
  hlm_ffn(m, l, x, o);
  hlm_add(x, o, H);
  free(normed); free(proj); free(co); free(o);
}

/* layer.rs:878-954 attn_forward_one + :1055-1078 forward_one */
static void hlm_gqa_layer(orc_hlm *m, size_t l, float *x) {
  const orc_hlm_cfg *c = &m->c;
  size_t H = c->hidden, hd = c->head_dim, nq = c->n_heads, nkv = c->n_kv_heads;
  size_t qd = m->qd, kvd = m->kvd, pos = m->pos, seq = pos + 1;
  float *normed = (float *)malloc(H * 4), *q = (float *)malloc(qd * 4);
  float *k = (float *)malloc(kvd * 4), *v = (float *)malloc(kvd * 4);
  float *att = (float *)malloc(qd * 4), *o = (float *)malloc(H * 4);
  float *scores = (float *)malloc(seq * 4);
  orc_rmsnorm_seq(x, m->attn_nw[l], c->eps, H, normed);
  orc_q4_0_gemv(qd, H, normed, m->w_q[l], q);
  orc_q4_0_gemv(kvd, H, normed, m->w_k[l], k);
  orc_q4_0_gemv(kvd, H, normed, m->w_v[l], v);
  hlm_head_norm(q, m->q_nw[l], nq, hd, c->eps);
  hlm_head_norm(k, m->k_nw[l], nkv, hd, c->eps);
  orc_rope_apply(q, m->rope_cos, m->rope_sin, 1, nq, hd, pos);
  orc_rope_apply(k, m->rope_cos, m->rope_sin, 1, nkv, hd, pos);
  memcpy(m->kc[l] + pos * kvd, k, kvd * 4);
  memcpy(m->vc[l] + pos * kvd, v, kvd * 4);
  size_t group = nq / nkv;
  float scale = 1.0f / sqrtf((float)hd);
  for (size_t qh = 0; qh < nq; qh++) {
    size_t kvh = qh / group;
    for (size_t p = 0; p < seq; p++) {
      const float *kp = m->kc[l] + p * kvd + kvh * hd;
      float dot = 0.0f;
      for (size_t d = 0; d < hd; d++) {
        float t = q[qh * hd + d] * kp[d];
        dot = dot + t;
      }
      scores[p] = dot * scale;
    }
    orc_softmax_slice(scores, seq);
    for (size_t d = 0; d < hd; d++) {
      float val = 0.0f;
      for (size_t p = 0; p < seq; p++) {
        float t = scores[p] * m->vc[l][p * kvd + kvh * hd + d];
        val = val + t;
      }
      att[qh * hd + d] = val;
    }
  }
  orc_q4_0_gemv(H, qd, att, m->w_o[l], o);
  hlm_add(x, o, H);
  hlm_ffn(m, l, x, o);
  hlm_add(x, o, H);
  free(normed); free(q); free(k); free(v); free(att); free(o); free(scores);
}

/* model.rs:240-290 decode_one (LFM2.5: no embedding norm) */
int orc_hlm_decode_one(orc_hlm *m, uint32_t token, float *logits) {
  const orc_hlm_cfg *c = &m->c;
  size_t H = c->hidden;
  if (m->pos >= c->max_seq) return ORC_ERR_INVALID_ARG;
  float *x = (float *)calloc(H, 4), *normed = (float *)malloc(H * 4);
  if (token < c->vocab) memcpy(x, m->embed + (size_t)token * H, H * 4);
  for (size_t l = 0; l < c->n_layers; l++) {
    if (c->layer_kinds[l] == 0) hlm_conv_layer(m, l, x);
    else hlm_gqa_layer(m, l, x);
  }
  m->pos++;
  orc_rmsnorm_seq(x, m->final_nw, c->eps, H, normed);
  memset(logits, 0, c->vocab * 4);
  orc_sgemm(1, c->vocab, H, normed, H, 0, m->embed, H, 1, logits, c->vocab);
  free(x); free(normed);
  return ORC_OK;
}

/* greedy generation: decode_one over the prompt, then argmax feedback */
int orc_hlm_generate(orc_hlm *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                     uint32_t *out_tokens, float *out_margins) {
  float *lg = (float *)malloc(m->c.vocab * 4);
  int rc = ORC_OK;
  for (size_t i = 0; i < n_prompt && rc == ORC_OK; i++) rc = orc_hlm_decode_one(m, prompt[i], lg);
  for (size_t t = 0; t < max_new && rc == ORC_OK; t++) {
    uint32_t tok = orc_argmax(lg, m->c.vocab);
    float second = -INFINITY;
    for (size_t i = 0; i < m->c.vocab; i++)
      if (i != tok && lg[i] > second) second = lg[i];
    out_tokens[t] = tok;
    if (out_margins) out_margins[t] = lg[tok] - second;
    if (t + 1 < max_new) rc = orc_hlm_decode_one(m, tok, lg);
  }
  free(lg);
  return rc;
}
