// Ternary (2-bit) linear layer: TernaryLinear
// (quantization/primitives/ternary_linear.rs).
//
// A block is 16 weights: an f32 scale and four code bytes (0b00 -1, 0b01 0,
// 0b10 +1, 0b11 0; weight 4b+j at bits 2j of byte b).  forward() adds or
// subtracts x per code in column order inside a block, then accumulates
// block_acc * scale over the blocks in order.  The block sums are independent
// of each other, so the device computes them in parallel (16 rows per
// workgroup, 16 threads per row on different blocks) and keeps only the
// chain over the blocks sequential: one thread per row adds the products in
// block order.
//
// HBM layout (repacked once): codes u32 and scales f32 in 64-row panels,
// [panel][block][64], so a wave's load of one block (lane = row) reads 256
// contiguous bytes of each plane.
#include <cstring>
#include <vector>

#include "linear.hpp"

namespace syn {

constexpr int kTerNT = 256;
constexpr int kTerRows = 16;                  // output rows per workgroup
constexpr int kTerGroups = kTerNT / kTerRows;  // block groups (threads per row)
constexpr int kTerChunk = 256;                 // blocks per LDS chunk (4096 columns)
constexpr int kTerPer = kTerChunk / kTerGroups;

// Thread t owns row t % 16 of the workgroup's 16 and, in every chunk of 256
// blocks, the 16 blocks g*16 .. g*16+15 of block group g = t / 16.  A block's
// sum adds v = +x, -x or 0 per code: the reference skips the zero codes, and
// adding +0.0 leaves the sum unchanged because a sum that starts at +0.0 and
// only adds or subtracts finite values is never -0.0 (and v is 0.0, not x,
// for a skipped non-finite x); so the add is the only operation on the
// dependency chain.
__global__ void __launch_bounds__(kTerNT)
    k_gemv_ternary(const uint32_t *__restrict__ codes, const float *__restrict__ scales, int bpr,
                   int k, const float *__restrict__ x, int ldx, float *__restrict__ y, int ldy,
                   int n) {
  __shared__ float xs[kTerChunk * 16];
  __shared__ float pb[kTerChunk][kTerRows];
  const int tid = threadIdx.x;
  const int r = tid % kTerRows, g = tid / kTerRows;
  const int row0 = blockIdx.x * kTerRows, m = blockIdx.y;
  const int nrow = min(row0 + r, n - 1);
  const float *xr = x + (size_t)m * ldx;
  // panel layout: element (row, block) at ((row/64)*bpr + block)*64 + row%64
  const size_t base = (size_t)(nrow / 64) * bpr * 64 + nrow % 64;
  float acc = 0.0f;
  for (int b0 = 0; b0 < bpr; b0 += kTerChunk) {
    const int nb = min(kTerChunk, bpr - b0);
    uint32_t cw[kTerPer];
    float sc[kTerPer];
#pragma unroll
    for (int j = 0; j < kTerPer; j++) {
      const size_t b = (size_t)(b0 + min(g * kTerPer + j, nb - 1));
      cw[j] = codes[base + b * 64];
      sc[j] = scales[base + b * 64];
    }
    for (int i = tid; i < nb * 16; i += kTerNT) {
      const int col = b0 * 16 + i;
      xs[i] = col < k ? xr[col] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTerPer; j++) {
      const int bl = g * kTerPer + j;  // block within the chunk
      if (bl < nb) {
        const int colb = (b0 + bl) * 16;
        const float4 *x4 = reinterpret_cast<const float4 *>(xs + bl * 16);
        float xv[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float4 t = x4[q];
          xv[4 * q] = t.x;
          xv[4 * q + 1] = t.y;
          xv[4 * q + 2] = t.z;
          xv[4 * q + 3] = t.w;
        }
        // columns past k count as zero codes (the reference skips them)
        const int valid = k - colb;
        const uint32_t keep =
            valid >= 16 ? 0xffffffffu : valid <= 0 ? 0u : 0xffffffffu >> (32 - 2 * valid);
        const uint32_t cwv = (cw[j] & keep) | (0x55555555u & ~keep);
        float bacc = 0.0f;
#pragma unroll
        for (int wi = 0; wi < 16; wi++) {
          // v = +x (code 2), -x (code 0) or 0 (codes 1, 3), without branches:
          // the sign flips when bit 1 is clear, odd codes mask to zero
          const uint32_t c = (cwv >> (2 * wi)) & 3u;
          const uint32_t vb =
              (__float_as_uint(xv[wi]) ^ ((~c & 2u) << 30)) & ((c & 1u) - 1u);
          bacc = bacc + __uint_as_float(vb);  // block_acc += x / -= x (ternary_linear.rs:200-206)
        }
        pb[bl][r] = bacc * sc[j];
      }
    }
    __syncthreads();
    if (g == 0) {
      // acc += block_acc * scale, blocks in order (ternary_linear.rs:209)
      int b = 0;
      for (; b + 8 <= nb; b += 8) {
        float p[8];
#pragma unroll
        for (int t = 0; t < 8; t++) p[t] = pb[b + t][r];
#pragma unroll
        for (int t = 0; t < 8; t++) acc = acc + p[t];
      }
      for (; b < nb; b++) acc = acc + pb[b][r];
    }
    __syncthreads();
  }
  if (g == 0 && row0 + r < n) y[(size_t)m * ldy + row0 + r] = acc;
}

// TernaryLinear::from_f32 (ternary_linear.rs:100-161) on the host: the block
// bytes of the reference's format
static void host_ternary_from_f32(const float *w, size_t n, size_t k, uint8_t *blocks) {
  const size_t bpr = (k + 15) / 16;
  for (size_t r = 0; r < n; r++) {
    const float *row = w + r * k;
    float s = 0.0f;
    for (size_t i = 0; i < k; i++) s += std::fabs(row[i]);
    const float mean_abs = k ? s / (float)k : 0.0f;
    const float thr = 0.5f * mean_abs;
    float nz_sum = 0.0f;
    size_t nz = 0;
    std::vector<uint8_t> code(bpr * 16, 1);
    for (size_t i = 0; i < k; i++) {
      if (row[i] > thr) code[i] = 2;
      else if (row[i] < -thr) code[i] = 0;
      if (code[i] != 1) {
        nz_sum += std::fabs(row[i]);
        nz++;
      }
    }
    const float scale = nz ? nz_sum / (float)nz : mean_abs;
    for (size_t b = 0; b < bpr; b++) {
      uint8_t *blk = blocks + (r * bpr + b) * 8;
      std::memcpy(blk, &scale, 4);
      for (int byte = 0; byte < 4; byte++) {
        uint8_t v = 0;
        for (int j = 0; j < 4; j++) v |= (uint8_t)(code[b * 16 + byte * 4 + j] << (2 * j));
        blk[4 + byte] = v;
      }
    }
  }
}

syn_status_t QLinearTernary::upload_blocks(const uint8_t *blocks, size_t n_, size_t k_) {
  n = n_;
  k = k_;
  bpr = (int)((k + 15) / 16);
  const size_t panels = (n + 63) / 64;
  std::vector<uint32_t> c(panels * bpr * 64, 0x55555555u);  // padding rows: zero codes
  std::vector<float> sc(panels * bpr * 64, 0.0f);
  for (size_t r = 0; r < n; r++)
    for (int b = 0; b < bpr; b++) {
      const uint8_t *blk = blocks + (r * bpr + b) * 8;
      const size_t dst = ((r / 64) * bpr + b) * 64 + r % 64;
      std::memcpy(&sc[dst], blk, 4);
      std::memcpy(&c[dst], blk + 4, 4);
    }
  SYN_TRY(codes.alloc(c.size() * 4));
  SYN_TRY(scales.alloc(sc.size() * 4));
  SYN_HIP(hipMemcpy(codes.p, c.data(), c.size() * 4, hipMemcpyHostToDevice));
  SYN_HIP(hipMemcpy(scales.p, sc.data(), sc.size() * 4, hipMemcpyHostToDevice));
  return SYN_OK;
}

syn_status_t QLinearTernary::from_f32(const float *w_nk, size_t n_, size_t k_) {
  std::vector<uint8_t> blocks(n_ * ((k_ + 15) / 16) * 8);
  host_ternary_from_f32(w_nk, n_, k_, blocks.data());
  return upload_blocks(blocks.data(), n_, k_);
}

syn_status_t QLinearTernary::gemv(size_t m, const float *d_x, size_t ldx, float *d_y,
                                  size_t ldy, hipStream_t s) {
  if (m == 0) return SYN_OK;
  if (m > 65535) return SYN_ERR_INVALID_ARG;
  hipLaunchKernelGGL(k_gemv_ternary, dim3((unsigned)((n + kTerRows - 1) / kTerRows), (unsigned)m),
                     dim3(kTerNT), 0, s, codes.as<uint32_t>(), scales.as<float>(), bpr, (int)k,
                     d_x, (int)ldx, d_y, (int)ldy, (int)n);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn
