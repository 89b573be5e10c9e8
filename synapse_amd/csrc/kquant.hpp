// GGUF-block formats Q8_0 / Q4_K / Q6_K resident in HBM (kquant.hip).
#pragma once

#include "linear.hpp"

namespace syn {

size_t kq_block_bytes(int fmt);
size_t kq_block_elems(int fmt);
// encode f32 [n,k] rows into the reference's block byte format
void kq_encode(int fmt, const float *w, size_t n, size_t k, uint8_t *out);
// host dequantizers of the reference (gguf.rs:255-288, 375-487): `nblocks`
// blocks of `fmt` bytes -> f32 values
void kq_dequant(int fmt, const uint8_t *bytes, size_t nblocks, float *out);
// the reference's f16 -> f32 converter (converter.rs:12-40, subnormals halve)
float f16_to_f32_reference(uint16_t h);

// bytes of a GEMM's f16 activation rows plus their per-row scales
// (kquant_gemm.hip), m rows of k elements
size_t f16_rows_bytes(size_t m, size_t k);

struct QLinearKQ {
  int fmt = 0;
  size_t n = 0, k = 0;
  int blocks = 0;  // blocks per row
  int planes = 0;  // 16-byte planes per block
  DevBuf wq;       // [P][blocks][planes][64][16]
  DevBuf wd;       // [P][blocks][64] f16 d (Q8_0, Q6_K)
  DevBuf xh;  // f16 activations for the MFMA GEMM
  size_t xh_bytes = 0;  // its size (f16_rows_bytes)
  SplitKSlots sk;  // gemv()'s one-launch K split at one row (split_k.hpp)
  // Q8_0: every block scale (as the reference converts it) is an f16 value,
  // so the GEMM may multiply in f16 (set at upload)
  bool q8_scales_f16_exact = true;
  syn_status_t upload(int fmt, const uint8_t *gguf, size_t n, size_t k);
  syn_status_t from_f32(int fmt, const float *w, size_t n, size_t k);
  size_t weight_bytes() const;
  // y[m,n] = x[m,k] W^T, f32 activations (M rows, any M; M > 8 runs gemm())
  syn_status_t gemv(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                    hipStream_t s);
  // f16 MFMA prefill GEMM (kquant_gemm.hip)
  syn_status_t gemm(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                    hipStream_t s);
  syn_status_t prepare(size_t max_m);
};

}  // namespace syn
