// Quantized linear layers resident in HBM (host-side classes behind the
// syn_hip_qlinear_* handles and the model drivers).
#pragma once

#include <vector>

#include "common.hpp"
#include "split_k.hpp"

namespace syn {

// Panel layout shared by the GEMV kernels: weights are cut into panels of 64
// output rows; inside a panel the K axis is cut into 16-byte chunks and the
// 64 rows' copies of chunk c are stored back to back:
//   byte (n, kbyte) -> ((n/64 * C + kbyte/16) * 64 + n%64) * 16 + kbyte%16
// so one wave64 load instruction (lane = row) reads 1 KiB contiguously and
// every lane owns one output row: no cross-lane reduction, and the
// activation chunk is wave-uniform.
constexpr int kPanelRows = 64;

struct GemvPlan {
  int panels = 0;   // ceil(N/64)
  int chunks = 0;   // 16-byte K chunks per row (C)
  int ksplit = 1;   // workgroups along K
  int cs = 0;       // chunks per K slice
  int waves = 1;    // waves per workgroup
};

GemvPlan make_gemv_plan(size_t n, size_t k_chunks, bool chunked_kc);

// INT8 W8A8 linear: QuantizedLinear (quantization/primitives/int8_linear.rs)
struct QLinearInt8 {
  size_t n = 0, k = 0;
  int chunks = 0;       // K16 / 16
  DevBuf w;             // panel layout, int8
  DevBuf scales;        // f32 [N64]
  DevBuf part;          // int32 split-K partials
  size_t part_elems = 0;
  DevBuf xq, sx;        // activation quantization scratch (forward())
  size_t xq_rows = 0;
  // gemv()'s one-launch K split: packed 64-bit row accumulators [16][N64]
  // (exact sum and arrivals), zero between calls (the slice that completes a
  // row reads and clears it)
  DevBuf sk_acc;
  int sk_panels = 0;
  syn_status_t ensure_sk();

  // host_nk: int8 [n,k] row per output; scales f32[n]
  syn_status_t upload_nk(const int8_t *host_nk, const float *host_scales, size_t n_, size_t k_);
  syn_status_t upload_kn(const int8_t *host_kn, size_t ldb, const float *host_scales, size_t n_,
                         size_t k_);
  // QuantizedLinear::from_f32 (int8_linear.rs:35-70) on host, then upload.
  syn_status_t from_f32(const float *w_nk, size_t n_, size_t k_);
  size_t weight_bytes() const { return n * k + n * 4; }
  // y[m, n] (row stride ldy) from pre-quantized rows xq (row stride ldx);
  // m <= 16 is one launch (a K split adds into sk_acc)
  syn_status_t gemv(size_t m, const int8_t *d_xq, size_t ldx, const float *d_sx, float *d_y,
                    size_t ldy, hipStream_t s);
  // the same with the split-K partials in d_part (part_elems_for(min(m, 16))
  // int32; unused when that is 0) and a second reduce launch
  syn_status_t gemv_part(size_t m, const int8_t *d_xq, size_t ldx, const float *d_sx,
                         float *d_y, size_t ldy, int *d_part, hipStream_t s);
  size_t part_elems_for(size_t m) const;
  syn_status_t ensure_part(size_t elems);
  // allocate split-K scratch for up to max_m activation rows (needed before
  // a graph capture: nothing may allocate while a step is being recorded)
  syn_status_t prepare(size_t max_m);
};

// launch the device quantizer (quantize.zig:12-47) on rows of x
syn_status_t launch_quantize_rows(const float *d_x, size_t m, size_t k, size_t ldx, int8_t *d_q,
                                  size_t ldq, float *d_s, hipStream_t s);

// INT8 MFMA GEMM for M > 16 (int8_gemm.hip); W in the panel layout
syn_status_t launch_gemm_w8a8(const int8_t *xq, size_t ldx, const float *sx, size_t M,
                              const void *W, const float *ws, size_t N, int C, float *y,
                              size_t ldy, hipStream_t s);

// host-side reference quantizers (used at load time)
void host_minmax_scales(const float *w, size_t ch, size_t chsz, float *scales);
void host_quantize_weights_nk(const float *w, const float *scales, size_t n, size_t k,
                              int8_t *out_nk);

// The split-K partials of one GEMV output row set, left for the kernel that
// consumes the output: row r = sum over k < ks of p[k * stride + r], summed
// from 0.0f in k order; ks = 1 is the output
// itself (stride unused).
struct PartRows {
  const float *p = nullptr;
  int ks = 1;
  int stride = 0;
};

// Q4_0 linear: Q4Linear (q4_linear.rs); f32 activations.
struct QLinearQ4_0 {
  size_t n = 0, k = 0;
  int blocks = 0;      // K/32
  DevBuf nib;          // [P][blocks][64][16] nibble bytes
  DevBuf sc;           // [P][blocks][64] f16 bits
  DevBuf part;         // f32 split-K partials
  size_t part_elems = 0;
  DevBuf asum;         // per-call block sums of the activation rows
  size_t asum_rows = 0;
  // block scales read with the Rust f16 converter (subnormals halved): the
  // reference's GGUF Q4_0 path; false = the Zig GEMV's IEEE conversion
  bool rs_f16_scales = false;
  bool has_subnormal_scale = false;  // some block scale is an f16 subnormal (set at upload)
  DevBuf xh;                         // f16 activations for the MFMA GEMM
  size_t xh_bytes = 0;  // its size (f16_rows_bytes)
  SplitKSlots sk;  // gemv()'s one-launch K split at one row (split_k.hpp)
  syn_status_t upload_packed(const uint8_t *packed, size_t n_, size_t k_);
  syn_status_t from_f32(const float *w_nk, size_t n_, size_t k_);
  // allocate the split-K partials of GEMV batches up to max_m rows (so that
  // gemv() allocates nothing, e.g. under HIP graph capture)
  syn_status_t prepare(size_t max_m);
  size_t weight_bytes() const { return n * (k / 32) * 18; }
  // y[m,n] = x[m,k] W^T, f32 activations; m > 16 runs gemm() when gemm_ok()
  syn_status_t gemv(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                    hipStream_t s);
  // one activation row, its K split left to the consumer: the GEMV kernel
  // writes its split-K partials (prepare(1) must have run) and *out names
  // them; with a single K slice it writes y[n] and *out names y
  syn_status_t gemv_parts(const float *d_x, float *d_y, PartRows *out, hipStream_t s);
  // f16 MFMA prefill GEMM (kquant_gemm.hip): weights (nibble - 8) * d and
  // activations rounded once to f16, f32 accumulation
  syn_status_t gemm(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                    hipStream_t s);
  // the GEMM decodes the scales as IEEE f16 values: not for halved subnormals
  bool gemm_ok() const { return !(rs_f16_scales && has_subnormal_scale); }
};

// Ternary linear: TernaryLinear (ternary_linear.rs); f32 activations.
struct QLinearTernary {
  size_t n = 0, k = 0;
  int bpr = 0;         // blocks of 16 weights per row
  DevBuf codes;        // u32 [P][bpr][64]
  DevBuf scales;       // f32 [P][bpr][64]
  // the reference's blocks: per block an f32 scale and four code bytes
  syn_status_t upload_blocks(const uint8_t *blocks, size_t n_, size_t k_);
  syn_status_t from_f32(const float *w_nk, size_t n_, size_t k_);
  size_t weight_bytes() const { return n * (size_t)bpr * 8; }
  syn_status_t gemv(size_t m, const float *d_x, size_t ldx, float *d_y, size_t ldy,
                    hipStream_t s);
};

// Q4Linear::from_f32 + pack_for_zig (q4_linear.rs:64-121), host side.
void host_q4_pack(const float *w, size_t n, size_t k, uint8_t *packed);

void fill_normal(float *dst, size_t n, uint64_t seed, float stddev);
void fill_normal_parallel(float *dst, size_t n, uint64_t seed, float stddev);

}  // namespace syn
