// syn_sgemm compatibility export (synapse.h:181-184, exports.zig:725-761) and
// the syn_hip_-prefixed aliases of the four reference-signature entry points.
//
// syn_sgemm is the reference's f32 GEMM, C = op(A) op(B) row-major, with host
// pointers.  Its values are fixed by sgemmTiled (matmul.zig:125-184): for
// M <= 16 and A untransposed, one f32GemvRow per row (:142-155, :223-305)
// overwrites C: with B transposed every column in the 32- and 8-wide column
// blocks is a fused multiply-add chain over p and the tail columns are plain
// multiply-then-add chains; with B as is, the 32-wide blocks are fused and
// the rest plain.  Otherwise the GOTO path (:157-183) accumulates into C:
// each element is one chain over p starting from C's value, fused inside
// full 8x8 micro-tiles (:454-496) and plain in the edge tiles (rows of a
// partial 8-row panel of a 256-row block, columns of a partial 8-column
// panel of a 4096-column block).  One device thread per output element runs
// exactly that chain, so the shim is bit-identical to the reference's order;
// it exists for the parity contract of the exported name, not for speed
// (the device decoders run their own f32 GEMV/GEMM kernels).
#include <vector>

#include "common.hpp"

namespace syn {

__global__ void __launch_bounds__(256)
    k_sgemm_ref(size_t m, size_t n, size_t k, const float *__restrict__ a, size_t lda, int ta,
                const float *__restrict__ b, size_t ldb, int tb, float *__restrict__ c,
                size_t ldc) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= m * n) return;
  const size_t i = e / n, j = e % n;
  bool fused;
  float acc;
  if (m <= 16 && !ta) {
    const size_t n32 = n - n % 32;
    const size_t n8 = n32 + (n - n32) / 8 * 8;
    fused = tb ? j < n8 : j < n32;
    acc = 0.0f;
  } else {
    const size_t ic = i / 256 * 256, mc = (m - ic < 256) ? m - ic : 256;
    const size_t ir = (i - ic) / 8 * 8;
    const size_t jc = j / 4096 * 4096, nc = (n - jc < 4096) ? n - jc : 4096;
    const size_t jr = (j - jc) / 8 * 8;
    fused = (mc - ir) >= 8 && (nc - jr) >= 8;
    acc = c[i * ldc + j];
  }
  for (size_t p = 0; p < k; p++) {
    const float av = ta ? a[p * lda + i] : a[i * lda + p];
    const float bv = tb ? b[j * ldb + p] : b[p * ldb + j];
    if (fused) {
      acc = __builtin_fmaf(av, bv, acc);
    } else {
      const float t = av * bv;
      acc = acc + t;
    }
  }
  c[i * ldc + j] = acc;
}

}  // namespace syn

using namespace syn;

extern "C" {

syn_status_t syn_sgemm(size_t m, size_t n, size_t k, const float *a, size_t lda, int trans_a,
                       const float *b, size_t ldb, int trans_b, float *c, size_t ldc) {
  if (!a || !b || !c) return SYN_ERR_NULL_PTR;
  if (m == 0 || n == 0 || k == 0) return SYN_OK;  // exports.zig:741
  SYN_TRY(ensure_init());
  // elements each host matrix spans with its leading dimension
  const size_t na = trans_a ? (k - 1) * lda + m : (m - 1) * lda + k;
  const size_t nb = trans_b ? (n - 1) * ldb + k : (k - 1) * ldb + n;
  const size_t nc = (m - 1) * ldc + n;
  DevBuf da, db, dc;
  SYN_TRY(da.alloc(na * 4));
  SYN_TRY(db.alloc(nb * 4));
  SYN_TRY(dc.alloc(nc * 4));
  hipStream_t s = default_stream();
  SYN_HIP(hipMemcpyAsync(da.p, a, na * 4, hipMemcpyHostToDevice, s));
  SYN_HIP(hipMemcpyAsync(db.p, b, nb * 4, hipMemcpyHostToDevice, s));
  SYN_HIP(hipMemcpyAsync(dc.p, c, nc * 4, hipMemcpyHostToDevice, s));  // the GOTO path accumulates
  const size_t total = m * n;
  hipLaunchKernelGGL(k_sgemm_ref, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, m, n, k,
                     da.as<float>(), lda, trans_a, db.as<float>(), ldb, trans_b, dc.as<float>(),
                     ldc);
  SYN_LAUNCH_CHECK();
  SYN_HIP(hipMemcpyAsync(c, dc.p, nc * 4, hipMemcpyDeviceToHost, s));
  SYN_HIP(hipStreamSynchronize(s));
  return SYN_OK;
}

// the same entry points under names a static reference archive does not
// define, so a binary that links that archive can still reach these
syn_status_t syn_hip_sgemm(size_t m, size_t n, size_t k, const float *a, size_t lda, int trans_a,
                           const float *b, size_t ldb, int trans_b, float *c, size_t ldc) {
  return syn_sgemm(m, n, k, a, lda, trans_a, b, ldb, trans_b, c, ldc);
}
syn_status_t syn_hip_quantize_per_channel_int8(const float *data, size_t channels,
                                               size_t channel_size, int8_t *out, float *scales) {
  return syn_quantize_per_channel_int8(data, channels, channel_size, out, scales);
}
syn_status_t syn_hip_qgemm_int8(size_t m, size_t n, size_t k, const int8_t *a, size_t lda,
                                const int8_t *b, size_t ldb, float *c, size_t ldc,
                                const float *scales_a, const float *scales_b) {
  return syn_qgemm_int8(m, n, k, a, lda, b, ldb, c, ldc, scales_a, scales_b);
}
syn_status_t syn_hip_q4_0_gemv(size_t n, size_t k, const float *a, const uint8_t *b_q4,
                               float *c) {
  return syn_q4_0_gemv(n, k, a, b_q4, c);
}

}  // extern "C"
