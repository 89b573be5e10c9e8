// INT8 W8A8 path: activation quantizer (A1), weight quantizer at load (A2),
// decode GEMV (A3) and the KC-chunked prefill form (A4).
//
// Reference semantics (zig/src/ops/qmatmul.zig):
//   M <= 16 : C[i,j] = (f32(sum_k a[i,k] b[k,j]) * sa[i]) * sb[j]   (:54-66, :171-256)
//   M  > 16 : C[i,j] = sum over KC=512 chunks, in order, of
//             (f32(chunk i32 sum) * sa[i]) * sb[j]                   (:68-99, :515-525)
// Integer sums are exact in any order, so the GPU splits K freely inside a
// chunk; only the f32 epilogue order is fixed.
#include <algorithm>
#include <cmath>
#include <vector>

#include <mutex>
#include <string>
#include "kquant.hpp"
#include "linear.hpp"

namespace syn {

// --------------------------------------------------------------- quantizer
// one workgroup per row; max|x| is order-free, the rest is elementwise
__global__ void __launch_bounds__(256) k_quantize_rows(const float *__restrict__ x, int K,
                                                       int ldx, int8_t *__restrict__ q, int ldq,
                                                       float *__restrict__ scales) {
  __shared__ float red[256];
  const int row = blockIdx.x;
  const float *xr = x + (size_t)row * ldx;
  int8_t *qr = q + (size_t)row * ldq;
  float mx = 0.0f;
  for (int j = threadIdx.x; j < K; j += 256) {
    const float a = fabsf(xr[j]);
    if (a > mx) mx = a;
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  const float max_abs = red[0];
  if (max_abs == 0.0f) {
    for (int j = threadIdx.x; j < K; j += 256) qr[j] = 0;
    if (threadIdx.x == 0) scales[row] = 1.0f;
    return;
  }
  const float inv = 127.0f / max_abs;
  for (int j = threadIdx.x; j < K; j += 256) {
    float r = roundf(xr[j] * inv);
    r = fminf(127.0f, fmaxf(-127.0f, r));
    qr[j] = (int8_t)(int)r;
  }
  if (threadIdx.x == 0) scales[row] = max_abs / 127.0f;
}

syn_status_t launch_quantize_rows(const float *d_x, size_t m, size_t k, size_t ldx, int8_t *d_q,
                                  size_t ldq, float *d_s, hipStream_t s) {
  if (m == 0 || k == 0) return SYN_OK;
  hipLaunchKernelGGL(k_quantize_rows, dim3((unsigned)m), dim3(256), 0, s, d_x, (int)k, (int)ldx,
                     d_q, (int)ldq, d_s);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// --------------------------------------------------------------- GEMV
// grid (panels, ksplit); blockDim = 64 * waves.  Lane = output row of the
// panel; each wave walks 16-byte K chunks (one 1 KiB load per chunk) and does
// 4 v_dot4_i32_i8 per activation row.  Waves reduce in LDS (i32, exact).
// A K split either writes per-slice partials for k_gemv_reduce (SK false), or
// (SK true, one launch) adds them into 64-bit accumulators acc64[M][N64]
// with device-scope atomics: one add carries a row's exact partial sum (bits
// 0-39, two's complement: |sum| < 2^39) and one arrival (bits 40-63), so the
// returned old value plus the add is the row's running total and arrival
// count.  The slice whose add completes the count (the row's last, which
// need not be the same workgroup for every row) applies the epilogue and
// clears the accumulator for the next call with a device-scope atomic
// store.  Integer sums are exact in any order.
template <int M, bool SK>
__global__ void __launch_bounds__(1024)
    k_gemv_w8a8(const i32x4 *__restrict__ W, const float *__restrict__ ws,
                const int8_t *__restrict__ xq, int ldx, const float *__restrict__ sx,
                float *__restrict__ y, int ldy, int *__restrict__ part,
                unsigned long long *__restrict__ acc64, int N, int C, int cs) {
  extern __shared__ int red[];  // [waves][M][64]
  const int panel = blockIdx.x, ks = blockIdx.y;
  const int nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c0 = ks * cs;
  const int c1 = min(C, c0 + cs);
  const i32x4 *Wp = W + (size_t)panel * C * 64 + lane;
  int acc[M];
#pragma unroll
  for (int m = 0; m < M; m++) acc[m] = 0;

  int c = c0 + wave;
  for (; c + 3 * nw < c1; c += 4 * nw) {
    i32x4 w[4];
#pragma unroll
    for (int u = 0; u < 4; u++) w[u] = __builtin_nontemporal_load(Wp + (size_t)(c + u * nw) * 64);
#pragma unroll
    for (int u = 0; u < 4; u++) {
#pragma unroll
      for (int m = 0; m < M; m++) {
        const i32x4 xv =
            *reinterpret_cast<const i32x4 *>(xq + (size_t)m * ldx + (size_t)(c + u * nw) * 16);
        acc[m] = __builtin_amdgcn_sdot4(w[u].x, xv.x, acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(w[u].y, xv.y, acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(w[u].z, xv.z, acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(w[u].w, xv.w, acc[m], false);
      }
    }
  }
  for (; c < c1; c += nw) {
    const i32x4 w = __builtin_nontemporal_load(Wp + (size_t)c * 64);
#pragma unroll
    for (int m = 0; m < M; m++) {
      const i32x4 xv = *reinterpret_cast<const i32x4 *>(xq + (size_t)m * ldx + (size_t)c * 16);
      acc[m] = __builtin_amdgcn_sdot4(w.x, xv.x, acc[m], false);
      acc[m] = __builtin_amdgcn_sdot4(w.y, xv.y, acc[m], false);
      acc[m] = __builtin_amdgcn_sdot4(w.z, xv.z, acc[m], false);
      acc[m] = __builtin_amdgcn_sdot4(w.w, xv.w, acc[m], false);
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++) red[(wave * M + m) * 64 + lane] = acc[m];
  __syncthreads();
  const int N64 = gridDim.x * 64;
  if constexpr (SK) {
    for (int t = threadIdx.x; t < M * 64; t += blockDim.x) {
      const int m = t >> 6, r = t & 63, row = panel * 64 + r;
      int s = 0;
      for (int w = 0; w < nw; w++) s += red[(w * M + m) * 64 + r];
      unsigned long long *a = acc64 + (size_t)m * N64 + row;
      const unsigned long long add = (1ull << 40) + (unsigned long long)(long long)s;
      const unsigned long long tot =
          __hip_atomic_fetch_add(a, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
      const long long sum = (long long)(tot << 24) >> 24;
      if ((int)((tot - (unsigned long long)sum) >> 40) == (int)gridDim.y) {  // the row is complete
        __hip_atomic_store(a, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (row < N) {
          const float f = (float)(int)sum * sx[m];
          y[(size_t)m * ldy + row] = f * ws[row];
        }
      }
    }
    return;
  }
  for (int t = threadIdx.x; t < M * 64; t += blockDim.x) {
    const int m = t >> 6, r = t & 63;
    int s = 0;
    for (int w = 0; w < nw; w++) s += red[(w * M + m) * 64 + r];
    const int row = panel * 64 + r;
    if (gridDim.y == 1) {
      if (row < N) {
        const float f = (float)s * sx[m];
        y[(size_t)m * ldy + row] = f * ws[row];
      }
    } else {
      part[((size_t)ks * M + m) * N64 + row] = s;
    }
  }
}

// Second stage of a K split.  chunked==0: exact i32 total, then the GEMV
// epilogue.  chunked==1: slices are the reference's KC=512 chunks and the
// f32 epilogue is accumulated slice by slice in order (qmatmul.zig:515-525).
__global__ void __launch_bounds__(256)
    k_gemv_reduce(const int *__restrict__ part, int ksplit, int M, int N, int N64,
                  const float *__restrict__ sx, const float *__restrict__ ws,
                  float *__restrict__ y, int ldy, int chunked) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * N) return;
  const int m = idx / N, row = idx - m * N;
  if (!chunked) {
    int s = 0;
    for (int k = 0; k < ksplit; k++) s += part[((size_t)k * M + m) * N64 + row];
    const float f = (float)s * sx[m];
    y[(size_t)m * ldy + row] = f * ws[row];
  } else {
    float c = 0.0f;
    for (int k = 0; k < ksplit; k++) {
      const float f = (float)part[((size_t)k * M + m) * N64 + row] * sx[m];
      const float t = f * ws[row];
      c = c + t;
    }
    y[(size_t)m * ldy + row] = c;
  }
}

GemvPlan make_gemv_plan(size_t n, size_t k_chunks, bool chunked_kc) {
  GemvPlan p;
  p.panels = (int)cdiv(n, kPanelRows);
  p.chunks = (int)k_chunks;
  if (chunked_kc) {
    p.cs = 32;  // KC = 512 bytes = 32 chunks
    p.ksplit = (int)cdiv(k_chunks, 32);
  } else {
    int ks = 1;
    if (p.panels < 240) {
      ks = (int)cdiv(256, p.panels);
      ks = std::min<int>(ks, (int)std::max<size_t>(1, k_chunks / 4));
    }
    p.cs = (int)cdiv(k_chunks, ks);
    p.ksplit = (int)cdiv(k_chunks, p.cs);
  }
  p.waves = std::min(16, std::max(1, p.cs));
  return p;
}

// acc64 != nullptr: the single-launch split-K form (the packed accumulators);
// otherwise per-slice partials in part (or none without a split)
template <int M>
static void launch_gemv_m(const GemvPlan &p, const i32x4 *W, const float *ws, const int8_t *xq,
                          int ldx, const float *sx, float *y, int ldy, int *part,
                          unsigned long long *acc64, int N, hipStream_t s) {
  const int waves = std::min(p.waves, M >= 8 ? 8 : 16);
  const size_t shm = (size_t)waves * M * 64 * sizeof(int);
  if (acc64 && p.ksplit > 1)
    hipLaunchKernelGGL((k_gemv_w8a8<M, true>), dim3(p.panels, p.ksplit), dim3(64 * waves), shm, s,
                       W, ws, xq, ldx, sx, y, ldy, nullptr, acc64, N, p.chunks, p.cs);
  else
    hipLaunchKernelGGL((k_gemv_w8a8<M, false>), dim3(p.panels, p.ksplit), dim3(64 * waves), shm,
                       s, W, ws, xq, ldx, sx, y, ldy, part, nullptr, N, p.chunks, p.cs);
}

typedef void (*gemv_launcher)(const GemvPlan &, const i32x4 *, const float *, const int8_t *, int,
                              const float *, float *, int, int *, unsigned long long *, int,
                              hipStream_t);
static const gemv_launcher kGemvLaunch[17] = {
    nullptr,          launch_gemv_m<1>,  launch_gemv_m<2>,  launch_gemv_m<3>,
    launch_gemv_m<4>, launch_gemv_m<5>,  launch_gemv_m<6>,  launch_gemv_m<7>,
    launch_gemv_m<8>, launch_gemv_m<9>,  launch_gemv_m<10>, launch_gemv_m<11>,
    launch_gemv_m<12>, launch_gemv_m<13>, launch_gemv_m<14>, launch_gemv_m<15>,
    launch_gemv_m<16>};

syn_status_t QLinearInt8::ensure_part(size_t elems) {
  if (part_elems >= elems) return SYN_OK;
  SYN_HIP(hipDeviceSynchronize());  // the old buffer may still be read by queued work
  SYN_TRY(part.alloc(elems * sizeof(int)));
  part_elems = elems;
  return SYN_OK;
}

syn_status_t QLinearInt8::prepare(size_t max_m) {
  const size_t mb = std::min<size_t>(16, std::max<size_t>(1, max_m));
  const GemvPlan p = make_gemv_plan(n, (size_t)chunks, false);
  const size_t need = p.ksplit > 1 ? (size_t)p.ksplit * mb * p.panels * 64 : 0;
  if (need) SYN_TRY(ensure_part(need));
  return ensure_sk();
}

syn_status_t QLinearInt8::ensure_sk() {
  const GemvPlan p = make_gemv_plan(n, (size_t)chunks, false);
  if (p.ksplit <= 1 || sk_panels >= p.panels) return SYN_OK;
  SYN_HIP(hipDeviceSynchronize());  // the old buffers may still be in use by queued work
  sk_panels = p.panels;
  SYN_TRY(sk_acc.alloc((size_t)16 * p.panels * 64 * sizeof(unsigned long long)));
  SYN_HIP(hipMemset(sk_acc.p, 0, sk_acc.bytes));  // calls leave them cleared
  SYN_HIP(hipDeviceSynchronize());  // the memset runs on the null stream, not the caller's
  return SYN_OK;
}

size_t QLinearInt8::part_elems_for(size_t m) const {
  if (m == 0 || m > 16 || n == 0 || k == 0) return 0;  // M > 16 runs the GEMM, no partials
  const GemvPlan p = make_gemv_plan(n, (size_t)chunks, false);
  return p.ksplit > 1 ? (size_t)p.ksplit * m * p.panels * 64 : 0;
}

syn_status_t QLinearInt8::gemv(size_t m, const int8_t *d_xq, size_t ldx, const float *d_sx,
                               float *d_y, size_t ldy, hipStream_t s) {
  if (m == 0 || n == 0 || k == 0) return SYN_OK;
  if (m > 16) return gemv_part(m, d_xq, ldx, d_sx, d_y, ldy, nullptr, s);
  SYN_TRY(ensure_sk());
  const GemvPlan p = make_gemv_plan(n, (size_t)chunks, false);
  kGemvLaunch[m](p, w.as<i32x4>(), scales.as<float>(), d_xq, (int)ldx, d_sx, d_y, (int)ldy,
                 nullptr, sk_acc.as<unsigned long long>(), (int)n, s);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

syn_status_t QLinearInt8::gemv_part(size_t m, const int8_t *d_xq, size_t ldx, const float *d_sx,
                                    float *d_y, size_t ldy, int *d_part, hipStream_t s) {
  if (m == 0 || n == 0 || k == 0) return SYN_OK;
  if (m > 16)  // qmatmul.zig:68-99: packed GEMM with the KC-chunked epilogue -> MFMA kernel
    return launch_gemm_w8a8(d_xq, ldx, d_sx, m, w.p, scales.as<float>(), n, chunks, d_y, ldy, s);
  const bool chunked = false;  // M <= 16 runs int8GemvRow per row (qmatmul.zig:54-66)
  const GemvPlan p = make_gemv_plan(n, (size_t)chunks, false);
  const size_t N64 = (size_t)p.panels * 64;
  for (size_t m0 = 0; m0 < m; m0 += 16) {
    const int mb = (int)std::min<size_t>(16, m - m0);
    kGemvLaunch[mb](p, w.as<i32x4>(), scales.as<float>(), d_xq + m0 * ldx, (int)ldx, d_sx + m0,
                    d_y + m0 * ldy, (int)ldy, d_part, nullptr, (int)n, s);
    SYN_LAUNCH_CHECK();
    if (p.ksplit > 1) {
      const int total = mb * (int)n;
      hipLaunchKernelGGL(k_gemv_reduce, dim3(cdiv(total, 256)), dim3(256), 0, s, d_part,
                         p.ksplit, mb, (int)n, (int)N64, d_sx + m0, scales.as<float>(),
                         d_y + m0 * ldy, (int)ldy, chunked ? 1 : 0);
      SYN_LAUNCH_CHECK();
    }
  }
  return SYN_OK;
}

// --------------------------------------------------------------- load time
// calibration.rs:11-24
void host_minmax_scales(const float *w, size_t ch, size_t chsz, float *scales) {
  for (size_t c = 0; c < ch; c++) {
    float mx = 0.0f;
    const float *r = w + c * chsz;
    for (size_t j = 0; j < chsz; j++) mx = std::fmax(mx, std::fabs(r[j]));
    scales[c] = (mx == 0.0f) ? 1.0f : mx / 127.0f;
  }
}

// int8_linear.rs:42-61 (kept in [N,K]; the reference then transposes to [K,N])
void host_quantize_weights_nk(const float *w, const float *scales, size_t n, size_t k,
                              int8_t *out) {
  for (size_t c = 0; c < n; c++) {
    const float s = scales[c];
    if (s == 0.0f) {
      std::memset(out + c * k, 0, k);
      continue;
    }
    const float inv = 1.0f / s;
    for (size_t j = 0; j < k; j++) {
      float v = std::round(w[c * k + j] * inv);
      v = std::min(127.0f, std::max(-128.0f, v));
      out[c * k + j] = (int8_t)v;
    }
  }
}

template <class Get>
static syn_status_t upload_panels(QLinearInt8 &L, const float *host_scales, size_t n, size_t k,
                                  Get get) {
  L.n = n;
  L.k = k;
  L.chunks = (int)cdiv(k, 16);
  const size_t P = cdiv(n, 64), C = (size_t)L.chunks;
  std::vector<int8_t> buf(P * C * 64 * 16, 0);
  for (size_t row = 0; row < n; row++) {
    const size_t p = row / 64, r = row % 64;
    for (size_t kk = 0; kk < k; kk++)
      buf[((p * C + kk / 16) * 64 + r) * 16 + kk % 16] = get(row, kk);
  }
  std::vector<float> sc(P * 64, 0.0f);
  std::memcpy(sc.data(), host_scales, n * sizeof(float));
  SYN_TRY(L.w.alloc(buf.size()));
  SYN_TRY(L.scales.alloc(sc.size() * sizeof(float)));
  SYN_HIP(hipMemcpy(L.w.p, buf.data(), buf.size(), hipMemcpyHostToDevice));
  SYN_HIP(hipMemcpy(L.scales.p, sc.data(), sc.size() * sizeof(float), hipMemcpyHostToDevice));
  return SYN_OK;
}

syn_status_t QLinearInt8::upload_nk(const int8_t *h, const float *hs, size_t n_, size_t k_) {
  return upload_panels(*this, hs, n_, k_, [&](size_t r, size_t kk) { return h[r * k_ + kk]; });
}

syn_status_t QLinearInt8::upload_kn(const int8_t *h, size_t ldb, const float *hs, size_t n_,
                                    size_t k_) {
  return upload_panels(*this, hs, n_, k_, [&](size_t r, size_t kk) { return h[kk * ldb + r]; });
}

syn_status_t QLinearInt8::from_f32(const float *w_nk, size_t n_, size_t k_) {
  std::vector<float> sc(n_);
  std::vector<int8_t> q(n_ * k_);
  host_minmax_scales(w_nk, n_, k_, sc.data());
  host_quantize_weights_nk(w_nk, sc.data(), n_, k_, q.data());
  return upload_nk(q.data(), sc.data(), n_, k_);
}

// ------------------------------------------------- allocation-free forward
// Device scratch of syn_hip_qlinear_forward_noalloc, for callers that cannot
// allocate (HIP graph capture, serving loops): quantized activation rows,
// their scales and the split-K partials of one call.  Each GPU the library
// runs on holds its own copy until the process ends; every call on a GPU
// shares it, so calls that overlap on one GPU race.
constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// zero bytes [k, ldq) of each of m rows
__global__ void k_zero_row_pad(int8_t *q, size_t m, size_t k, size_t ldq) {
  for (size_t r = blockIdx.x; r < m; r += gridDim.x)
    for (size_t j = k + threadIdx.x; j < ldq; j += blockDim.x) q[r * ldq + j] = 0;
}

// the device address of `scratch` on the current device, resolved on the
// first call per device (host code never passes the array's name itself)
static syn_status_t noalloc_scratch(unsigned char **out) {
  static std::mutex mu;
  static unsigned char *addr[64] = {};
  int dev = 0;
  SYN_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("qlinear_forward_noalloc: device index out of range");
    return SYN_ERR_INVALID_ARG;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void *p = nullptr;
    SYN_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) {
      set_error("qlinear_forward_noalloc: scratch address unavailable");
      return SYN_ERR_HIP;
    }
    addr[dev] = static_cast<unsigned char *>(p);
  }
  *out = addr[dev];
  return SYN_OK;
}

}  // namespace syn

// =================================================================== C ABI
using namespace syn;

struct syn_hip_qlinear_s {
  int fmt = 0;
  QLinearInt8 i8;
  QLinearQ4_0 q4;
  QLinearKQ kq;
  QLinearTernary ter;
};

static bool is_kq(int fmt) {
  return fmt == SYN_HIP_FMT_Q8_0 || fmt == SYN_HIP_FMT_Q4_K || fmt == SYN_HIP_FMT_Q6_K;
}

extern "C" {

syn_status_t syn_hip_quantize_rows(const float *d_x, size_t m, size_t k, size_t ldx, int8_t *d_q,
                                   size_t ldq, float *d_scales, void *stream) {
  if (!d_x || !d_q || !d_scales) return SYN_ERR_NULL_PTR;
  if (m == 0 || k == 0) return SYN_ERR_INVALID_ARG;  // exports.zig:1284
  if (ldx < k || ldq < k) return SYN_ERR_SHAPE_MISMATCH;
  SYN_TRY(ensure_init());
  return launch_quantize_rows(d_x, m, k, ldx, d_q, ldq, d_scales, pick_stream(stream));
}

syn_status_t syn_hip_qlinear_create(int fmt, size_t n, size_t k, const void *host_weights,
                                    const float *host_scales, int layout,
                                    syn_hip_qlinear_t **out) {
  if (!out || !host_weights) return SYN_ERR_NULL_PTR;
  if (n == 0 || k == 0) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  auto *h = new syn_hip_qlinear_s();
  h->fmt = fmt;
  syn_status_t st = SYN_OK;
  if (fmt == SYN_HIP_FMT_INT8) {
    if (!host_scales) st = SYN_ERR_NULL_PTR;
    else if (layout == SYN_HIP_LAYOUT_KN)
      st = h->i8.upload_kn((const int8_t *)host_weights, n, host_scales, n, k);
    else if (layout == SYN_HIP_LAYOUT_NK)
      st = h->i8.upload_nk((const int8_t *)host_weights, host_scales, n, k);
    else
      st = SYN_ERR_INVALID_ARG;
  } else if (fmt == SYN_HIP_FMT_Q4_0) {
    st = (k % 32) ? SYN_ERR_SHAPE_MISMATCH : h->q4.upload_packed((const uint8_t *)host_weights, n, k);
    h->q4.rs_f16_scales = layout == SYN_HIP_LAYOUT_GGUF_DEQUANT;
  } else if (is_kq(fmt)) {
    st = (k % kq_block_elems(fmt)) ? SYN_ERR_SHAPE_MISMATCH
                                   : h->kq.upload(fmt, (const uint8_t *)host_weights, n, k);
  } else if (fmt == SYN_HIP_FMT_TERNARY) {
    st = h->ter.upload_blocks((const uint8_t *)host_weights, n, k);
  } else {
    st = SYN_ERR_INVALID_ARG;
  }
  if (st != SYN_OK) {
    delete h;
    return st;
  }
  *out = h;
  return SYN_OK;
}

syn_status_t syn_hip_qlinear_from_f32(int fmt, size_t n, size_t k, const float *host_w,
                                      syn_hip_qlinear_t **out) {
  if (!out || !host_w) return SYN_ERR_NULL_PTR;
  if (n == 0 || k == 0) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  auto *h = new syn_hip_qlinear_s();
  h->fmt = fmt;
  syn_status_t st;
  if (fmt == SYN_HIP_FMT_INT8) st = h->i8.from_f32(host_w, n, k);
  else if (fmt == SYN_HIP_FMT_Q4_0) st = (k % 32) ? SYN_ERR_SHAPE_MISMATCH : h->q4.from_f32(host_w, n, k);
  else if (is_kq(fmt))
    st = (k % kq_block_elems(fmt)) ? SYN_ERR_SHAPE_MISMATCH : h->kq.from_f32(fmt, host_w, n, k);
  else if (fmt == SYN_HIP_FMT_TERNARY) st = h->ter.from_f32(host_w, n, k);
  else st = SYN_ERR_INVALID_ARG;
  if (st != SYN_OK) {
    delete h;
    return st;
  }
  *out = h;
  return SYN_OK;
}

syn_status_t syn_hip_qlinear_forward_pre_quantized(syn_hip_qlinear_t *h, size_t m,
                                                   const int8_t *d_xq, size_t ldxq,
                                                   const float *d_sx, float *d_y, void *stream) {
  if (!h) return SYN_ERR_NULL_PTR;
  if (h->fmt != SYN_HIP_FMT_INT8) return SYN_ERR_INVALID_ARG;
  if (m == 0) return SYN_OK;
  if (!d_xq || !d_sx || !d_y) return SYN_ERR_NULL_PTR;
  // the kernel reads activation rows in whole 16-byte chunks
  if (ldxq % 16 || ldxq < (size_t)h->i8.chunks * 16) return SYN_ERR_SHAPE_MISMATCH;
  return h->i8.gemv(m, d_xq, ldxq, d_sx, d_y, h->i8.n, pick_stream(stream));
}

syn_status_t syn_hip_qlinear_forward(syn_hip_qlinear_t *h, size_t m, const float *d_x,
                                     float *d_y, void *stream) {
  if (!h) return SYN_ERR_NULL_PTR;
  if (m == 0) return SYN_OK;
  if (!d_x || !d_y) return SYN_ERR_NULL_PTR;
  hipStream_t s = pick_stream(stream);
  if (h->fmt == SYN_HIP_FMT_Q4_0) return h->q4.gemv(m, d_x, h->q4.k, d_y, h->q4.n, s);
  if (is_kq(h->fmt)) return h->kq.gemv(m, d_x, h->kq.k, d_y, h->kq.n, s);
  if (h->fmt == SYN_HIP_FMT_TERNARY) return h->ter.gemv(m, d_x, h->ter.k, d_y, h->ter.n, s);
  if (h->fmt != SYN_HIP_FMT_INT8) return SYN_ERR_INVALID_ARG;
  QLinearInt8 &L = h->i8;
  const size_t ldq = (size_t)L.chunks * 16;
  if (L.xq_rows < m) {
    SYN_HIP(hipDeviceSynchronize());
    SYN_TRY(L.xq.alloc(m * ldq));
    SYN_TRY(L.sx.alloc(m * sizeof(float)));
    SYN_HIP(hipMemsetAsync(L.xq.p, 0, m * ldq, s));
    L.xq_rows = m;
  }
  SYN_TRY(launch_quantize_rows(d_x, m, L.k, L.k, L.xq.as<int8_t>(), ldq, L.sx.as<float>(), s));
  return L.gemv(m, L.xq.as<int8_t>(), ldq, L.sx.as<float>(), d_y, L.n, s);
}

syn_status_t syn_hip_qlinear_forward_noalloc(syn_hip_qlinear_t *h, size_t m, const float *d_x,
                                             float *d_y, void *stream) {
  if (!h) return SYN_ERR_NULL_PTR;
  if (h->fmt != SYN_HIP_FMT_INT8) {
    set_error("qlinear_forward_noalloc: INT8 handles only (the other formats use no scratch)");
    return SYN_ERR_INVALID_ARG;
  }
  if (m == 0) return SYN_OK;
  if (!d_x || !d_y) return SYN_ERR_NULL_PTR;
  QLinearInt8 &L = h->i8;
  const size_t ldq = (size_t)L.chunks * 16;
  // scratch: quantized rows [m, ldq] | row scales [m] | split-K partials
  const size_t off_sx = round_up(m * ldq, 256);
  const size_t off_part = round_up(off_sx + m * sizeof(float), 256);
  const size_t need = off_part + L.part_elems_for(std::min<size_t>(m, 16)) * sizeof(int);
  if (need > kNoAllocScratchBytes) {
    set_error("qlinear_forward_noalloc: " + std::to_string(m) + " rows of this linear need " +
              std::to_string(need) + " bytes of scratch, more than the fixed " +
              std::to_string(kNoAllocScratchBytes));
    return SYN_ERR_INVALID_ARG;
  }
  unsigned char *base = nullptr;
  SYN_TRY(noalloc_scratch(&base));
  hipStream_t s = pick_stream(stream);
  int8_t *xq = reinterpret_cast<int8_t *>(base);
  float *sx = reinterpret_cast<float *>(base + off_sx);
  int *part = reinterpret_cast<int *>(base + off_part);
  if (ldq > L.k) {  // the row padding the kernels read in whole 16-byte chunks starts at zero
    hipLaunchKernelGGL(k_zero_row_pad, dim3((unsigned)std::min<size_t>(m, 65535)), dim3(64), 0, s,
                       xq, m, L.k, ldq);
    SYN_LAUNCH_CHECK();
  }
  SYN_TRY(launch_quantize_rows(d_x, m, L.k, L.k, xq, ldq, sx, s));
  return L.gemv_part(m, xq, ldq, sx, d_y, L.n, part, s);
}

syn_status_t syn_hip_qlinear_info(const syn_hip_qlinear_t *h, size_t *n, size_t *k, int *fmt,
                                  size_t *weight_bytes) {
  if (!h) return SYN_ERR_NULL_PTR;
  size_t nn, kk, wb;
  if (h->fmt == SYN_HIP_FMT_INT8) {
    nn = h->i8.n; kk = h->i8.k; wb = h->i8.weight_bytes();
  } else if (h->fmt == SYN_HIP_FMT_Q4_0) {
    nn = h->q4.n; kk = h->q4.k; wb = h->q4.weight_bytes();
  } else if (h->fmt == SYN_HIP_FMT_TERNARY) {
    nn = h->ter.n; kk = h->ter.k; wb = h->ter.weight_bytes();
  } else {
    nn = h->kq.n; kk = h->kq.k; wb = h->kq.weight_bytes();
  }
  if (n) *n = nn;
  if (k) *k = kk;
  if (fmt) *fmt = h->fmt;
  if (weight_bytes) *weight_bytes = wb;
  return SYN_OK;
}

syn_status_t syn_hip_qlinear_time(syn_hip_qlinear_t *h, size_t m, const float *d_x,
                                  const int8_t *d_xq, size_t ldxq, const float *d_sx, float *d_y,
                                  size_t iters, float *avg_ms) {
  if (!h || !avg_ms) return SYN_ERR_NULL_PTR;
  if (iters == 0 || m == 0) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  hipStream_t s = default_stream();
  auto run = [&]() -> syn_status_t {
    if (h->fmt == SYN_HIP_FMT_INT8)
      return syn_hip_qlinear_forward_pre_quantized(h, m, d_xq, ldxq, d_sx, d_y, s);
    return syn_hip_qlinear_forward(h, m, d_x, d_y, s);
  };
  SYN_TRY(run());  // warm-up (and any one-time scratch allocation)
  SYN_HIP(hipStreamSynchronize(s));
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  SYN_HIP(hipEventRecord(a, s));
  syn_status_t st = SYN_OK;
  for (size_t i = 0; i < iters && st == SYN_OK; i++) st = run();
  SYN_HIP(hipEventRecord(b, s));
  SYN_HIP(hipEventSynchronize(b));
  float ms = 0.0f;
  SYN_HIP(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  SYN_TRY(st);
  *avg_ms = ms / (float)iters;
  return SYN_OK;
}

syn_status_t syn_hip_qlinear_time_set(syn_hip_qlinear_t *const *hs, size_t count, size_t m,
                                      const float *d_x, const int8_t *d_xq, size_t ldxq,
                                      const float *d_sx, float *d_y, size_t rounds,
                                      float *avg_ms) {
  if (!hs || !avg_ms) return SYN_ERR_NULL_PTR;
  if (count == 0 || rounds == 0 || m == 0) return SYN_ERR_INVALID_ARG;
  for (size_t i = 0; i < count; i++)
    if (!hs[i]) return SYN_ERR_NULL_PTR;
  SYN_TRY(ensure_init());
  hipStream_t s = default_stream();
  auto run = [&](syn_hip_qlinear_t *h) -> syn_status_t {
    if (h->fmt == SYN_HIP_FMT_INT8)
      return syn_hip_qlinear_forward_pre_quantized(h, m, d_xq, ldxq, d_sx, d_y, s);
    return syn_hip_qlinear_forward(h, m, d_x, d_y, s);
  };
  for (size_t i = 0; i < count; i++) SYN_TRY(run(hs[i]));  // warm-up, one-time scratch
  SYN_HIP(hipStreamSynchronize(s));
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  SYN_HIP(hipEventRecord(a, s));
  syn_status_t st = SYN_OK;
  for (size_t r = 0; r < rounds && st == SYN_OK; r++)
    for (size_t i = 0; i < count && st == SYN_OK; i++) st = run(hs[i]);
  SYN_HIP(hipEventRecord(b, s));
  SYN_HIP(hipEventSynchronize(b));
  float ms = 0.0f;
  SYN_HIP(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  SYN_TRY(st);
  *avg_ms = ms / (float)(rounds * count);
  return SYN_OK;
}

syn_status_t syn_hip_qlinear_destroy(syn_hip_qlinear_t *h) {
  delete h;
  return SYN_OK;
}

// ---- reference-signature entry points (host pointers) ----
syn_status_t syn_quantize_per_channel_int8(const float *data, size_t channels,
                                           size_t channel_size, int8_t *out, float *scales) {
  if (!data || !out || !scales) return SYN_ERR_NULL_PTR;
  if (channels == 0 || channel_size == 0) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  hipStream_t s = default_stream();
  DevBuf dx, dq, ds;
  const size_t n = channels * channel_size;
  SYN_TRY(dx.alloc(n * 4));
  SYN_TRY(dq.alloc(n));
  SYN_TRY(ds.alloc(channels * 4));
  SYN_HIP(hipMemcpyAsync(dx.p, data, n * 4, hipMemcpyHostToDevice, s));
  SYN_TRY(launch_quantize_rows(dx.as<float>(), channels, channel_size, channel_size,
                               dq.as<int8_t>(), channel_size, ds.as<float>(), s));
  SYN_HIP(hipMemcpyAsync(out, dq.p, n, hipMemcpyDeviceToHost, s));
  SYN_HIP(hipMemcpyAsync(scales, ds.p, channels * 4, hipMemcpyDeviceToHost, s));
  SYN_HIP(hipStreamSynchronize(s));
  return SYN_OK;
}

syn_status_t syn_qgemm_int8(size_t m, size_t n, size_t k, const int8_t *a, size_t lda,
                            const int8_t *b, size_t ldb, float *c, size_t ldc,
                            const float *scales_a, const float *scales_b) {
  if (!a || !b || !c || !scales_a || !scales_b) return SYN_ERR_NULL_PTR;
  if (m == 0 || n == 0 || k == 0) return SYN_OK;  // exports.zig:1331
  if (lda < k || ldb < n || ldc < n) return SYN_ERR_SHAPE_MISMATCH;
  SYN_TRY(ensure_init());
  hipStream_t s = default_stream();
  QLinearInt8 L;
  SYN_TRY(L.upload_kn(b, ldb, scales_b, n, k));
  const size_t ldq = (size_t)L.chunks * 16;
  std::vector<int8_t> ha(m * ldq, 0);
  for (size_t i = 0; i < m; i++) std::memcpy(ha.data() + i * ldq, a + i * lda, k);
  DevBuf dq, dsa, dc;
  SYN_TRY(dq.alloc(ha.size()));
  SYN_TRY(dsa.alloc(m * 4));
  SYN_TRY(dc.alloc(m * n * 4));
  SYN_HIP(hipMemcpyAsync(dq.p, ha.data(), ha.size(), hipMemcpyHostToDevice, s));
  SYN_HIP(hipMemcpyAsync(dsa.p, scales_a, m * 4, hipMemcpyHostToDevice, s));
  SYN_TRY(L.gemv(m, dq.as<int8_t>(), ldq, dsa.as<float>(), dc.as<float>(), n, s));
  std::vector<float> hc(m * n);
  SYN_HIP(hipMemcpyAsync(hc.data(), dc.p, m * n * 4, hipMemcpyDeviceToHost, s));
  SYN_HIP(hipStreamSynchronize(s));
  for (size_t i = 0; i < m; i++) std::memcpy(c + i * ldc, hc.data() + i * n, n * 4);
  return SYN_OK;
}

}  // extern "C"
