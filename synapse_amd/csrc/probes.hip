// Achievable-peak probes of the GPU the library runs on (harness helpers,
// no reference counterpart): dense MFMA loops for f16 and i8, and an HBM
// streaming read.  The roofline fractions the benchmark reports use the
// published peaks; these give the measured ceilings beside them.
#include <algorithm>
#include <vector>

#include "common.hpp"
#include "reduce_order.hpp"

namespace syn {

typedef _Float16 pf16x8 __attribute__((ext_vector_type(8)));
typedef float pf32x4 __attribute__((ext_vector_type(4)));

// 8 independent accumulator chains per wave; operands change each iteration
// so nothing is hoisted
__global__ void __launch_bounds__(256) k_probe_mfma_f16(int iters, float *__restrict__ out) {
  pf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (float)(threadIdx.x + i));
    b[i] = (_Float16)(0.002f * (float)(threadIdx.x - i));
  }
  pf32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; c++) acc[c] = pf32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; c++) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  if (s == 12345.678f) out[blockIdx.x] = s;  // keeps the loop alive; never true in practice
}

typedef float pf32x16 __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) k_probe_mfma_f16_32(int iters, float *__restrict__ out) {
  pf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (float)(threadIdx.x + i));
    b[i] = (_Float16)(0.002f * (float)(threadIdx.x - i));
  }
  pf32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[c][r] = 0.0f;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < 4; c++)
      acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; c++) s += acc[c][0] + acc[c][5] + acc[c][10] + acc[c][15];
  if (s == 12345.678f) out[blockIdx.x] = s;
}

__global__ void __launch_bounds__(256) k_probe_mfma_i8(int iters, int *__restrict__ out) {
  i32x4 a, b;
  a = i32x4{(int)threadIdx.x, 3, 5, 7};
  b = i32x4{11, (int)threadIdx.x, 13, 17};
  i32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; c++) acc[c] = i32x4{0, 0, 0, 0};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int c = 0; c < 8; c++) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  if (s == 123456789) out[blockIdx.x] = s;
}

typedef int pi32x16 __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) k_probe_mfma_i8_32(int iters, int *__restrict__ out) {
  const i32x4 a = i32x4{(int)threadIdx.x, 3, 5, 7};
  const i32x4 b = i32x4{11, (int)threadIdx.x, 13, 17};
  pi32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[c][r] = 0;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) s += acc[c][0] + acc[c][5] + acc[c][10] + acc[c][15];
  if (s == 123456789) out[blockIdx.x] = s;
}

// streaming read: each thread sums 16-byte words over a grid-stride loop
__global__ void __launch_bounds__(256) k_probe_read(const i32x4 *__restrict__ p, size_t n16,
                                                    int *__restrict__ out) {
  i32x4 s = i32x4{0, 0, 0, 0};
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const i32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const i32x4 c = __builtin_nontemporal_load(p + i + 2 * stride),
                d = __builtin_nontemporal_load(p + i + 3 * stride);
    s += a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) s += __builtin_nontemporal_load(p + i);
  if ((s.x ^ s.y ^ s.z ^ s.w) == 0x5eed5eed) out[blockIdx.x] = 1;
}

// the reference-order sequential sums of n values: out[0] one lane's chain
// (seq_sum), out[1] the wave-cooperative chain (wave_seq_sum), out[2] its
// clocks, out[3] the long-row wave chain (wave_seq_sum_long), out[4] its
// clocks
__global__ void __launch_bounds__(64) k_probe_seq_sum(const float *v, int n, float *out) {
  extern __shared__ __align__(16) float sv[];
  for (int j = threadIdx.x; j < ((n + 3) & ~3); j += 64) sv[j] = j < n ? v[j] : 0.0f;
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const float w = wave_seq_sum(sv, n, 0.0f);
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const float wl = wave_seq_sum_long(sv, n, 0.0f);
  const unsigned long long t2 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = seq_sum(sv, n);
    out[1] = w;
    out[2] = (float)(t1 - t0);
    out[3] = wl;
    out[4] = (float)(t2 - t1);
  }
}

}  // namespace syn

using namespace syn;

extern "C" syn_status_t syn_hip_probe_seq_sum(const float *host, size_t n, float *out5) {
  if (!host || !out5) return SYN_ERR_NULL_PTR;
  if (n == 0 || n > 16384) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  DevBuf dv, dout;
  SYN_TRY(dv.alloc(n * 4));
  SYN_TRY(dout.alloc(32));
  SYN_HIP(hipMemcpy(dv.p, host, n * 4, hipMemcpyHostToDevice));
  hipLaunchKernelGGL(k_probe_seq_sum, dim3(1), dim3(64), ((n + 3) & ~(size_t)3) * 4, 0,
                     dv.as<float>(), (int)n, dout.as<float>());
  SYN_LAUNCH_CHECK();
  SYN_HIP(hipMemcpy(out5, dout.p, 20, hipMemcpyDeviceToHost));
  return SYN_OK;
}

extern "C" syn_status_t syn_hip_probe_mfma(int kind, size_t iters, double *tflops) {
  if (!tflops) return SYN_ERR_NULL_PTR;
  if (iters == 0 || iters > (1u << 24) || kind < 0 || kind > 3) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  int dev = 0, cus = 256;
  SYN_HIP(hipGetDevice(&dev));
  SYN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int blocks = cus * 8;  // 8 waves per SIMD
  DevBuf out;
  SYN_TRY(out.alloc((size_t)blocks * 4));
  hipStream_t s = default_stream();
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  for (int rep = 0; rep < 2; rep++) {  // the first run warms up clocks
    SYN_HIP(hipEventRecord(a, s));
    if (kind == 0)
      hipLaunchKernelGGL(k_probe_mfma_f16, dim3(blocks), dim3(256), 0, s, (int)iters,
                         out.as<float>());
    else if (kind == 1)
      hipLaunchKernelGGL(k_probe_mfma_i8, dim3(blocks), dim3(256), 0, s, (int)iters,
                         out.as<int>());
    else if (kind == 2)
      hipLaunchKernelGGL(k_probe_mfma_f16_32, dim3(blocks), dim3(256), 0, s, (int)iters,
                         out.as<float>());
    else
      hipLaunchKernelGGL(k_probe_mfma_i8_32, dim3(blocks), dim3(256), 0, s, (int)iters,
                         out.as<int>());
    SYN_LAUNCH_CHECK();
    SYN_HIP(hipEventRecord(b, s));
    SYN_HIP(hipEventSynchronize(b));
  }
  float ms = 0.0f;
  SYN_HIP(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  // per MFMA: 16x16x32 f16 = 16384 flops (8 chains); 16x16x64 i8 = 32768
  // ops (8 chains); 32x32x16 f16 = 32768 flops (4 chains); 32x32x32 i8 =
  // 65536 ops (4 chains)
  const double per = kind == 0 ? 16384.0 : kind == 3 ? 65536.0 : 32768.0;
  const double chains = kind >= 2 ? 4.0 : 8.0;
  const double ops = (double)blocks * 4 /* waves */ * chains * (double)iters * per;
  *tflops = ops / ((double)ms * 1e-3) / 1e12;
  return SYN_OK;
}

extern "C" syn_status_t syn_hip_probe_hbm_read(size_t bytes, double *gb_s) {
  if (!gb_s) return SYN_ERR_NULL_PTR;
  if (bytes < (1u << 20)) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  bytes &= ~(size_t)15;
  DevBuf buf, out;
  SYN_TRY(buf.alloc(bytes));
  hipStream_t s = default_stream();
  SYN_HIP(hipMemsetAsync(buf.p, 1, bytes, s));
  int dev = 0, cus = 256;
  SYN_HIP(hipGetDevice(&dev));
  SYN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int blocks = cus * 16;
  SYN_TRY(out.alloc((size_t)blocks * 4));
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  float best = 1e30f;
  for (int rep = 0; rep < 4; rep++) {
    SYN_HIP(hipEventRecord(a, s));
    hipLaunchKernelGGL(k_probe_read, dim3(blocks), dim3(256), 0, s, buf.as<i32x4>(), bytes / 16,
                       out.as<int>());
    SYN_LAUNCH_CHECK();
    SYN_HIP(hipEventRecord(b, s));
    SYN_HIP(hipEventSynchronize(b));
    float ms = 0.0f;
    SYN_HIP(hipEventElapsedTime(&ms, a, b));
    if (rep > 0 && ms < best) best = ms;
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *gb_s = (double)bytes / ((double)best * 1e-3) / 1e9;
  return SYN_OK;
}

// ---------------------------------------------------------------- step structure
// What a dependency level of the decode step costs when it is a kernel
// boundary, and what it would cost as a grid barrier inside one persistent
// kernel (the two ways to order the step's stages).
namespace syn {

__global__ void k_probe_tiny(float *out, int i) {
  if (threadIdx.x == 0) out[blockIdx.x] = (float)i;
}

// mode 0: one arrival counter, the last arrival publishes the generation,
// the others poll it with device-scope read-modify-writes (fetch_or 0);
// mode 1: eight arrival counters (by workgroup id), their last arrivals
// count on a top counter, whose last arrival publishes; everyone polls with
// a short sleep; modes 2 and 3: as 0 and 1, but the generation is published
// by a device-scope atomic store and polled by device-scope atomic loads
// (no read-modify-write traffic on the polled word), no sleep.  Every poll
// gives up after a bounded number of tries (counted in *timeouts, and the
// workgroup leaves), so a wait cannot hang the GPU.
__global__ void k_probe_barrier(unsigned *cnt, int nbar, int mode, unsigned *timeouts,
                                unsigned long long *ts) {
  const unsigned G = gridDim.x;
  __shared__ unsigned s_stop;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int b = 0; b < nbar; b++) {
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned target = (unsigned)(b + 1);
      bool late = false;
      bool arrive_top = true;
      const bool grouped = mode == 1 || mode == 3, loads = mode >= 2;
      if (grouped) {
        const unsigned grp = blockIdx.x & 7, gsz = (G - grp + 7) / 8;
        const unsigned old = __hip_atomic_fetch_add(cnt + 128 + 64 * grp, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        arrive_top = old == target * gsz - 1;
      }
      const unsigned need = grouped ? 8u : G;
      if (arrive_top) {
        const unsigned o2 =
            __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (o2 == target * need - 1) {
          if (loads)
            __hip_atomic_store(cnt + 64, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            __hip_atomic_exchange(cnt + 64, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      for (long n = 0;; n++) {
        const unsigned g =
            loads ? __hip_atomic_load(cnt + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                  : __hip_atomic_fetch_or(cnt + 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (g >= target) break;
        if (mode == 1) __builtin_amdgcn_s_sleep(1);
        if (n > 1000000) {
          late = true;
          break;
        }
      }
      if (late) atomicAdd(timeouts, 1u);
      s_stop = late ? 1u : 0u;
    }
    __syncthreads();
    if (s_stop) return;
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    ts[2 * blockIdx.x] = t0;
    ts[2 * blockIdx.x + 1] = t1;
  }
}

}  // namespace syn

// Graph replay of n dependent tiny kernels of `wgs` workgroups: us per kernel.
extern "C" syn_status_t syn_hip_probe_graph_floor(int n, int wgs, double *us_per_kernel) {
  if (!us_per_kernel) return SYN_ERR_NULL_PTR;
  if (n < 1 || n > 4096 || wgs < 1 || wgs > 65536) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  hipStream_t s;
  SYN_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  DevBuf out;
  SYN_TRY(out.alloc((size_t)wgs * 4));
  hipGraph_t g;
  hipGraphExec_t ge = nullptr;
  SYN_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  for (int i = 0; i < n; i++)
    hipLaunchKernelGGL(k_probe_tiny, dim3(wgs), dim3(256), 0, s, out.as<float>(), i);
  SYN_HIP(hipStreamEndCapture(s, &g));
  hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  for (int w = 0; w < 3; w++) SYN_HIP(hipGraphLaunch(ge, s));
  SYN_HIP(hipEventRecord(a, s));
  const int reps = 20;
  for (int r = 0; r < reps; r++) SYN_HIP(hipGraphLaunch(ge, s));
  SYN_HIP(hipEventRecord(b, s));
  SYN_HIP(hipEventSynchronize(b));
  float ms = 0.0f;
  SYN_HIP(hipEventElapsedTime(&ms, a, b));
  *us_per_kernel = (double)ms * 1e3 / ((double)reps * n);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipGraphExecDestroy(ge);
  (void)hipStreamDestroy(s);
  return SYN_OK;
}

// nbar grid barriers among `wgs` co-resident workgroups (cooperative launch):
// us per barrier, from the first workgroup's start to the last one's end
extern "C" syn_status_t syn_hip_probe_grid_barrier(int wgs, int mode, int nbar,
                                                   double *us_per_barrier, int *timeouts) {
  if (!us_per_barrier || !timeouts) return SYN_ERR_NULL_PTR;
  if (wgs < 8 || nbar < 1 || nbar > 100000 || mode < 0 || mode > 3)
    return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  int dev = 0, cus = 0;
  SYN_HIP(hipGetDevice(&dev));
  SYN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (wgs > cus) return SYN_ERR_INVALID_ARG;  // one workgroup per CU: all co-resident
  DevBuf cnt, to, ts;
  SYN_TRY(cnt.alloc(4096 * 4));
  SYN_TRY(to.alloc(4));
  SYN_TRY(ts.alloc((size_t)wgs * 16));
  SYN_HIP(hipMemset(cnt.p, 0, cnt.bytes));
  SYN_HIP(hipMemset(to.p, 0, 4));
  SYN_HIP(hipDeviceSynchronize());
  unsigned *pc = cnt.as<unsigned>(), *pt = to.as<unsigned>();
  unsigned long long *pts = ts.as<unsigned long long>();
  void *args[] = {&pc, &nbar, &mode, &pt, &pts};
  SYN_HIP(hipLaunchCooperativeKernel((const void *)k_probe_barrier, dim3(wgs), dim3(256), args,
                                     0, default_stream()));
  SYN_HIP(hipStreamSynchronize(default_stream()));
  std::vector<unsigned long long> h((size_t)wgs * 2);
  SYN_HIP(hipMemcpy(h.data(), ts.p, h.size() * 8, hipMemcpyDeviceToHost));
  unsigned ht = 0;
  SYN_HIP(hipMemcpy(&ht, to.p, 4, hipMemcpyDeviceToHost));
  unsigned long long lo = ~0ull, hi = 0;
  for (int i = 0; i < wgs; i++) {
    lo = std::min(lo, h[2 * i]);
    hi = std::max(hi, h[2 * i + 1]);
  }
  *timeouts = (int)ht;
  *us_per_barrier = ht ? 0.0 : (double)(hi - lo) * 0.01 / nbar;  // s_memrealtime: 100 MHz
  return SYN_OK;
}
