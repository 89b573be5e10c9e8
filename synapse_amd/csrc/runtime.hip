// Device bookkeeping behind the C ABI: error strings, per-device library
// stream, memory and hipEvent timers, plus the host-side f16 helpers and the
// synthetic-input generator.
#include <cmath>
#include <algorithm>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common.hpp"

namespace syn {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

syn_status_t hip_fail(hipError_t e, const char *what, const char *file, int line) {
  set_error(std::string(what) + ": " + hipGetErrorString(e) + " (" + file + ":" +
            std::to_string(line) + ")");
  if (e == hipErrorOutOfMemory) return SYN_ERR_OUT_OF_MEMORY;
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return SYN_ERR_NO_DEVICE;
  if (e == hipErrorLaunchFailure || e == hipErrorInvalidConfiguration)
    return SYN_ERR_LAUNCH;
  return SYN_ERR_HIP;
}

static std::mutex g_mu;
static std::vector<hipStream_t> g_streams;  // per device

syn_status_t ensure_init() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice", __FILE__, __LINE__);
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_streams.size() <= dev) g_streams.resize(dev + 1, nullptr);
  if (!g_streams[dev]) {
    hipStream_t s;
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreate", __FILE__, __LINE__);
    g_streams[dev] = s;
  }
  return SYN_OK;
}

LaunchEvents &launch_events() {
  thread_local LaunchEvents e;
  return e;
}

hipStream_t default_stream() {
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_streams.size() > dev && g_streams[dev]) return g_streams[dev];
  return nullptr;
}

float f16_to_f32_ieee(uint16_t bits) {
  uint32_t sign = ((uint32_t)(bits >> 15)) << 31, exp5 = (bits >> 10) & 0x1fu,
           mant = bits & 0x3ffu, out;
  if (exp5 == 0) {
    if (mant == 0) {
      out = sign;
    } else {
      uint32_t m = mant, e = 0;
      while ((m & 0x400u) == 0) { m <<= 1; e++; }
      out = sign | ((127u - 15u + 1u - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp5 == 31) {
    out = sign | 0x7f800000u | (mant << 13);
  } else {
    out = sign | ((exp5 + 127u - 15u) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

uint16_t f32_to_f16_trunc(float val) {
  uint32_t bits;
  std::memcpy(&bits, &val, 4);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exp = (int32_t)((bits >> 23) & 0xffu);
  uint32_t man = bits & 0x7fffffu;
  if (exp == 0) return (uint16_t)sign;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man != 0 ? 0x200u : 0u));
  int32_t ne = exp - 127 + 15;
  if (ne >= 31) return (uint16_t)(sign | 0x7c00u);
  if (ne <= 0) return (uint16_t)sign;
  return (uint16_t)(sign | ((uint32_t)ne << 10) | (man >> 13));
}

// SplitMix64 + Box-Muller: the synthetic-input contract (seed per tensor).
static inline uint64_t splitmix64(uint64_t &s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

void fill_normal(float *dst, size_t n, uint64_t seed, float stddev) {
  uint64_t s = seed;
  const double two_pi = 6.283185307179586476925286766559;
  const double sd = (double)stddev;
  size_t i = 0;
  while (i < n) {
    double u1 = ((double)(splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
    double r = std::sqrt(-2.0 * std::log(u1));
    double z0 = r * std::cos(two_pi * u2);
    double z1 = r * std::sin(two_pi * u2);
    dst[i++] = (float)(z0 * sd);
    if (i < n) dst[i++] = (float)(z1 * sd);
  }
}

// Same stream as fill_normal, split over threads: pair p (elements 2p, 2p+1)
// uses draws 2p and 2p+1, so a chunk starting at even element e starts from
// state seed + e * gamma.
void fill_normal_parallel(float *dst, size_t n, uint64_t seed, float stddev) {
  unsigned nt = std::thread::hardware_concurrency();
  nt = nt == 0 ? 1 : (nt > 16 ? 16 : nt);
  if (n < (size_t)1 << 20 || nt == 1) {
    fill_normal(dst, n, seed, stddev);
    return;
  }
  const size_t per = ((n / nt) + 1) & ~(size_t)1;
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; t++) {
    const size_t b = (size_t)t * per;
    if (b >= n) break;
    const size_t e = std::min(n, b + per);
    th.emplace_back([=] { fill_normal(dst + b, e - b, seed + (uint64_t)b * 0x9E3779B97F4A7C15ULL, stddev); });
  }
  for (auto &x : th) x.join();
}

}  // namespace syn

using namespace syn;

extern "C" {

const char *syn_hip_last_error(void) { return g_last_error.c_str(); }

syn_status_t syn_hip_device_count(int *count) {
  if (!count) return SYN_ERR_NULL_PTR;
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e != hipSuccess) {
    *count = 0;
    return hip_fail(e, "hipGetDeviceCount", __FILE__, __LINE__);
  }
  return SYN_OK;
}

syn_status_t syn_hip_init(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    set_error("no HIP device visible");
    return SYN_ERR_NO_DEVICE;
  }
  if (device < 0 || device >= n) return SYN_ERR_INVALID_ARG;
  SYN_HIP(hipSetDevice(device));
  return ensure_init();
}

syn_status_t syn_hip_malloc(void **dptr, size_t bytes) {
  if (!dptr) return SYN_ERR_NULL_PTR;
  SYN_TRY(ensure_init());
  hipError_t e = hipMalloc(dptr, bytes ? bytes : 256);
  if (e != hipSuccess) {
    *dptr = nullptr;
    return hip_fail(e, "hipMalloc", __FILE__, __LINE__);
  }
  return SYN_OK;
}

syn_status_t syn_hip_free(void *dptr) {
  if (!dptr) return SYN_OK;
  SYN_HIP(hipFree(dptr));
  return SYN_OK;
}

syn_status_t syn_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (!dst || !src) return bytes ? SYN_ERR_NULL_PTR : SYN_OK;
  SYN_TRY(ensure_init());
  SYN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, default_stream()));
  SYN_HIP(hipStreamSynchronize(default_stream()));
  return SYN_OK;
}

syn_status_t syn_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (!dst || !src) return bytes ? SYN_ERR_NULL_PTR : SYN_OK;
  SYN_TRY(ensure_init());
  SYN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, default_stream()));
  SYN_HIP(hipStreamSynchronize(default_stream()));
  return SYN_OK;
}

syn_status_t syn_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  if (!dst || !src) return bytes ? SYN_ERR_NULL_PTR : SYN_OK;
  SYN_TRY(ensure_init());
  SYN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, default_stream()));
  SYN_HIP(hipStreamSynchronize(default_stream()));
  return SYN_OK;
}

syn_status_t syn_hip_memset(void *dst, int value, size_t bytes) {
  if (!dst) return bytes ? SYN_ERR_NULL_PTR : SYN_OK;
  SYN_TRY(ensure_init());
  SYN_HIP(hipMemsetAsync(dst, value, bytes, default_stream()));
  SYN_HIP(hipStreamSynchronize(default_stream()));
  return SYN_OK;
}

syn_status_t syn_hip_synchronize(void) {
  SYN_HIP(hipDeviceSynchronize());
  return SYN_OK;
}

syn_status_t syn_hip_stream_create(void **stream) {
  if (!stream) return SYN_ERR_NULL_PTR;
  SYN_TRY(ensure_init());
  hipStream_t s;
  SYN_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = (void *)s;
  return SYN_OK;
}

syn_status_t syn_hip_stream_destroy(void *stream) {
  if (!stream) return SYN_OK;
  SYN_HIP(hipStreamDestroy((hipStream_t)stream));
  return SYN_OK;
}

syn_status_t syn_hip_stream_synchronize(void *stream) {
  SYN_TRY(ensure_init());
  SYN_HIP(hipStreamSynchronize(pick_stream(stream)));
  return SYN_OK;
}

struct syn_hip_timer_s {
  hipEvent_t a = nullptr, b = nullptr;
};

syn_status_t syn_hip_timer_create(syn_hip_timer_t **timer) {
  if (!timer) return SYN_ERR_NULL_PTR;
  SYN_TRY(ensure_init());
  auto *t = new syn_hip_timer_t();
  if (hipEventCreate(&t->a) != hipSuccess || hipEventCreate(&t->b) != hipSuccess) {
    delete t;
    set_error("hipEventCreate failed");
    return SYN_ERR_HIP;
  }
  *timer = t;
  return SYN_OK;
}

syn_status_t syn_hip_timer_start(syn_hip_timer_t *t, void *stream) {
  if (!t) return SYN_ERR_NULL_PTR;
  SYN_HIP(hipEventRecord(t->a, pick_stream(stream)));
  return SYN_OK;
}

syn_status_t syn_hip_timer_stop(syn_hip_timer_t *t, void *stream) {
  if (!t) return SYN_ERR_NULL_PTR;
  SYN_HIP(hipEventRecord(t->b, pick_stream(stream)));
  return SYN_OK;
}

syn_status_t syn_hip_timer_elapsed_ms(syn_hip_timer_t *t, float *ms) {
  if (!t || !ms) return SYN_ERR_NULL_PTR;
  SYN_HIP(hipEventSynchronize(t->b));
  SYN_HIP(hipEventElapsedTime(ms, t->a, t->b));
  return SYN_OK;
}

syn_status_t syn_hip_timer_destroy(syn_hip_timer_t *t) {
  if (!t) return SYN_OK;
  (void)hipEventDestroy(t->a);
  (void)hipEventDestroy(t->b);
  delete t;
  return SYN_OK;
}

syn_status_t syn_hip_fill_normal(float *host_dst, size_t n, uint64_t seed, float stddev) {
  if (!host_dst) return n ? SYN_ERR_NULL_PTR : SYN_OK;
  fill_normal(host_dst, n, seed, stddev);
  return SYN_OK;
}

}  // extern "C"
