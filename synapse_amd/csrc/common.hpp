// Shared host/device helpers for the gfx950 backend.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/synapse_hip.h"

namespace syn {

// ---------------------------------------------------------------- errors
void set_error(const std::string &msg);
syn_status_t hip_fail(hipError_t e, const char *what, const char *file, int line);

#define SYN_HIP(call)                                                      \
  do {                                                                     \
    hipError_t e_ = (call);                                                \
    if (e_ != hipSuccess) return ::syn::hip_fail(e_, #call, __FILE__, __LINE__); \
  } while (0)

#define SYN_LAUNCH_CHECK()                                                 \
  do {                                                                     \
    hipError_t e_ = hipGetLastError();                                     \
    if (e_ != hipSuccess) return ::syn::hip_fail(e_, "kernel launch", __FILE__, __LINE__); \
  } while (0)

#define SYN_TRY(expr)                                                      \
  do {                                                                     \
    syn_status_t s_ = (expr);                                              \
    if (s_ != SYN_OK) return s_;                                           \
  } while (0)

// ---------------------------------------------------------------- runtime
// Library stream of the current device (created on first use, default
// priority).  stream==nullptr in the API means this stream.
syn_status_t ensure_init();
hipStream_t default_stream();
inline hipStream_t pick_stream(void *s) { return s ? (hipStream_t)s : default_stream(); }

// Kernel timing with the dispatch's own timestamps: when `start` is set, the
// next SYN_LAUNCH records the kernel's start and end on these events
// (hipExtLaunchKernelGGL) and clears them; otherwise it is a plain launch.
// Host-thread local; set only by benchmark helpers, never under capture.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents &launch_events();
#define SYN_LAUNCH(kern, grid, block, shm, stream, ...)                                   \
  do {                                                                                  \
    ::syn::LaunchEvents &ev_ = ::syn::launch_events();                                  \
    if (ev_.start) {                                                                    \
      hipExtLaunchKernelGGL(kern, grid, block, shm, stream, ev_.start, ev_.stop, 0u,    \
                            __VA_ARGS__);                                               \
      ev_.start = ev_.stop = nullptr;                                                   \
    } else {                                                                            \
      hipLaunchKernelGGL(kern, grid, block, shm, stream, __VA_ARGS__);                  \
    }                                                                                   \
  } while (0)

// RAII device buffer (hipMalloc'd once at set-up, never on a hot path).
struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  DevBuf(DevBuf &&o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; o.bytes = 0; }
  DevBuf &operator=(DevBuf &&o) noexcept {
    if (this != &o) { release(); p = o.p; bytes = o.bytes; o.p = nullptr; o.bytes = 0; }
    return *this;
  }
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  syn_status_t alloc(size_t n) {
    release();
    if (n == 0) n = 256;
    hipError_t e = hipMalloc(&p, n);
    if (e != hipSuccess) {
      p = nullptr;
      set_error(std::string("hipMalloc failed: ") + hipGetErrorString(e));
      return SYN_ERR_OUT_OF_MEMORY;
    }
    bytes = n;
    return SYN_OK;
  }
  template <class T> T *as() const { return reinterpret_cast<T *>(p); }
};

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
__host__ __device__ inline int round_up4(int x) { return (x + 3) & ~3; }
inline size_t cdiv(size_t x, size_t a) { return (x + a - 1) / a; }

// ---------------------------------------------------------------- host f16
// qmatmul.zig:346-371 (IEEE-exact)
float f16_to_f32_ieee(uint16_t bits);
// q4_linear.rs:9-33 (truncating)
uint16_t f32_to_f16_trunc(float v);

}  // namespace syn

// ---------------------------------------------------------------- device math
// Fixed point for order-free float sums (the fused f32 decoders' split-K
// atomics): value * 2^32 in an int64; sums of these are exact in any order,
// so split-K workgroups can add them with integer atomics.  A value is
// saturated at +-2^27 (2^59 fixed), far beyond any activation, so that up to
// 16 saturated addends cannot wrap the int64; NaN saturates to +2^27 (the
// fused decoders turn a non-finite activation into a saturated finite one
// instead of propagating it).
__device__ __forceinline__ long long kqf_fix(float v) {
  const double d = (double)v * 4294967296.0;
  constexpr double lim = 576460752303423488.0;  // 2^59
  return d != d ? (long long)lim : __double2ll_rn(fmin(fmax(d, -lim), lim));
}
__device__ __forceinline__ float kqf_unfix(long long a) {
  return (float)((double)a * 2.3283064365386963e-10);
}

// clang vector types (usable with __builtin_nontemporal_load)
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// T[i] = asuint64(2^(i/32)) - (i << 47)
static __constant__ uint64_t syn_exp2_tab[32] = {
      0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
      0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
      0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
      0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
      0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
      0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
      0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
      0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

// glibc 2.35 expf (the published exp2f_data / e_expf.c algorithm, 32-entry
// table, degree-3 polynomial in double) including the FMA contractions of the
// x86-64 FMA ifunc build.  Upstream: glibc sysdeps/ieee754/flt-32/e_expf.c
// and e_exp2f_data.c (LGPL-2.1-or-later), contributed from ARM's
// optimized-routines (math/expf.c, exp2f_data.c; MIT OR Apache-2.0 WITH
// LLVM-exception).  The table values here were recomputed from 2^(i/32).  Checked on the CPU against the host's expf over all
// 2^32 inputs; keeps SiLU and softmax bit-identical to the reference's
// f32::exp on Linux.
// tab: the 32-entry table above, or a copy of it (in LDS, so that a lookup
// does not wait behind outstanding global loads)
__device__ __forceinline__ float syn_expf_tab(float x, const uint64_t *tab) {
  const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double SHIFT = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const uint32_t ux = __float_as_uint(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88 or nan
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = __builtin_fma(InvLn2N, xd, SHIFT);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd -= SHIFT;
  const double r = __builtin_fma(InvLn2N, xd, -kd);
  uint64_t t = tab[ki & 31u];
  t += ki << 47;
  const double s = __longlong_as_double((long long)t);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

__device__ __forceinline__ float syn_expf(float x) { return syn_expf_tab(x, syn_exp2_tab); }

// reference SiLU: x / (1 + exp(-x))  (ops/activation.rs:30-32)
__device__ __forceinline__ float syn_silu(float x) { return x / (1.0f + syn_expf(-x)); }
__device__ __forceinline__ float syn_silu_tab(float x, const uint64_t *tab) {
  return x / (1.0f + syn_expf_tab(-x, tab));
}

// Rust converter f16->f32 (weight_loading/converter.rs:12-40): subnormal
// inputs come out at half their IEEE value (shift counter starts at 1).
__device__ __forceinline__ float syn_f16_to_f32_rs(uint32_t h) {
  // branch-free (selects), so it can sit in software-pipelined loops
  const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  const uint32_t s = sign << 31;
  const uint32_t normal = s | ((exp + 127u - 15u) << 23) | (mant << 13);
  const uint32_t lz = __clz(mant | 1u) - 21;  // shifts until bit 10 is set (mant != 0)
  const uint32_t sub = s | ((127u - 15u + 1u - (1u + lz)) << 23) | (((mant << lz) & 0x3ffu) << 13);
  const uint32_t special = s | (0xffu << 23) | (mant << 13);
  const uint32_t r = exp == 0 ? (mant == 0 ? s : sub) : (exp == 31 ? special : normal);
  return __uint_as_float(r);
}

// The same values through the hardware conversion: IEEE f16 -> f32 (exact,
// f16 denormals are on) halved for subnormal inputs.  No data-dependent
// control flow, so a pipelined loop keeps precise memory-counter waits; NaN
// payloads may differ from the bit-built value (a NaN stays a NaN).
__device__ __forceinline__ float syn_f16_to_f32_rs_hw(uint32_t h) {
  const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  return f * ((h & 0x7c00u) == 0 ? 0.5f : 1.0f);
}

// lane l's 16 bytes at src land at lds_base + 16 * l (gfx950
// global_load_lds_dwordx4; lds_base is wave-uniform)
__device__ __forceinline__ void g2lds16(const void *src, void *lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_base, 16,
                                   0, 0);
}

// IEEE f16->f32 (qmatmul.zig:346-371 semantics)
__device__ __forceinline__ float syn_f16_to_f32_ieee(uint32_t h) {
  const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  if (exp == 0) {
    if (mant == 0) return __uint_as_float(sign << 31);
    const uint32_t lz = __clz(mant) - 21;
    const uint32_t m = ((mant << lz) & 0x3ffu) << 13;
    return __uint_as_float((sign << 31) | ((127u - 15u + 1u - lz) << 23) | m);
  }
  if (exp == 31) return __uint_as_float((sign << 31) | 0x7f800000u | (mant << 13));
  return __uint_as_float((sign << 31) | ((exp + 127u - 15u) << 23) | (mant << 13));
}
