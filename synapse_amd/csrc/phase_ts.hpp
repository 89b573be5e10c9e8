// Optional phase timestamps of workgroup 0, thread 0 (compiled in only with
// -DSYN_PHASE_TIMING; read back with the syn_hip_debug_*phase_ts exports of
// the instrumented build).  Timestamps stay in registers until
// SYN_TS_FLUSH_TO at the end of the kernel, so the instrumented build issues
// no extra memory operations mid-kernel.
#pragma once

#ifdef SYN_PHASE_TIMING
#define SYN_TS_DECL unsigned long long syn_ts_[16] = {};
#define SYN_TS(i) syn_ts_[(i)] = __builtin_amdgcn_s_memtime()
#define SYN_TSR(i) syn_ts_[(i)] = __builtin_amdgcn_s_memrealtime()
// pass the kernel's timestamp registers into an inlined helper
#define SYN_TS_PARAM , unsigned long long *syn_ts_
#define SYN_TS_PASS , syn_ts_
#define SYN_TS_FLUSH_TO(arr, base)                                      \
  do {                                                                  \
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)         \
      for (int i_ = 0; i_ < 16; i_++) (arr)[(base) + i_] = syn_ts_[i_]; \
  } while (0)
#else
#define SYN_TS_DECL
#define SYN_TS_PARAM
#define SYN_TS_PASS
#define SYN_TS(i) \
  do {            \
  } while (0)
#define SYN_TSR(i) \
  do {             \
  } while (0)
#define SYN_TS_FLUSH_TO(arr, base) \
  do {                             \
  } while (0)
#endif
