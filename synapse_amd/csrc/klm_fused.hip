// Fused f32 decode step of the K-quant CausalLM (one token, batch 1).
//
// The op-by-op step (klm.hip layer()) launches ten kernels per layer:
// RMSNorm, QKV GEMV + split-K reduce, attention, O GEMV + reduce, RMSNorm,
// gate|up GEMV, SwiGLU, down GEMV + reduce.  At batch 1 each of them is
// latency-bound; this file rebuilds the layer as five:
//
//   K1  QKV rows of rmsnorm(r), split K
//   K2  per (kv head, 64-position chunk): q/k/v of the new token, head
//       norms, RoPE, KV append, scores, chunk softmax and P.V for the group's
//       query heads (flash-decoding partials)
//   K3  combine of the chunk partials ; O rows, split K, added into r
//   K4  gate and up rows of rmsnorm(r) over the whole K ; h = silu(gate) * up
//   K5  down rows of h, split K, added into r
//
// then the lm_head rows of rmsnorm(r) with a per-panel top-2, and one merge.
// The residual stream r and the QKV outputs are fixed-point accumulators
// (value * 2^32 in an int64): split-K workgroups add their dot products with
// integer atomics, whose sums are exact in any order, so the step is
// deterministic and a consumer reads one vector.  A prologue that needs a
// whole row (RMSNorm's sum of squares, the softmax combine) is computed
// redundantly by every workgroup; its loads are issued before the weight
// loads, and the norm's 1/rms multiplies the finished dot products.
//
// The math is the reference's f32 CausalLM (models/lm/causal_lm.rs:195-278,
// decoder_layer.rs:51-138) with the weights decoded exactly (kq_unit.hpp); the
// sums run in tree or split order and the residual is held to 2^-32, so
// results agree with it to rounding (tests grade this path by tolerance
// against the oracle).
#include <algorithm>
#include <type_traits>

#include "decode_fused.hpp"
#include "klm_fused.hpp"
#include "kq_unit.hpp"
#include "liv_conv.hpp"
#include "phase_ts.hpp"

namespace syn {

namespace {

#ifdef SYN_PHASE_TIMING
__device__ unsigned long long kqf_phase_ts[256];
#endif

constexpr int kMaxNW = 16;      // waves per GEMV workgroup: one 256-element unit each
constexpr int kRounds = 4;      // 4-element groups of a norm row per thread: H <= 4096
constexpr int kGmax = 8;        // query heads per kv head
constexpr size_t kLdsMax = 60 * 1024;  // dynamic part, beside the static arrays

// Weight unit = 256 elements of a row: one Q4_K / Q6_K superblock or eight
// Q8_0 blocks.  NPU 16-byte planes per unit, DPU separate f16 d values,
// activation sums per GRP elements (0: none).
template <int FMT>
struct KqfFmt;
template <>
struct KqfFmt<SYN_HIP_FMT_Q4_K> {
  static constexpr int BPU = 1, NPB = 9, NPU = 9, DPU = 0, GRP = 32;
};
template <>
struct KqfFmt<SYN_HIP_FMT_Q6_K> {
  static constexpr int BPU = 1, NPB = 13, NPU = 13, DPU = 1, GRP = 16;
};
template <>
struct KqfFmt<SYN_HIP_FMT_Q8_0> {
  static constexpr int BPU = 8, NPB = 2, NPU = 16, DPU = 8, GRP = 0;
};
template <>  // eight 32-element blocks, one nibble plane each; sums per block
struct KqfFmt<SYN_HIP_FMT_Q4_0> {
  static constexpr int BPU = 8, NPB = 1, NPU = 8, DPU = 8, GRP = 32;
};

int groups_per_unit(int fmt) {
  return fmt == SYN_HIP_FMT_Q4_K || fmt == SYN_HIP_FMT_Q4_0 ? 8
         : fmt == SYN_HIP_FMT_Q6_K                          ? 16
                                                            : 0;
}

enum { OUT_ACC = 0, OUT_GU = 1, OUT_TOP2 = 2 };

struct KqfOut {
  long long *acc = nullptr;  // ACC: fixed-point accumulator of the rows
  long long *zero = nullptr;  // cleared first: zero[0 .. nzero)
  int nzero = 0;
  float *y = nullptr;  // GU: h; TOP2: logits
  int inter = 0;       // GU: gate rows (the up rows follow)
  float *pv = nullptr;
  int *pi = nullptr;
  float *pv2 = nullptr;
};

// Lane moves within a row of 16 lanes (DPP, no LDS traffic): xor 1, xor 2,
// mirror within 8 (quad i <-> quad 1-i), mirror within 16.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// sum (max) over groups of N lanes (N = 4, 8, 16), in every lane of the group
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_mov<kDppXor1>(v);
  if (N > 2) v += dpp_mov<kDppXor2>(v);
  if (N > 4) v += dpp_mov<kDppHalfMirror>(v);
  if (N > 8) v += dpp_mov<kDppMirror>(v);
  return v;
}
template <int N>
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, dpp_mov<kDppXor1>(v));
  if (N > 2) v = fmaxf(v, dpp_mov<kDppXor2>(v));
  if (N > 4) v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
  if (N > 8) v = fmaxf(v, dpp_mov<kDppMirror>(v));
  return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// over the 64 lanes, wave-uniform result (rows of 16, then four readlanes)
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = group_max<16>(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

typedef long long i64x2 __attribute__((ext_vector_type(2)));

// 32 activations of a stage from LDS (all lanes read the same address)
__device__ __forceinline__ void lds_x32(float (&x)[32], const float *src) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 v = reinterpret_cast<const float4 *>(src)[i];
    x[4 * i] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
}

__device__ __forceinline__ void pin_plane(const u32x4 &v) {
  u32x4 &w = const_cast<u32x4 &>(v);
  asm volatile("" : "+v"(w));
}

// One 256-element unit in eight stages of 32 activations (or stages
// [T0, T0 + NS) of it, for a wave that takes part of a unit): with DB the
// activations of stage t+1 are read from LDS before stage t's FMAs (two
// register buffers), else each stage reads its own (one buffer, for
// workgroups of 16 waves whose register budget is 128; other waves hide the
// LDS latency).  The scheduling barriers keep the compiler from hoisting all
// 256 reads.
template <int FMT, bool DB, int T0 = 0, int NS = 8>
__device__ __forceinline__ void kqf_unit(u32x4 *pl, const uint16_t *dh, const float *xs,
                                         const float *as, float &acc) {
  asm volatile("" ::: "memory");  // no LDS read of the unit moves above its branch
  float xb[DB ? 2 : 1][32];
  float av[16];
  if constexpr (FMT == SYN_HIP_FMT_Q4_K || FMT == SYN_HIP_FMT_Q4_0) {
#pragma unroll
    for (int i = 0; i < 8; i++) av[i] = as[i];
  } else if constexpr (FMT == SYN_HIP_FMT_Q6_K) {
#pragma unroll
    for (int i = 0; i < 16; i++) av[i] = as[i];
  }
  // block scales first: their conversion branches would otherwise split the
  // stages into blocks that the compiler reorders as a whole
  float d = 0.0f, dmin = 0.0f, dq[8];
  if constexpr (FMT == SYN_HIP_FMT_Q4_K) {
    d = syn_f16_to_f32_rs(pl[0].x & 0xffffu);
    dmin = syn_f16_to_f32_rs(pl[0].x >> 16);
  } else if constexpr (FMT == SYN_HIP_FMT_Q6_K) {
    d = syn_f16_to_f32_rs(dh[0]);
  } else if constexpr (FMT == SYN_HIP_FMT_Q4_0) {
    // IEEE f16 scales (the Q4 GEMV's reading; handles with halved subnormal
    // scales are not offered to this kernel), pinned here so the conversion
    // (and the wait for the loads) is not hoisted into the entry's branch
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t h = dh[j];
      asm volatile("" : "+v"(h));
      dq[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) dq[j] = syn_f16_to_f32_rs(dh[j]);
  }
  if constexpr (DB) lds_x32(xb[T0 & 1], xs + T0 * 32);
#pragma unroll
  for (int t = T0; t < T0 + NS; t++) {
    if constexpr (DB) {
      if (t + 1 < T0 + NS) lds_x32(xb[(t + 1) & 1], xs + (t + 1) * 32);
    } else {
      lds_x32(xb[0], xs + t * 32);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the stage's weight planes become visible here, so their decode is not
    // hoisted into earlier stages
    if constexpr (FMT == SYN_HIP_FMT_Q4_K) {
      pin_plane(pl[1 + t]);
    } else if constexpr (FMT == SYN_HIP_FMT_Q6_K) {
      pin_plane(pl[t]);
      pin_plane(pl[8 + (t >> 1)]);
    } else if constexpr (FMT == SYN_HIP_FMT_Q4_0) {
      pin_plane(pl[t]);
    } else {
      pin_plane(pl[2 * t]);
      pin_plane(pl[2 * t + 1]);
    }
    const float *xc = xb[DB ? (t & 1) : 0];
    if constexpr (FMT == SYN_HIP_FMT_Q4_K) {
      kq4_stage(pl, t, d, dmin, xc, av[t], acc);
    } else if constexpr (FMT == SYN_HIP_FMT_Q6_K) {
      kq6_group(pl, 2 * t, d, xc, av[2 * t], acc);
      kq6_group(pl, 2 * t + 1, d, xc + 16, av[2 * t + 1], acc);
    } else if constexpr (FMT == SYN_HIP_FMT_Q4_0) {
      kq40_block(pl[t], dq[t], xc, av[t], acc);
    } else {
      kq8_block(pl, t, dq[t], xc, acc);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Part of a Q4_0 unit for workgroups that give each unit WPU waves (2 or 4):
// NB = 8 / WPU 32-element blocks, the part's planes and scales in pl / dh,
// its activations and block sums in xs / as.
template <bool DB, int NB>
__device__ __forceinline__ void kqf_q40_part(u32x4 *pl, const uint16_t *dh, const float *xs,
                                             const float *as, float &acc) {
  asm volatile("" ::: "memory");  // no LDS read of the part moves above its branch
  float xb[DB ? 2 : 1][32];
  float av[NB], dq[NB];
#pragma unroll
  for (int i = 0; i < NB; i++) av[i] = as[i];
#pragma unroll
  for (int j = 0; j < NB; j++) {  // IEEE f16 scales, converted after the prologue
    uint32_t h = dh[j];
    asm volatile("" : "+v"(h));
    dq[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  if constexpr (DB) lds_x32(xb[0], xs);
#pragma unroll
  for (int t = 0; t < NB; t++) {
    if constexpr (DB) {
      if (t + 1 < NB) lds_x32(xb[(t + 1) & 1], xs + (t + 1) * 32);
    } else {
      lds_x32(xb[0], xs + t * 32);
    }
    __builtin_amdgcn_sched_barrier(0);
    pin_plane(pl[t]);
    kq40_block(pl[t], dq[t], xb[DB ? (t & 1) : 0], av[t], acc);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ------------------------------------------------------------------ GEMV
// grid (row groups, K splits), NW waves (NW >= bs).  Row group = a 64-row
// panel (lane = row), or for OUT_GU 32 gate rows j.. and the 32 up rows
// inter+j.. in lanes 32..63 (two 512-byte halves of a plane load).  Split s
// covers the units [s*bs, s*bs + bs), one per wave (or WPU waves per unit,
// each a part of its stages), all requested at entry.
// Prologue threads hold 4 consecutive elements per round, so an activation
// group (32 elements for Q4_K, 16 for Q6_K) is summed across 8 or 4 lanes.
// dynamic LDS: activation slice [bs*256] | group sums [bs*256/GRP] |
// (ATTN) chunk logits and weights [2][heads of the slice][nch], 1/den [heads]
template <int FMT, int PRO, int OUT, int NW, int WPU>
__global__ void __launch_bounds__(NW * 64)
    k_kqf_gemv(const u32x4 *__restrict__ W, const uint16_t *__restrict__ Wd, int B, int N,
               int bs, KqfIn in, KqfOut out) {
  static_assert(WPU == 1 || FMT == SYN_HIP_FMT_Q4_0 ||
                    ((FMT == SYN_HIP_FMT_Q4_K || FMT == SYN_HIP_FMT_Q6_K) && OUT == OUT_ACC),
                "split units: Q4_0, or Q4_K / Q6_K into the split-K accumulator");
  constexpr int NBP = 8 / WPU;  // Q4_0 blocks per wave when WPU > 1
  using F = KqfFmt<FMT>;
  constexpr int kNT = NW * 64;
  constexpr int GPU = F::GRP ? 256 / F::GRP : 0;
  constexpr int LPG = F::GRP ? F::GRP / 4 : 1;
  SYN_TS_DECL
  SYN_TSR(14);
  SYN_TS(0);
  extern __shared__ __align__(16) float xs[];
  __shared__ float red[NW * 64];
  __shared__ float ssr[NW];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nU = B / F::BPU;
  const int u0 = blockIdx.y * bs, nu_wg = min(nU, u0 + bs) - u0;
  const int k0 = u0 * 256, nk = nu_wg * 256;
  float *as = xs + bs * 256;
  float4 *xs4 = reinterpret_cast<float4 *>(xs);
  int row;
  if constexpr (OUT == OUT_GU) {
    const int j = blockIdx.x * 32 + (lane & 31);
    row = lane < 32 ? j : out.inter + j;
  } else {
    row = blockIdx.x * 64 + lane;
  }
  const u32x4 *Wl = W + (size_t)(row >> 6) * B * F::NPB * 64 + (row & 63);
  const uint16_t *Wdl = Wd + (size_t)(row >> 6) * B * 64 + (row & 63);

  // 2. this wave's unit in flight: Q4_0 (8 planes) requests it at entry, so
  // the prologue runs under the weights' HBM latency; the K-quant formats
  // (up to 16 planes) after the prologue
  constexpr bool kEarlyW = FMT == SYN_HIP_FMT_Q4_0;
  // WPU waves per unit: wave w takes part w % WPU of unit w / WPU
  const int uw = wave / WPU, uh = wave % WPU;
  const bool has_unit = uw < nu_wg;
  u32x4 buf[F::NPU];
  uint16_t dbuf[F::DPU > 0 ? F::DPU : 1];
  // Q4_K / Q6_K parts: stages [T0, T0 + 8 / WPU) of the unit, with only the
  // planes those stages read (Q4_K: plane 0 and the stages' sub-block
  // planes; Q6_K: the stages' ql planes, their qh planes, the scale plane
  // and d), requested right before they are decoded
  constexpr bool kKqPart = WPU > 1 && FMT != SYN_HIP_FMT_Q4_0;
  auto kq_part = [&](auto T0c, float &a) {
    constexpr int T0 = decltype(T0c)::value;
    const int u = u0 + uw;
    const u32x4 *src = Wl + (size_t)u * F::NPB * 64;
    if constexpr (FMT == SYN_HIP_FMT_Q4_K) {
      buf[0] = __builtin_nontemporal_load(src);
#pragma unroll
      for (int t = T0; t < T0 + NBP; t++) buf[1 + t] = __builtin_nontemporal_load(src + (1 + t) * 64);
    } else if constexpr (FMT == SYN_HIP_FMT_Q6_K) {
#pragma unroll
      for (int t = T0; t < T0 + NBP; t++) {
        buf[t] = __builtin_nontemporal_load(src + t * 64);
        if (t == T0 || (t & 1) == 0)
          buf[8 + (t >> 1)] = __builtin_nontemporal_load(src + (8 + (t >> 1)) * 64);
      }
      buf[12] = __builtin_nontemporal_load(src + 12 * 64);
      dbuf[0] = __builtin_nontemporal_load(Wdl + (size_t)u * 64);
    }
    kqf_unit<FMT, (NW < 16), T0, NBP>(buf, dbuf, xs + uw * 256, as + uw * GPU, a);
  };
  auto issue_unit = [&]() {
    if (kKqPart) return;
    if (has_unit) {
      const int u = u0 + uw;
      const u32x4 *src = Wl + (size_t)u * F::BPU * F::NPB * 64;
      if constexpr (WPU > 1) {
#pragma unroll
        for (int p = 0; p < NBP; p++)
          buf[p] = __builtin_nontemporal_load(src + (NBP * uh + p) * 64);
#pragma unroll
        for (int j = 0; j < NBP; j++)
          dbuf[j] = __builtin_nontemporal_load(Wdl + ((size_t)u * F::BPU + NBP * uh + j) * 64);
      } else {
#pragma unroll
        for (int p = 0; p < F::NPU; p++) buf[p] = __builtin_nontemporal_load(src + p * 64);
#pragma unroll
        for (int j = 0; j < F::DPU; j++)
          dbuf[j] = __builtin_nontemporal_load(Wdl + ((size_t)u * F::BPU + j) * 64);
      }
    }
  };
  auto compute_unit = [&](float &a) {
    if constexpr (kKqPart && WPU == 2) {
      if (uh == 0) kq_part(std::integral_constant<int, 0>{}, a);
      else kq_part(std::integral_constant<int, 4>{}, a);
    } else if constexpr (kKqPart) {
      if (uh == 0) kq_part(std::integral_constant<int, 0>{}, a);
      else if (uh == 1) kq_part(std::integral_constant<int, 2>{}, a);
      else if (uh == 2) kq_part(std::integral_constant<int, 4>{}, a);
      else kq_part(std::integral_constant<int, 6>{}, a);
    } else if constexpr (WPU > 1)
      kqf_q40_part<(NW < 16), NBP>(buf, dbuf, xs + uw * 256 + uh * (256 / WPU),
                                   as + uw * GPU + uh * NBP, a);
    else
      kqf_unit<FMT, (NW < 16)>(buf, dbuf, xs + wave * 256, as + wave * GPU, a);
  };
  if constexpr (kEarlyW) issue_unit();
  asm volatile("" ::: "memory");

  // 1. the prologue's loads, ahead of the weights
  const int H4 = in.H >> 2;
  i64x2 rl[kRounds][2];  // NORM: the residual row, fixed point
  float4 el[kRounds];    // EMBED: the embedding row; NONE: the slice
  float4 gl[kRounds];    // NORM / EMBED: gains of the slice
  const float *erow = nullptr;
  int pos = 0, nl = 0;
  float2 ml0 = make_float2(-__builtin_inff(), 0.0f);  // ATTN: (m, l) of chunk `lane`
  float4 ob0[8];                                     // ATTN: first 8 chunks of this thread
  if constexpr (PRO == KQF_PRO_NORM || PRO == KQF_PRO_EMBED) {
    if constexpr (PRO == KQF_PRO_EMBED) {
      const uint32_t tok = in.st->token;
      erow = tok < (uint32_t)in.vocab ? in.embed + (size_t)tok * in.H : nullptr;
    }
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int i = tid + r * kNT;
      if (i < H4) {
        if constexpr (PRO == KQF_PRO_NORM) {
          rl[r][0] = reinterpret_cast<const i64x2 *>(in.r)[2 * i];
          rl[r][1] = reinterpret_cast<const i64x2 *>(in.r)[2 * i + 1];
        } else {
          el[r] = erow ? reinterpret_cast<const float4 *>(erow)[i] : make_float4(0, 0, 0, 0);
        }
        const int kk = 4 * i - k0;
        if (kk >= 0 && kk < nk) gl[r] = reinterpret_cast<const float4 *>(in.gain)[i];
      }
    }
  } else if constexpr (PRO == KQF_PRO_NONE) {
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int i = tid + r * kNT;
      if (i < nk / 4) el[r] = reinterpret_cast<const float4 *>(in.x + k0)[i];
    }
  } else if constexpr (PRO == KQF_PRO_ATTN) {
    // the first chunks' partials are read before the position is known
    // (chunk indices clamped in bounds; chunks past the position are masked)
    const int hd = in.hd, hs = __builtin_ctz(hd), h0 = k0 >> hs, nhs = nk >> hs;
    if (wave < nhs)
      ml0 = reinterpret_cast<const float2 *>(in.aml)[(size_t)(h0 + wave) * in.nch +
                                                     min(lane, in.nch - 1)];
    if (tid < nk / 4) {
      const int hl = (4 * tid) >> hs, d = 4 * tid - (hl << hs);
      const float4 *o = reinterpret_cast<const float4 *>(in.ao + ((size_t)(h0 + hl) * in.nch) * hd + d);
#pragma unroll
      for (int c = 0; c < 8; c++) ob0[c] = o[(size_t)min(c, in.nch - 1) * (hd / 4)];
    }
    pos = in.st->pos;
    nl = pos / 64 + 1;  // chunks holding live positions
    SYN_TS(8);
  }
  asm volatile("" ::: "memory");
  // 3. the activation slice [k0, k0 + nk) and its group sums
  auto put = [&](int i, float4 v) {  // slice float4 i (wave-uniform validity)
    xs4[i] = v;
    if constexpr (GPU > 0) {
      const float gs = group_sum<LPG>((v.x + v.y) + (v.z + v.w));
      if ((lane & (LPG - 1)) == LPG - 1) as[(4 * i) / F::GRP] = gs;
    }
  };
  if constexpr (PRO == KQF_PRO_NORM || PRO == KQF_PRO_EMBED) {
    const bool wr = PRO == KQF_PRO_EMBED && in.r_out && blockIdx.x == 0 && blockIdx.y == 0;
    float ss = 0.0f;
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int i = tid + r * kNT;
      if (i < H4) {  // H4 is a multiple of 64: wave-uniform
        float4 a;
        if constexpr (PRO == KQF_PRO_NORM) {
          a = make_float4(kqf_unfix(rl[r][0].x), kqf_unfix(rl[r][0].y), kqf_unfix(rl[r][1].x),
                          kqf_unfix(rl[r][1].y));
        } else {
          a = el[r];
          if (wr) {
            i64x2 *ro = reinterpret_cast<i64x2 *>(in.r_out);
            ro[2 * i] = i64x2{kqf_fix(a.x), kqf_fix(a.y)};
            ro[2 * i + 1] = i64x2{kqf_fix(a.z), kqf_fix(a.w)};
          }
        }
        ss += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
        const int kk = 4 * i - k0;
        if (kk >= 0 && kk < nk) {  // slice bounds are multiples of 256: wave-uniform
          const float4 g = gl[r];
          put(kk >> 2, make_float4(a.x * g.x, a.y * g.y, a.z * g.z, a.w * g.w));
        }
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) ssr[wave] = ss;
  } else if constexpr (PRO == KQF_PRO_NONE) {
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int i = tid + r * kNT;
      if (i < nk / 4) put(i, el[r]);
    }
  } else if constexpr (PRO == KQF_PRO_CONV) {
    // the slice's channels; row group 0 writes their next state half
    const int cpos = in.st->pos, inner = in.inner, ck = in.ck;
    const size_t half = (size_t)inner * ck;
    const float *sold = in.cstate + (size_t)(cpos & 1) * half;
    float *snew = blockIdx.x == 0 ? in.cstate + (size_t)((cpos + 1) & 1) * half : nullptr;
    for (int t = tid; t < nk; t += kNT) {  // one channel per thread
      const int ch = k0 + t;
      xs[t] = liv_conv_channel(kqf_unfix(in.cacc[ch]), kqf_unfix(in.cacc[inner + ch]),
                               kqf_unfix(in.cacc[2 * inner + ch]), ck, sold + (size_t)ch * ck,
                               snew ? snew + (size_t)ch * ck : nullptr, in.cw + (size_t)ch * ck,
                               in.cb ? in.cb + ch : nullptr);
    }
    __syncthreads();
    for (int i = tid; i < nk / 4; i += kNT) put(i, xs4[i]);  // nk / 4: a multiple of 64
  } else {  // x = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c
    const int hd = in.hd, hs = __builtin_ctz(hd), h0 = k0 >> hs, nhs = nk >> hs, nch = in.nch;
    float *cm = as + bs * GPU;  // [nhs][nch] chunk maxima, then weights
    float *cl = cm + nhs * nch;  // [nhs][nch] chunk sums
    float *inv = cl + nhs * nch;  // [nhs]
    for (int hl = wave; hl < nhs; hl += NW) {
      const float2 *ml = reinterpret_cast<const float2 *>(in.aml) + (size_t)(h0 + hl) * nch;
      float M = -__builtin_inff();
      // the first 64 chunks of the wave's first head come from the entry loads
      for (int c0 = hl == wave ? 64 : 0; c0 < nl; c0 += 64) {
        const int c = c0 + lane;
        float2 v = make_float2(-__builtin_inff(), 0.0f);
        if (c < nl) {
          v = ml[c];
          cm[hl * nch + c] = v.x;
          cl[hl * nch + c] = v.y;
        }
        M = fmaxf(M, wave_max(v.x));
      }
      if (hl == wave) {
        const float2 v = lane < nl ? ml0 : make_float2(-__builtin_inff(), 0.0f);
        if (lane < nl) {
          cm[hl * nch + lane] = v.x;
          cl[hl * nch + lane] = v.y;
        }
        M = fmaxf(M, wave_max(v.x));
        SYN_TS(12);
      }
      float den = 0.0f;
      for (int c0 = 0; c0 < nl; c0 += 64) {
        const int c = c0 + lane;
        float e = 0.0f, l = 0.0f;
        if (c < nl) {
          e = __expf(cm[hl * nch + c] - M);
          l = cl[hl * nch + c];
          cm[hl * nch + c] = e;
        }
        den += wave_sum(e * l);
      }
      if (lane == 0) inv[hl] = 1.0f / den;
    }
    SYN_TS(9);
    __syncthreads();
    SYN_TS(10);
    // thread float4 i: 4 elements of head hl.  The first batch of the first
    // float4 comes from the registers loaded at entry.  Chunks past the
    // position are never multiplied in (their partials are stale or unwritten).
    auto combine = [&](int i, float4 a, int c0) {
      const int hl = (4 * i) >> hs, d = 4 * i - (hl << hs);
      const float *w = cm + hl * nch;
      const float4 *o = reinterpret_cast<const float4 *>(in.ao + ((size_t)(h0 + hl) * nch) * hd + d);
      for (; c0 < nl; c0 += 8) {
        float4 ob[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
          ob[j] = c0 + j < nl ? o[(size_t)(c0 + j) * (hd / 4)] : make_float4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float wc = c0 + j < nl ? w[c0 + j] : 0.0f;
          a.x = __builtin_fmaf(wc, ob[j].x, a.x);
          a.y = __builtin_fmaf(wc, ob[j].y, a.y);
          a.z = __builtin_fmaf(wc, ob[j].z, a.z);
          a.w = __builtin_fmaf(wc, ob[j].w, a.w);
        }
      }
      const float iv = inv[hl];
      put(i, make_float4(a.x * iv, a.y * iv, a.z * iv, a.w * iv));
    };
    if (tid < nk / 4) {  // nk/4 is a multiple of 64: wave-uniform
      const int hl = (4 * tid) >> hs;
      const float *w = cm + hl * nch;
      float4 a = make_float4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float wc = j < nl ? w[j] : 0.0f;
        const float4 ob = j < nl ? ob0[j] : make_float4(0, 0, 0, 0);
        a.x = __builtin_fmaf(wc, ob.x, a.x);
        a.y = __builtin_fmaf(wc, ob.y, a.y);
        a.z = __builtin_fmaf(wc, ob.z, a.z);
        a.w = __builtin_fmaf(wc, ob.w, a.w);
      }
      combine(tid, a, 8);
    }
    for (int i = tid + kNT; i < nk / 4; i += kNT) combine(i, make_float4(0, 0, 0, 0), 0);
    SYN_TS(11);
  }
  SYN_TS(2);
  __syncthreads();
  SYN_TS(3);
  if constexpr (!kEarlyW) issue_unit();
  asm volatile("" ::: "memory");
  SYN_TS(1);


  SYN_TS(4);

  // 4. the unit
  float acc = 0.0f;
  if (has_unit) compute_unit(acc);
  SYN_TS(5);

  if constexpr (OUT == OUT_TOP2) {
    // lm_head (no K split): the workgroup takes the 64-row panels blockIdx.x,
    // + gridDim.x, ... after one prologue; each wave requests its unit of the
    // next panel before the current panel's reduction
    const int np = (N + 63) >> 6;
    float inv = 1.0f;
    if constexpr (PRO == KQF_PRO_NORM || PRO == KQF_PRO_EMBED) {
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; w++) t += ssr[w];
      inv = 1.0f / sqrtf(t / (float)in.H + in.eps);
    }
    Top2v best{-__builtin_inff(), -1, -__builtin_inff()};
    for (int g = blockIdx.x; g < np; g += gridDim.x) {
      red[wave * 64 + lane] = acc;
      const int gn = g + gridDim.x;
      if (gn < np) {
        Wl = W + (size_t)gn * B * F::NPB * 64 + lane;
        Wdl = Wd + (size_t)gn * B * 64 + lane;
        issue_unit();
      }
      __syncthreads();
      if (wave == 0) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) v += red[w * 64 + lane];
        v *= inv;
        const int r = g * 64 + lane;
        Top2v c{-__builtin_inff(), -1, -__builtin_inff()};
        if (r < N) {
          out.y[r] = v;
          c = Top2v{v, r, -__builtin_inff()};
        }
        best = top2v_merge(best, wave_top2(c));
      }
      __syncthreads();  // red is written again for the next panel
      if (gn < np) {
        acc = 0.0f;
        if (has_unit) compute_unit(acc);
      }
    }
    if (wave == 0 && lane == 0) {
      out.pv[blockIdx.x] = best.v1;
      out.pi[blockIdx.x] = best.i1;
      out.pv2[blockIdx.x] = best.v2;
    }
    return;
  }

  // 5. epilogue: waves in order, then the row's consumer form
  red[wave * 64 + lane] = acc;
  __syncthreads();
  SYN_TS(6);
  if (out.zero) {  // clear the next consumer's accumulator (its readers have
                   // finished); last, so no load of this kernel waits on the stores
    const int nthr = gridDim.x * gridDim.y * kNT;
    for (int i = (blockIdx.y * gridDim.x + blockIdx.x) * kNT + tid; i < out.nzero; i += nthr)
      out.zero[i] = 0;
  }
  if (wave != 0) return;
  float v = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; w++) v += red[w * 64 + lane];
  if constexpr (PRO == KQF_PRO_NORM || PRO == KQF_PRO_EMBED) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) t += ssr[w];
    v *= 1.0f / sqrtf(t / (float)in.H + in.eps);
  }
  if constexpr (OUT == OUT_ACC) {
    if (row < N)
      atomicAdd(reinterpret_cast<unsigned long long *>(out.acc) + row,
                (unsigned long long)kqf_fix(v));
  } else if constexpr (OUT == OUT_GU) {
    const float up = __shfl_xor(v, 32);
    if (lane < 32) {
      const float sig = 1.0f / (1.0f + syn_expf(-v));  // silu as k_swiglu_f32
      const float t = v * sig;
      out.y[blockIdx.x * 32 + lane] = t * up;
    }
  }
  SYN_TS(7);
  SYN_TSR(15);
  SYN_TS_FLUSH_TO(kqf_phase_ts, (OUT == OUT_GU ? 32 : OUT == OUT_TOP2 ? 64
                                 : PRO == KQF_PRO_ATTN ? 16 : PRO == KQF_PRO_NONE ? 48 : 0));
}

// ------------------------------------------------------------------ attention
// grid (n_kv, chunks of 64 positions), 256 threads; chunks past the token's
// position exit at once.  The K tile of the chunk is one 64-position tile of
// the cache (lane = position, wave = a quarter of the d-quads); V is read as
// position quads (thread = output column d, TPD position groups).
template <int HD>
__global__ void __launch_bounds__(256)
    k_kqf_attn(const long long *__restrict__ qkv, int nh, int nkv, const float *__restrict__ qn,
               const float *__restrict__ kn, float eps, const float *__restrict__ cosT,
               const float *__restrict__ sinT, const StepState *__restrict__ st,
               float *__restrict__ kc, float *__restrict__ vc, int S, float *__restrict__ ao,
               float *__restrict__ aml, int nch) {
  constexpr int HD4 = HD / 4, DW = HD4 / 4, TPD = 256 / HD, QPT = 16 / TPD, HALF = HD / 2;
  constexpr int NQ = ((kGmax + 2) * HD + 255) / 256;  // q/k/v values per thread
  SYN_TS_DECL
  SYN_TSR(14);
  SYN_TS(0);
  __shared__ __align__(16) float raw[(kGmax + 2) * HD];
  __shared__ float red_s[4 * kGmax * 64];
  __shared__ float esm[kGmax * 64];
  __shared__ float pvr[kGmax * 256];
  const int g = blockIdx.x, c = blockIdx.y;
  const int p0 = c * 64;
  const int G = nh / nkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int tiles = (S + 63) >> 6, s4 = (S + 3) >> 2;
  const int qd = nh * HD, kvd = nkv * HD, n3 = (G + 2) * HD;
  // 1. the new token's q (G heads), k and v, and its RoPE row
  long long qv[NQ];
#pragma unroll
  for (int j = 0; j < NQ; j++) {
    const int i = tid + j * 256;
    if (i < n3) {
      const int hh = i / HD, dd = i - hh * HD;
      const int col = hh < G ? (g * G + hh) * HD + dd
                             : (hh == G ? qd + g * HD + dd : qd + kvd + g * HD + dd);
      qv[j] = qkv[col];
    }
  }
  // 2. cached K and V of the chunk in flight before the position is known
  // (quads clamped in bounds; positions past pos are masked below)
  const float4 *Kt = reinterpret_cast<const float4 *>(kc) + (size_t)(g * tiles + c) * HD4 * 64;
  float4 kr[DW];
#pragma unroll
  for (int j = 0; j < DW; j++) kr[j] = Kt[(wave * DW + j) * 64 + lane];
  const int d = tid % HD, grp = tid / HD;
  const float4 *Vt = reinterpret_cast<const float4 *>(vc) + (size_t)g * s4 * HD + d;
  float4 vr[QPT];
#pragma unroll
  for (int j = 0; j < QPT; j++)
    vr[j] = Vt[(size_t)min(c * 16 + grp * QPT + j, s4 - 1) * HD];
  const int pos = st->pos;
  if (p0 > pos) return;
  // positions past pos (stale cache rows) are zeroed, not multiplied by 0
#pragma unroll
  for (int j = 0; j < QPT; j++) {
    const int p = p0 + 4 * (grp * QPT + j);
    vr[j].x = p <= pos ? vr[j].x : 0.0f;
    vr[j].y = p + 1 <= pos ? vr[j].y : 0.0f;
    vr[j].z = p + 2 <= pos ? vr[j].z : 0.0f;
    vr[j].w = p + 3 <= pos ? vr[j].w : 0.0f;
  }
  float cs = 0.0f, sn = 0.0f;
  if (lane < HALF) {
    cs = cosT[(size_t)pos * HALF + lane];
    sn = sinT[(size_t)pos * HALF + lane];
  }
#pragma unroll
  for (int j = 0; j < NQ; j++) {
    const int i = tid + j * 256;
    if (i < n3) raw[i] = kqf_unfix(qv[j]);
  }
  SYN_TS(1);
  __syncthreads();
  SYN_TS(2);
  // 3. head RMSNorm (norm.rs:78-93) and rotate-half RoPE (rope.rs:13-43) of
  // the q heads and the k head, one wave per head
  for (int hh = wave; hh <= G; hh += 4) {
    float *r = raw + hh * HD;
    float x1 = 0.0f, x2 = 0.0f;
    if (lane < HALF) {
      x1 = r[lane];
      x2 = r[lane + HALF];
    }
    const float *wn = hh < G ? qn : kn;
    if (wn) {
      const float ss = wave_sum(x1 * x1 + x2 * x2);
      const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
      if (lane < HALF) {
        x1 = (x1 * wn[lane]) * sc;
        x2 = (x2 * wn[lane + HALF]) * sc;
      }
    }
    if (lane < HALF) {
      r[lane] = x1 * cs - x2 * sn;
      r[lane + HALF] = x2 * cs + x1 * sn;
    }
  }
  __syncthreads();
  SYN_TS(3);
  const float *knew = raw + G * HD, *vnew = raw + (G + 1) * HD;
  const int pl = pos - p0;  // < 64: this chunk holds the new position
  // 4. KV append (the only writer of cache row pos in this step)
  if (pl < 64)
    for (int i = tid; i < HD; i += 256) {
      kc[kv_k_index(pos, g, i, HD, S)] = knew[i];
      vc[kv_v_index(pos, g, i, HD, S)] = vnew[i];
    }
  // 5. scores over this wave's d-quads; the new position from LDS
  if (lane == pl) {
#pragma unroll
    for (int j = 0; j < DW; j++) kr[j] = reinterpret_cast<const float4 *>(knew)[wave * DW + j];
  }
#pragma unroll
  for (int gi = 0; gi < kGmax; gi++) {
    if (gi < G) {
      const float4 *q4 = reinterpret_cast<const float4 *>(raw + gi * HD) + wave * DW;
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < DW; j++) {
        const float4 q = q4[j];
        s = __builtin_fmaf(q.x, kr[j].x, s);
        s = __builtin_fmaf(q.y, kr[j].y, s);
        s = __builtin_fmaf(q.z, kr[j].z, s);
        s = __builtin_fmaf(q.w, kr[j].w, s);
      }
      red_s[(wave * kGmax + gi) * 64 + lane] = s;
    }
  }
  __syncthreads();
  SYN_TS(4);
  // 6. chunk softmax of each query head (one wave per head)
  const float scale = 1.0f / sqrtf((float)HD);
  for (int gi = wave; gi < G; gi += 4) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) s += red_s[(w * kGmax + gi) * 64 + lane];
    const bool live = lane <= pl;
    s = live ? s * scale : -__builtin_inff();
    const float m = wave_max(s);
    const float e = live ? __expf(s - m) : 0.0f;
    const float l = wave_sum(e);
    esm[gi * 64 + lane] = e;
    if (lane == 0) {
      float *ml = aml + ((size_t)(g * G + gi) * nch + c) * 2;
      ml[0] = m;
      ml[1] = l;
    }
  }
  __syncthreads();
  SYN_TS(5);
  // 7. P.V over this thread's position quads; the new position from LDS
#pragma unroll
  for (int j = 0; j < QPT; j++) {
    const int q = grp * QPT + j;
    if (q == (pl >> 2) && pl < 64) {
      const float vn = vnew[d];
      const int t = pl & 3;
      vr[j].x = t == 0 ? vn : vr[j].x;
      vr[j].y = t == 1 ? vn : vr[j].y;
      vr[j].z = t == 2 ? vn : vr[j].z;
      vr[j].w = t == 3 ? vn : vr[j].w;
    }
  }
#pragma unroll
  for (int gi = 0; gi < kGmax; gi++) {
    if (gi < G) {
      const float *e = esm + gi * 64 + grp * QPT * 4;
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < QPT; j++) {
        a = __builtin_fmaf(e[4 * j], vr[j].x, a);
        a = __builtin_fmaf(e[4 * j + 1], vr[j].y, a);
        a = __builtin_fmaf(e[4 * j + 2], vr[j].z, a);
        a = __builtin_fmaf(e[4 * j + 3], vr[j].w, a);
      }
      pvr[(gi * TPD + grp) * HD + d] = a;
    }
  }
  __syncthreads();
  SYN_TS(6);
  for (int i = tid; i < G * HD; i += 256) {
    const int gi = i / HD, dd = i - gi * HD;
    float o = 0.0f;
#pragma unroll
    for (int t = 0; t < TPD; t++) o += pvr[(gi * TPD + t) * HD + dd];
    ao[((size_t)(g * G + gi) * nch + c) * HD + dd] = o;
  }
  SYN_TS(7);
  SYN_TSR(15);
  SYN_TS_FLUSH_TO(kqf_phase_ts, 80);
}

template <int FMT, int PRO, int OUT, int WPU = 1>
void launch_nw(int nw, dim3 grid, size_t lds, hipStream_t s, const u32x4 *W, const uint16_t *Wd,
               int B, int N, int bs, const KqfIn &in, const KqfOut &o) {
  switch (nw) {
    case 4:
      SYN_LAUNCH((k_kqf_gemv<FMT, PRO, OUT, 4, WPU>), grid, dim3(256), lds, s, W, Wd, B, N, bs,
                 in, o);
      break;
    case 8:
      SYN_LAUNCH((k_kqf_gemv<FMT, PRO, OUT, 8, WPU>), grid, dim3(512), lds, s, W, Wd, B, N, bs,
                 in, o);
      break;
    case 12:
      SYN_LAUNCH((k_kqf_gemv<FMT, PRO, OUT, 12, WPU>), grid, dim3(768), lds, s, W, Wd, B, N, bs,
                 in, o);
      break;
    default:
      SYN_LAUNCH((k_kqf_gemv<FMT, PRO, OUT, 16, WPU>), grid, dim3(1024), lds, s, W, Wd, B, N, bs,
                 in, o);
      break;
  }
}

// waves per workgroup: one per unit of the split, rounded up to 4, 8, 12, 16
inline int waves_for(int bs) { return bs <= 4 ? 4 : bs <= 8 ? 8 : bs <= 12 ? 12 : 16; }

template <int PRO, int OUT>
syn_status_t launch_gemv(const KqfW &w, const KqfPlan &p, const KqfIn &in, const KqfOut &o,
                         hipStream_t s) {
  size_t lds = (size_t)p.bs * (256 + groups_per_unit(w.fmt)) * sizeof(float);
  if (PRO == KQF_PRO_ATTN) {
    const size_t nhs = (size_t)p.bs * 256 / in.hd;
    lds += (2 * nhs * in.nch + nhs) * sizeof(float);
  }
  if (lds > kLdsMax || p.ks < 1 || p.groups < 1 || p.bs > kMaxNW) {
    set_error("fused K-quant GEMV: launch shape exceeds the workgroup's LDS or waves");
    return SYN_ERR_INVALID_ARG;
  }
  const dim3 grid(p.groups, p.ks);
  const int nw = waves_for(p.bs);
  const u32x4 *W = static_cast<const u32x4 *>(w.wq);
  const uint16_t *Wd = static_cast<const uint16_t *>(w.wd);
  switch (w.fmt) {
    // Q4_K / Q6_K into the split-K accumulator: four (else two) waves per
    // unit while they fit the workgroup, each decoding a quarter (half) of
    // it, so the decode left after the last weights land is shorter
    // (LLaMA-3.2-3B step: 1.002-1.007 ms/token against 1.015 with two and
    // 1.051-1.055 with one; with four, splitting K towards 128, 300 or 400
    // workgroups instead of 200 measured 1.061, 1.155 and 1.094)
    case SYN_HIP_FMT_Q4_K:
      if constexpr (OUT == OUT_ACC) {
        if (4 * p.bs <= kMaxNW) {
          launch_nw<SYN_HIP_FMT_Q4_K, PRO, OUT, 4>(waves_for(4 * p.bs), grid, lds, s, W, Wd,
                                                   w.blocks, (int)w.n, p.bs, in, o);
          break;
        }
        if (2 * p.bs <= kMaxNW) {
          launch_nw<SYN_HIP_FMT_Q4_K, PRO, OUT, 2>(waves_for(2 * p.bs), grid, lds, s, W, Wd,
                                                   w.blocks, (int)w.n, p.bs, in, o);
          break;
        }
      }
      launch_nw<SYN_HIP_FMT_Q4_K, PRO, OUT>(nw, grid, lds, s, W, Wd, w.blocks, (int)w.n, p.bs, in,
                                            o);
      break;
    case SYN_HIP_FMT_Q6_K:
      if constexpr (OUT == OUT_ACC) {
        if (4 * p.bs <= kMaxNW) {
          launch_nw<SYN_HIP_FMT_Q6_K, PRO, OUT, 4>(waves_for(4 * p.bs), grid, lds, s, W, Wd,
                                                   w.blocks, (int)w.n, p.bs, in, o);
          break;
        }
        if (2 * p.bs <= kMaxNW) {
          launch_nw<SYN_HIP_FMT_Q6_K, PRO, OUT, 2>(waves_for(2 * p.bs), grid, lds, s, W, Wd,
                                                   w.blocks, (int)w.n, p.bs, in, o);
          break;
        }
      }
      launch_nw<SYN_HIP_FMT_Q6_K, PRO, OUT>(nw, grid, lds, s, W, Wd, w.blocks, (int)w.n, p.bs, in,
                                            o);
      break;
    case SYN_HIP_FMT_Q8_0:
      launch_nw<SYN_HIP_FMT_Q8_0, PRO, OUT>(nw, grid, lds, s, W, Wd, w.blocks, (int)w.n, p.bs, in,
                                            o);
      break;
    case SYN_HIP_FMT_Q4_0:
      // four or two waves per unit (a quarter or half of the decode per
      // wave) while they fit the workgroup
      if (4 * p.bs <= kMaxNW)
        launch_nw<SYN_HIP_FMT_Q4_0, PRO, OUT, 4>(waves_for(4 * p.bs), grid, lds, s, W, Wd,
                                                 w.blocks, (int)w.n, p.bs, in, o);
      else if (2 * p.bs <= kMaxNW)
        launch_nw<SYN_HIP_FMT_Q4_0, PRO, OUT, 2>(waves_for(2 * p.bs), grid, lds, s, W, Wd,
                                                 w.blocks, (int)w.n, p.bs, in, o);
      else
        launch_nw<SYN_HIP_FMT_Q4_0, PRO, OUT>(nw, grid, lds, s, W, Wd, w.blocks, (int)w.n, p.bs,
                                              in, o);
      break;
    default:
      set_error("fused K-quant GEMV: unsupported format");
      return SYN_ERR_INVALID_ARG;
  }
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace

KqfW::KqfW(const QLinearKQ &w)
    : fmt(w.fmt), n(w.n), k(w.k), blocks(w.blocks), wq(w.wq.p), wd(w.wd.p) {}
KqfW::KqfW(const QLinearQ4_0 &w)
    : fmt(SYN_HIP_FMT_Q4_0), n(w.n), k(w.k), blocks(w.blocks), wq(w.nib.p), wd(w.sc.p) {}

bool kqf_fits(int H, int qd, int inter, int nh, int nkv, int hd, int max_seq, const int *fmts,
              int nfmt) {
  for (int i = 0; i < nfmt; i++)
    if (fmts[i] != SYN_HIP_FMT_Q4_K && fmts[i] != SYN_HIP_FMT_Q6_K &&
        fmts[i] != SYN_HIP_FMT_Q8_0 && fmts[i] != SYN_HIP_FMT_Q4_0)
      return false;
  // whole 256-element units along every K; a norm row in kRounds float4 per
  // thread; the slice of a split-K GEMV without a norm in kRounds too
  if (H % 256 || qd % 256 || inter % 256 || H > kRounds * 4 * 256) return false;
  if (hd != 16 && hd != 32 && hd != 64 && hd != 128) return false;
  if (nkv <= 0 || nh % nkv || nh / nkv > kGmax || nh * hd != qd) return false;
  return max_seq >= 1;
}

KqfPlan kqf_plan(const KqfW &w, bool gu) {
  KqfPlan p;
  p.units = (int)(w.k / 256);
  if (gu) {  // the SwiGLU epilogue needs whole dot products: no K split
    p.groups = (int)(w.n / 64);
    p.bs = p.units;
    p.ks = 1;
    return p;
  }
  p.groups = (int)cdiv(w.n, (size_t)64);
  // split K until the grid covers the 256 CUs (about one workgroup each)
  // and a split has at most kMaxNW units (one per wave)
  int ks = 1;
  while (ks < p.units && (p.groups * ks < 200 || cdiv((size_t)p.units, (size_t)ks) > kMaxNW))
    ks++;
  p.bs = (int)cdiv((size_t)p.units, (size_t)ks);
  p.ks = (int)cdiv((size_t)p.units, (size_t)p.bs);
  return p;
}

syn_status_t kqf_gemv(const KqfW &w, const KqfPlan &p, int pro, const KqfIn &in,
                      long long *acc, long long *zero, int nzero, hipStream_t s) {
  KqfOut o;
  o.acc = acc;
  o.zero = zero;
  o.nzero = nzero;
  switch (pro) {
    case KQF_PRO_NORM: return launch_gemv<KQF_PRO_NORM, OUT_ACC>(w, p, in, o, s);
    case KQF_PRO_EMBED: return launch_gemv<KQF_PRO_EMBED, OUT_ACC>(w, p, in, o, s);
    case KQF_PRO_ATTN: return launch_gemv<KQF_PRO_ATTN, OUT_ACC>(w, p, in, o, s);
    case KQF_PRO_CONV: return launch_gemv<KQF_PRO_CONV, OUT_ACC>(w, p, in, o, s);
    default: return launch_gemv<KQF_PRO_NONE, OUT_ACC>(w, p, in, o, s);
  }
}

syn_status_t kqf_gate_up(const KqfW &w, const KqfPlan &p, const KqfIn &in, int inter,
                         float *h, hipStream_t s) {
  KqfOut o;
  o.y = h;
  o.inter = inter;
  return launch_gemv<KQF_PRO_NORM, OUT_GU>(w, p, in, o, s);
}

syn_status_t kqf_lm_head(const KqfW &w, const KqfPlan &p, const KqfIn &in, float *logits,
                         float *pv, int *pi, float *pv2, hipStream_t s) {
  KqfOut o;
  o.y = logits;
  o.pv = pv;
  o.pi = pi;
  o.pv2 = pv2;
  return launch_gemv<KQF_PRO_NORM, OUT_TOP2>(w, p, in, o, s);
}

syn_status_t kqf_attention(const long long *qkv, int nh, int nkv, int hd, const float *qn,
                           const float *kn, float eps, const float *cosT, const float *sinT,
                           const StepState *st, float *kc, float *vc, int max_seq, float *ao,
                           float *aml, hipStream_t s) {
  const int nch = kqf_chunks(max_seq);
  const dim3 grid(nkv, nch);
#define KQF_ATTN(HD_)                                                                      \
  SYN_LAUNCH((k_kqf_attn<HD_>), grid, dim3(256), 0, s, qkv, nh, nkv, qn, kn, eps, cosT, sinT, \
             st, kc, vc, max_seq, ao, aml, nch)
  switch (hd) {
    case 16: KQF_ATTN(16); break;
    case 32: KQF_ATTN(32); break;
    case 64: KQF_ATTN(64); break;
    case 128: KQF_ATTN(128); break;
    default:
      set_error("fused attention: head_dim must be 16, 32, 64 or 128");
      return SYN_ERR_INVALID_ARG;
  }
#undef KQF_ATTN
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn

#ifdef SYN_PHASE_TIMING
extern "C" syn_status_t syn_hip_debug_kqf_phase_ts(unsigned long long *host, int n) {
  if (!host || n <= 0 || n > 256) return SYN_ERR_INVALID_ARG;
  SYN_HIP(hipDeviceSynchronize());
  SYN_HIP(hipMemcpyFromSymbol(host, HIP_SYMBOL(syn::kqf_phase_ts), (size_t)n * 8, 0,
                              hipMemcpyDeviceToHost));
  return SYN_OK;
}
#endif
