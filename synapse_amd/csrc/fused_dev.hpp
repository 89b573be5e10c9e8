// Device-side parts of the fused decode kernels (decode_fused.hip):
// workgroup reductions, the activation quantizer of a row
// held in registers, the GEMV prologues (residual + RMSNorm + quantize), and
// the attention chains in the reference's float order.
#pragma once

#include "decode_fused.hpp"
#include "phase_ts.hpp"
#include "reduce_order.hpp"

namespace syn {

// ------------------------------------------------------------------ helpers

// Rows of a prologue vector held per thread: element j = threadIdx.x + u*NT.
constexpr int RB = 8;

// One step of a wave max over non-negative values through a DPP lane move;
// lanes whose source is outside the row/wave read 0, which max ignores.
template <int CTRL>
__device__ __forceinline__ float dpp_fmax(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true);
  return fmaxf(v, __int_as_float(s));
}

// max over the 64 lanes of non-negative values: row_shr 1/2/4/8 leave each
// row's max in its lane 15, row_bcast 15/31 carry them to lane 63
__device__ __forceinline__ float wave_max_nonneg(float v) {
  v = dpp_fmax<0x111>(v);
  v = dpp_fmax<0x112>(v);
  v = dpp_fmax<0x114>(v);
  v = dpp_fmax<0x118>(v);
  v = dpp_fmax<0x142>(v);
  v = dpp_fmax<0x143>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Workgroup max of non-negative values, first half: each wave leaves its max
// in red[slot + wave].  The caller's next barrier publishes it.
template <int NT>
__device__ __forceinline__ void wg_max_post(float v, float *red, int slot) {
  v = wave_max_nonneg(v);
  if ((threadIdx.x & 63) == 0) red[slot + (threadIdx.x >> 6)] = v;
}

// second half (after a barrier)
template <int NT>
__device__ __forceinline__ float wg_max_get(const float *red, int slot) {
  float m = red[slot];
#pragma unroll
  for (int i = 1; i < NT / 64; i++) m = fmaxf(m, red[slot + i]);
  return m;
}

// quantizePerChannelInt8 (quantize.zig:12-47) of a row held in registers
// (element j = threadIdx.x + u*NT, valid for j < n), given the row's max|v|:
// writes q[j] and returns the row scale.
template <int NT, int R>
__device__ float quantize_regs_with_max(const float (&v)[R], int n, float mx, int8_t *q) {
  if (mx == 0.0f) {
#pragma unroll
    for (int u = 0; u < R; u++)
      if (threadIdx.x + u * NT < n) q[threadIdx.x + u * NT] = 0;
    return 1.0f;
  }
  const float inv = 127.0f / mx;
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int j = threadIdx.x + u * NT;
    if (j < n) {
      float r = roundf(v[u] * inv);
      r = fminf(127.0f, fmaxf(-127.0f, r));
      q[j] = (int8_t)(int)r;
    }
  }
  return mx / 127.0f;
}

// per-thread max|v[u]| over its valid elements (the reference's `if a > m`)
template <int NT, int R>
__device__ __forceinline__ float local_absmax(const float (&v)[R], int n) {
  float mx = 0.0f;
#pragma unroll
  for (int u = 0; u < R; u++) {
    const float a = fabsf(v[u]);
    if (threadIdx.x + u * NT < n && a > mx) mx = a;
  }
  return mx;
}

// the whole quantizer: workgroup max (one barrier), then quantize_regs_with_max
template <int NT, int R>
__device__ float quantize_regs(const float (&v)[R], int n, int8_t *q, float *red, int slot) {
  wg_max_post<NT>(local_absmax<NT, R>(v, n), red, slot);
  bar<NT>();
  return quantize_regs_with_max<NT, R>(v, n, wg_max_get<NT>(red, slot), q);
}

// ------------------------------------------------------------------ split-K GEMV
// PRO_NORM: residual + RMSNorm (sum of squares in the 4-chain order of
// ops/norm.rs) + quantize; PRO_MNORM: the same with one sequential sum of
// squares (pure_rust_ops.rs:96-112, the Mamba blocks' norm); PRO_QUANT:
// quantize an f32 vector; PRO_SWIGLU: silu(gate) * up of GEMV rows, then
// quantize; PRO_ROWS: quantize GEMV rows (RowSrc values); PRO_HQ: quantize
// this split's K range of an f32 vector whose max |v| another kernel has
// already reduced (hmax); PRO_CONV: the Mamba block's conv1d step + SiLU of
// GEMV rows over a 4-tap ring state (int8_mamba.rs:43-56), then quantize
enum {
  PRO_NORM = 0,
  PRO_QUANT = 1,
  PRO_SWIGLU = 2,
  PRO_MNORM = 3,
  PRO_ROWS = 4,
  PRO_HQ = 5,
  PRO_CONV = 6
};

struct ProArgs {
  // PRO_NORM: x = (base ? base : embed[st->token]) + delta
  const float *base;
  const float *embed;
  const StepState *st;
  int vocab;
  RowSrc delta;
  float *res_out;
  const float *nw;
  const float *zero_row;  // H zeros (the embedding row of an id >= vocab)
  float eps;
  // PRO_QUANT, PRO_HQ (with hmax = max |vec| as f32 bits)
  const float *vec;
  const unsigned *hmax;
  // PRO_ROWS
  RowSrc rows;
  // PRO_SWIGLU, PRO_CONV; exp_tab = device address of syn_exp2_tab, passed as a plain
  // pointer so its load is ordered like any other (a __constant__ load may be
  // moved behind the weight loads)
  RowSrc gu;
  const uint64_t *exp_tab;
  // PRO_CONV: rows (the new inputs), ring [H][4] (slot p % 4 holds the input
  // of position p), conv weights [H][4] and bias, conv_out = the conv + SiLU
  // values (workgroup 0, with the new ring slot)
  float *ring;
  const float *conv_w, *conv_b;
  float *conv_out;
  // all: prologue vector length (the GEMV's K) and the scale output
  int H;
  float *s_out;
};

struct GemvArgs {
  const i32x4 *W;
  int C, cs;
  int *acc;
  // gate|up pairs (GU kernels): grid panel p covers gate panel p and up
  // panel `pairs` + p of the stacked [gate | up] matrix; acc64[64p + r]
  // packs row 64p + r's gate and up sums and arrivals (gu_pack); the slice
  // that completes a row writes h = silu(gate) * up for it (ws: the stacked
  // rows' scales) and max |h| to hmax
  int pairs = 0;
  unsigned long long *acc64 = nullptr;
  const float *ws = nullptr;
  float *h = nullptr;
  unsigned *hmax = nullptr;
  const uint64_t *exp_tab = nullptr;
};

// One 64-bit accumulator per gate|up row: bits 0-27 the gate sum, 28-55 the
// up sum (two's complement fields), 56-63 the number of K slices added.
// Every field is added in the same integer add: the total is
// count * 2^56 + up * 2^28 + gate modulo 2^64, and |gate|, |up| < 2^27
// (K <= 8322 int8 products of magnitude <= 127 * 127) with at most 255
// slices recover each field exactly.
__device__ __forceinline__ unsigned long long gu_pack(int gate, int up) {
  return (1ull << 56) + ((unsigned long long)(long long)up << 28) +
         (unsigned long long)(long long)gate;
}
__device__ __forceinline__ long long gu_sext28(unsigned long long v) {
  return (long long)(v << 36) >> 36;
}
__device__ __forceinline__ void gu_unpack(unsigned long long t, int &gate, int &up, int &count) {
  const long long g = gu_sext28(t);
  const unsigned long long t1 = (t - (unsigned long long)g) >> 28;
  const long long u = gu_sext28(t1);
  gate = (int)g;
  up = (int)u;
  count = (int)((t1 - (unsigned long long)u) >> 28);
}

// ------------------------------------------------------------------ prologue parts
// PRO_NORM / PRO_MNORM loads: x = (base | embed row of st->token | zero row)
// + delta rows, the norm gains; issue() is called once these are requested,
// so the caller's weight loads queue behind them (element j = tid + u*NT,
// clamped to H-1)
template <int NT, int R, class Issue>
__device__ __forceinline__ void norm_prologue_load(const ProArgs &a, int H, float (&x)[R],
                                                   float (&nwv)[R], Issue issue) {
  const int tid = threadIdx.x;
  const float *src = a.base;
  if (!src) {
    const uint32_t tok = a.st->token;
    src = tok < (uint32_t)a.vocab ? a.embed + (size_t)tok * H : a.zero_row;
  }
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int j = min(tid + u * NT, H - 1);
    x[u] = src[j];
    nwv[u] = a.nw[j];
  }
  // without a delta the loads below read the norm gains instead (in-bounds,
  // values unused), so that no load sits behind a branch
  const bool has_delta = a.delta.acc != nullptr;
  const int *dacc = has_delta ? a.delta.acc : reinterpret_cast<const int *>(a.nw);
  const float *dws = has_delta ? a.delta.ws : a.nw;
  const float *dsxp = has_delta ? a.delta.sx : a.nw;
  int da[R];
  float dw[R];
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int j = min(tid + u * NT, H - 1);
    da[u] = dacc[j];
    dw[u] = dws[j];
  }
  const float dsx = dsxp[0];
  issue();
  if (has_delta) {
#pragma unroll
    for (int u = 0; u < R; u++) {
      const float f = (float)da[u] * dsx;
      const float d = f * dw[u];
      x[u] = x[u] + d;
    }
  }
}

// RMSNorm (ops/norm.rs:8-38): out = (x*w) * (1/sqrt(sumsq/n + eps)), then
// the quantizer's max|out|; returns the row scale with xq[0..H) written.
// Scaling by the positive `scale` is a monotonic rounding, so max|t*scale|
// = fl(max|t| * scale): the max of t = x*w is reduced while lanes 0-3 run
// the sum-of-squares chains (or lane 0 the single sequential sum, SEQ).
// sq: LDS, round4(H) floats.
template <int NT, int R, bool SEQ>
__device__ float norm_quant(float eps, int H, const float (&x)[R], const float (&nwv)[R],
                            float *sq, int8_t *xq, float *red SYN_TS_PARAM) {
  const int tid = threadIdx.x;
  float t[R];
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int j = tid + u * NT;
    if (j < H) sq[SEQ ? j : sq_slot(j, H)] = x[u] * x[u];
    t[u] = x[u] * nwv[u];
  }
  wg_max_post<NT>(local_absmax<NT, R>(t, H), red, 0);
  SYN_TS(10);
  bar<NT>();
  SYN_TS(11);
  float ss;
  if constexpr (SEQ) {
    if (tid < 64) {  // wave 0 runs the single chain
      const float r = wave_seq_sum_long(sq, H, 0.0f);
      if (tid == 0) red[36] = r;
    }
    bar<NT>();
    ss = red[36];
  } else {
    ss = sumsq_chains<NT>(sq, H, red);
  }
  SYN_TS(12);
  const float scale = 1.0f / sqrtf(ss / (float)H + eps);
  float nv[R];
#pragma unroll
  for (int u = 0; u < R; u++) nv[u] = t[u] * scale;
  float mx = wg_max_get<NT>(red, 0) * scale;
  if (!(mx <= 3.402823466e38f) || !(scale > 0.0f)) {  // inf/nan rows: reduce explicitly
    wg_max_post<NT>(local_absmax<NT, R>(nv, H), red, 16);
    bar<NT>();
    mx = wg_max_get<NT>(red, 16);
  }
  SYN_TS(13);
  return quantize_regs_with_max<NT, R>(nv, H, mx, xq);
}

// quantizePerChannelInt8 (quantize.zig:12-47) of elements [k0, k1) of a row
// whose max|v| is mx, held as element j = k0 + tid + u*NT; writes xq[j] and
// returns the row scale
template <int NT, int R>
__device__ float quantize_range_with_max(const float (&v)[R], int k0, int k1, float mx,
                                         int8_t *xq) {
  const int tid = threadIdx.x;
  if (mx == 0.0f) {
#pragma unroll
    for (int u = 0; u < R; u++)
      if (k0 + tid + u * NT < k1) xq[k0 + tid + u * NT] = 0;
    return 1.0f;
  }
  const float inv = 127.0f / mx;
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int j = k0 + tid + u * NT;
    if (j < k1) {
      float r = roundf(v[u] * inv);
      r = fminf(127.0f, fmaxf(-127.0f, r));
      xq[j] = (int8_t)(int)r;
    }
  }
  return mx / 127.0f;
}

// ------------------------------------------------------------------ attention parts
// max over the wave of any floats (invalid DPP sources keep -inf)
template <int CTRL>
__device__ __forceinline__ float dpp_fmax_any(float v) {
  const int s = __builtin_amdgcn_update_dpp((int)0xff800000u, __float_as_int(v), CTRL, 0xf, 0xf,
                                            false);
  return fmaxf(v, __int_as_float(s));
}
__device__ __forceinline__ float wave_max_any(float v) {
  v = dpp_fmax_any<0x111>(v);
  v = dpp_fmax_any<0x112>(v);
  v = dpp_fmax_any<0x114>(v);
  v = dpp_fmax_any<0x118>(v);
  v = dpp_fmax_any<0x142>(v);
  v = dpp_fmax_any<0x143>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

constexpr int kAttnNT = 256;
constexpr int kPvChunk = 128;            // positions per staged V chunk
constexpr int kPvGroups = kPvChunk / 4;  // 4-position groups per chunk

// V groups [g0, g0 + ngroups) (4 positions of one column per 16 bytes,
// indices clamped to the cache; ngroups rounded up to whole wave
// instructions) of columns [cb0, cb0 + CB) into dst[group][CB], issued by
// waves w0 .. w0 + nw - 1
template <int CB>
__device__ __forceinline__ void stage_v_chunk(const f32x4 *V4, int hd, int s4, int cb0, int g0,
                                              f32x4 *dst, int wave, int w0, int nw, int lane,
                                              int ngroups) {
  constexpr int GPI = 64 / CB;  // groups per wave instruction
  const int gl = lane / CB, col = lane % CB;
  for (int gi = (wave - w0) * GPI; gi < ngroups; gi += nw * GPI) {
    const int g = min(g0 + gi + gl, s4 - 1);
    g2lds16(V4 + (size_t)g * hd + cb0 + col, dst + gi * CB);
  }
}

// score chain sum_d q[d] * k[d], d = 0 .. HD-1 in order: q from LDS
// (broadcast), the K row in registers
template <int HD, bool FUSED>
__device__ __forceinline__ float q_dot_chain(const f32x4 *q4, const f32x4 (&kr)[HD / 4]) {
  constexpr int NB = HD / 4;
  constexpr int BS = NB < 8 ? NB : 8;
  constexpr int NBLK = NB / BS;
  float acc = 0.0f;
  f32x4 qa[BS], qb[BS];
  auto load = [&](f32x4(&r)[BS], int blk) {
#pragma unroll
    for (int k = 0; k < BS; k++) r[k] = q4[blk * BS + k];
  };
  auto step = [&](f32x4(&r)[BS], int blk) {
#pragma unroll
    for (int k = 0; k < BS; k++) {
      const f32x4 kv = kr[blk * BS + k];
      if constexpr (FUSED) {
        acc = __builtin_fmaf(r[k].x, kv.x, acc);
        acc = __builtin_fmaf(r[k].y, kv.y, acc);
        acc = __builtin_fmaf(r[k].z, kv.z, acc);
        acc = __builtin_fmaf(r[k].w, kv.w, acc);
      } else {
        float t;
        t = r[k].x * kv.x; acc = acc + t;
        t = r[k].y * kv.y; acc = acc + t;
        t = r[k].z * kv.z; acc = acc + t;
        t = r[k].w * kv.w; acc = acc + t;
      }
    }
  };
  load(qa, 0);
#pragma unroll
  for (int blk = 0; blk < NBLK; blk += 2) {
    if (blk + 1 < NBLK) load(qb, blk + 1);
    __builtin_amdgcn_sched_barrier(0);
    pin_regs(qa);
    step(qa, blk);
    if (blk + 1 < NBLK) {
      if (blk + 2 < NBLK) load(qa, blk + 2);
      __builtin_amdgcn_sched_barrier(0);
      pin_regs(qb);
      step(qb, blk + 1);
    }
  }
  return acc;
}

// The rounded-product form of the score chain: t_d = q[d] * k[d], then
// acc = acc + t_d for d = 0 .. HD-1 in order.  The products do not depend
// on the sum, so they are all formed first (in place of the K row, which
// the caller no longer needs) and the chain is one dependent add per
// element instead of a multiply and an add.  Same values and order as
// q_dot_chain<HD, false>.
template <int HD>
__device__ __forceinline__ float q_dot_chain_plain(const f32x4 *q4, f32x4 (&kr)[HD / 4]) {
  constexpr int NB = HD / 4;
  constexpr int BS = NB < 8 ? NB : 8;
#pragma unroll
  for (int blk = 0; blk < NB / BS; blk++) {
    f32x4 q[BS];
#pragma unroll
    for (int k = 0; k < BS; k++) q[k] = q4[blk * BS + k];
#pragma unroll
    for (int k = 0; k < BS; k++) {
      f32x4 &kv = kr[blk * BS + k];
      kv.x = q[k].x * kv.x;
      kv.y = q[k].y * kv.y;
      kv.z = q[k].z * kv.z;
      kv.w = q[k].w * kv.w;
    }
  }
  pin_regs(kr);  // every product formed before the chain starts
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < NB; c++) {
    acc = acc + kr[c].x;
    acc = acc + kr[c].y;
    acc = acc + kr[c].z;
    acc = acc + kr[c].w;
  }
  return acc;
}

// P.V chain of one column over whole 4-position groups [0, ng) of a staged
// chunk: probabilities e4 (LDS, broadcast), the column's V at vt[g * CB]
template <bool FUSED, int CB>
__device__ __forceinline__ float pv_chain(const f32x4 *e4, const f32x4 *vt, int ng, float acc) {
  auto step = [&](const f32x4 &E, const f32x4 &Vv) {
    if constexpr (FUSED) {
      acc = __builtin_fmaf(E.x, Vv.x, acc);
      acc = __builtin_fmaf(E.y, Vv.y, acc);
      acc = __builtin_fmaf(E.z, Vv.z, acc);
      acc = __builtin_fmaf(E.w, Vv.w, acc);
    } else {
      float t;
      t = E.x * Vv.x; acc = acc + t;
      t = E.y * Vv.y; acc = acc + t;
      t = E.z * Vv.z; acc = acc + t;
      t = E.w * Vv.w; acc = acc + t;
    }
  };
  f32x4 ea[8], va[8], eb[8], vb[8];
  auto load = [&](f32x4(&E)[8], f32x4(&Vr)[8], int blk) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      E[k] = e4[blk * 8 + k];
      Vr[k] = vt[(blk * 8 + k) * CB];
    }
  };
  auto run = [&](f32x4(&E)[8], f32x4(&Vr)[8]) {
    if constexpr (!FUSED) {  // the block's rounded products first, then its adds in order
#pragma unroll
      for (int k = 0; k < 8; k++) Vr[k] = E[k] * Vr[k];
      pin_regs(Vr);
#pragma unroll
      for (int k = 0; k < 8; k++) {
        acc = acc + Vr[k].x;
        acc = acc + Vr[k].y;
        acc = acc + Vr[k].z;
        acc = acc + Vr[k].w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; k++) step(E[k], Vr[k]);
    }
  };
  const int nb = ng >> 3;
  int blk = 0;
  if (nb > 0) {
    load(ea, va, 0);
    for (; blk + 1 < nb; blk += 2) {
      load(eb, vb, blk + 1);
      __builtin_amdgcn_sched_barrier(0);
      pin_regs(ea);
      pin_regs(va);
      run(ea, va);
      load(ea, va, min(blk + 2, nb - 1));  // in bounds; unused past the end
      __builtin_amdgcn_sched_barrier(0);
      pin_regs(eb);
      pin_regs(vb);
      run(eb, vb);
    }
    if (blk < nb) {
      pin_regs(ea);
      pin_regs(va);
      run(ea, va);
    }
  }
  // the last ng % 8 groups: one batch of reads, then the chains
  const int rg = ng - nb * 8;
  if (rg > 0) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int g = nb * 8 + min(k, rg - 1);
      ea[k] = e4[g];
      va[k] = vt[g * CB];
    }
    pin_regs(ea);
    pin_regs(va);
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (k < rg) step(ea[k], va[k]);
  }
  return acc;
}

template <int HD>
constexpr int attn_cb() {
  return HD < 64 ? HD : 64;
}

}  // namespace syn
