// Fused f32 decode step of the K-quant CausalLM (klm_fused.hip).
#pragma once

#include "kquant.hpp"
#include "layer_ops.hpp"

namespace syn {

// A weight matrix as the fused GEMV reads it: 16-byte planes
// [panel][block][plane][64 rows] and f16 d values [panel][block][64 rows]
// (QLinearKQ's layout; QLinearQ4_0's nibble planes and scales are the same
// with one plane per block).  Q4_0 scales are read as IEEE f16 values.
struct KqfW {
  int fmt = 0;
  size_t n = 0, k = 0;
  int blocks = 0;  // blocks per row
  const void *wq = nullptr;
  const void *wd = nullptr;
  KqfW(const QLinearKQ &w);
  KqfW(const QLinearQ4_0 &w);
};

// Launch shape of one split-K GEMV: `groups` row groups (64-row panels, or
// 32 gate + 32 up rows) x `ks` splits of `bs` 256-element units each.
struct KqfPlan {
  int groups = 0, units = 0, bs = 0, ks = 0;
};

// The decode GEMV's input row.  The residual stream and the split-K
// accumulators are fixed point, value * 2^32 in an int64 (sums of them are
// exact, so the split-K atomics are order-independent and deterministic).
struct KqfIn {
  // NORM: rmsnorm of the residual r; EMBED: rmsnorm of the embedding row of
  // st->token (a zero row past the vocabulary), whose fixed-point form
  // workgroup (0,0) stores to r_out.  The GEMV reads row * gain and scales
  // its dot products by 1/rms(row).
  const long long *r = nullptr;
  const float *embed = nullptr;
  int vocab = 0;
  long long *r_out = nullptr;
  const float *gain = nullptr;
  float eps = 0.0f;
  int H = 0;
  // NONE: the f32 row itself
  const float *x = nullptr;
  // ATTN: the combine of the attention's per-chunk partials
  const float *ao = nullptr, *aml = nullptr;
  int hd = 0, nch = 0;
  const StepState *st = nullptr;
  // CONV: the LIV conv step (liv_conv_channel) of the in_proj accumulator
  // cacc (rows [B | C | x], fixed point) over the state halves cstate
  // ([2][inner][ck]; row group 0 writes the next half), taps cw [inner][ck],
  // bias cb (may be null), at st->pos
  const long long *cacc = nullptr;
  float *cstate = nullptr;
  const float *cw = nullptr, *cb = nullptr;
  int inner = 0, ck = 0;
};

enum { KQF_PRO_NONE = 0, KQF_PRO_NORM = 1, KQF_PRO_EMBED = 2, KQF_PRO_ATTN = 3, KQF_PRO_CONV = 4 };

constexpr int kKqfTop2Groups = 256;  // lm_head workgroups: about one per CU

// whether the fused step supports a model of these shapes and formats
bool kqf_fits(int H, int qd, int inter, int nh, int nkv, int hd, int max_seq, const int *fmts,
              int nfmt);
// split plan of a GEMV over n rows and k inputs (gu: gate|up pairs, whole K)
KqfPlan kqf_plan(const KqfW &w, bool gu);
// split-K GEMV whose splits add their fixed-point dot products into acc[row]
// with atomics; zero[0 .. nzero) is cleared first (the QKV accumulator, for
// the next layer, by the O projection)
syn_status_t kqf_gemv(const KqfW &w, const KqfPlan &p, int pro, const KqfIn &in,
                      long long *acc, long long *zero, int nzero, hipStream_t s);
// gate|up rows (w = [gate; up], inter rows each) over the whole K of
// rmsnorm(r) and h = silu(gate) * up
syn_status_t kqf_gate_up(const KqfW &w, const KqfPlan &p, const KqfIn &in, int inter,
                         float *h, hipStream_t s);
// lm_head rows of rmsnorm(r) -> logits and a top-2 per workgroup (pv, pi,
// pv2); workgroup b takes the 64-row panels b, b + p.groups, ... (p.groups
// at most kKqfTop2Groups)
syn_status_t kqf_lm_head(const KqfW &w, const KqfPlan &p, const KqfIn &in, float *logits,
                         float *pv, int *pi, float *pv2, hipStream_t s);
// attention of one token per (kv head, 64-position chunk): q/k/v from the
// fixed-point QKV accumulator, head norms (qn/kn may be null), RoPE, KV
// append at st->pos, chunk softmax and P.V -> ao [nh][nch][hd], aml [nh][nch][2]
syn_status_t kqf_attention(const long long *qkv, int nh, int nkv, int hd, const float *qn,
                           const float *kn, float eps, const float *cosT, const float *sinT,
                           const StepState *st, float *kc, float *vc, int max_seq, float *ao,
                           float *aml, hipStream_t s);
inline int kqf_chunks(int max_seq) { return (max_seq + 63) / 64; }

}  // namespace syn
