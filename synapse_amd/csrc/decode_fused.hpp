// Fused INT8 W8A8 decode step (batch 1): five kernels per decoder layer
// instead of one per reference op.  See decode_fused.hip for the kernels.
#pragma once

#include "layer_ops.hpp"

namespace syn {

// The rows of a split-K INT8 GEMV as a consumer sees them:
//   value(r) = (f32(acc[r]) * sx[0]) * ws[r]
// (the M <= 16 epilogue of int8GemvRow, qmatmul.zig:171-256), where acc is
// the exact int32 dot product, accumulated over the K split with atomics.
// With `f` set the rows are a plain f32 vector instead: value(r) = f[r]
// (the f32 decoders' GEMV outputs).
struct RowSrc {
  const int *acc = nullptr;
  const float *sx = nullptr;
  const float *ws = nullptr;
  const float *f = nullptr;
  __host__ __device__ bool empty() const { return !acc && !f; }
};

__device__ __forceinline__ float row_value(const RowSrc &s, int r) {
  if (s.f) return s.f[r];
  const float f = (float)s.acc[r] * s.sx[0];
  return f * s.ws[r];
}
// the same with the source kind fixed at compile time (no branch, so the
// loads can stay in flight)
template <bool ACC>
__device__ __forceinline__ float row_value_t(const RowSrc &s, int r) {
  if constexpr (ACC) {
    const float f = (float)s.acc[r] * s.sx[0];
    return f * s.ws[r];
  } else {
    return s.f[r];
  }
}

// One INT8 linear in the panel layout, with the K split used in the step.
struct SplitGemv {
  const void *W = nullptr;   // panel layout (linear.hpp)
  const float *ws = nullptr; // per-row scales [N64]
  int N = 0, N64 = 0, C = 0; // rows, padded rows, 16-byte K chunks
  int ks = 1, cs = 0;        // K split, chunks per split
  int nt = 256;              // threads per workgroup
  int u = 1;                 // chunks per wave (prefetched at kernel entry)
  int *acc = nullptr;        // int32 accumulators [N64], zero before the step
  RowSrc rows(const float *sx) const { return RowSrc{acc, sx, ws}; }
};

// Choose the K split so that about `target_wg` workgroups stream the matrix
// and every wave holds at most 8 chunks (128 bytes per lane) in flight.
SplitGemv plan_split_gemv(const void *W, const float *ws, int N, int C, int target_wg, int nt);

// x = (base ? base : embed[state->token] or zero_row) + delta ; res_out = x
// (workgroup 0); xq = q8(rmsnorm(x, nw, eps)); s_out = its scale (workgroup
// 0); acc += xq . W over this split of K.  The sum of squares runs in the
// 4-chain order of ops/norm.rs, or as one sequential sum (the Mamba blocks'
// pure_rust rmsnorm) with sequential_sumsq.
syn_status_t launch_fused_norm_gemv(const float *base, const float *embed, const StepState *st,
                                    int vocab, const float *zero_row, RowSrc delta,
                                    float *res_out, const float *nw, float eps, int H,
                                    float *s_out, const SplitGemv &g, hipStream_t s,
                                    bool sequential_sumsq = false);
// xq = q8(rows[0..H)) of another split GEMV's rows ; s_out ; acc += xq . W
syn_status_t launch_fused_rows_gemv(RowSrc rows, int H, float *s_out, const SplitGemv &g,
                                    hipStream_t s);
// device address of the expf table syn_exp2_tab (per device), for kernels
// that stage it in LDS
const uint64_t *exp_table_address();
// x = silu(conv1d step of rows over the 4-tap ring, weights conv_w [H][4],
// bias conv_b) (int8_mamba.rs:43-56) ; xq = q8(x) ; s_out ; acc += xq . W;
// workgroup 0 writes x to conv_out and rows to ring slot st->pos % 4
syn_status_t launch_fused_conv_gemv(RowSrc rows, const StepState *st, float *ring,
                                    const float *conv_w, const float *conv_b, float *conv_out,
                                    int H, float *s_out, const SplitGemv &g, hipStream_t s);
// xq = q8(vec) ; s_out ; acc += xq . W
syn_status_t launch_fused_quant_gemv(const float *vec, int H, float *s_out, const SplitGemv &g,
                                     hipStream_t s);
// h = silu(gate) * up from the stacked [gate | up] rows ; xq = q8(h) ; acc += xq . W
syn_status_t launch_fused_swiglu_gemv(RowSrc gu, int inter, float *s_out, const SplitGemv &g,
                                      hipStream_t s);
// x_mid = x + delta (res_out, workgroup 0); xq = q8(rmsnorm(x_mid)); the
// stacked [gate | up] GEMV (int8 panel layout, 2*inter rows) split over K in
// pairs of panels (gate panel p with up panel inter/64 + p; g planned by
// plan_gu_pairs; g.acc holds inter 64-bit packed row accumulators (8-byte
// aligned, zero before the step); the slice that completes row j writes
// h[j] = silu(gate_j) * up_j and folds max |h| into hmax (f32 bits, atomic
// max; zero before the step); s_out = xq's scale
syn_status_t launch_gu_swiglu(const float *base, RowSrc delta, float *res_out, const float *nw,
                              float eps, int H, float *s_out, const SplitGemv &g, const float *ws,
                              int inter, float *h, unsigned *hmax, hipStream_t s);
bool gu_swiglu_fits(int H, int inter);
SplitGemv plan_gu_pairs(const void *W, const float *ws, int inter, int C, int target_wg, int nt);
// xq = q8(vec) over this split's K range with the max *hmax reduced
// elsewhere ; s_out ; acc += xq . W
syn_status_t launch_fused_hq_gemv(const float *vec, const unsigned *hmax, int H, float *s_out,
                                  const SplitGemv &g, hipStream_t s);
// per query head: q/k/v rows from the QKV partials, head RMSNorm, RoPE at
// state->pos, KV append, attention over positions [0, pos]; scores is
// [nh][max_seq] f32 scratch
syn_status_t launch_fused_attention(RowSrc qkv, int nh, int nkv, int hd, const float *qn,
                                    const float *kn, float eps, const float *cosT,
                                    const float *sinT, const StepState *st, float *kc, float *vc,
                                    int max_seq, float *scores, float *out, hipStream_t s);
bool fused_attention_fits(int hd, int max_seq);
// the fused GEMV prologue holds its activation row (f32 twice + int8) in LDS
bool fused_gemv_fits(int H);
// final residual + RMSNorm + quantize into global xq / s_out (one workgroup)
syn_status_t launch_fused_final_norm(const float *base, RowSrc delta, const float *nw, float eps,
                                     int H, int8_t *xq, float *s_out, hipStream_t s);
// per-panel top-2 of the lm_head rows (merged by launch_argmax_advance)
struct Top2v {
  float v1;
  int i1;
  float v2;
};

// larger value wins; on equal values the larger index (the last maximum,
// sampler.rs:217-224); v2 = the largest value other than the winner
__device__ __forceinline__ Top2v top2v_merge(Top2v a, Top2v b) {
  const bool bw = (b.v1 > a.v1) || (b.v1 == a.v1 && b.i1 > a.i1);
  const Top2v w = bw ? b : a, l = bw ? a : b;
  return Top2v{w.v1, w.i1, fmaxf(w.v2, l.v1)};
}

__device__ __forceinline__ Top2v wave_top2(Top2v t) {
  for (int o = 32; o > 0; o >>= 1) {
    Top2v u;
    u.v1 = __shfl_xor(t.v1, o);
    u.i1 = __shfl_xor(t.i1, o);
    u.v2 = __shfl_xor(t.v2, o);
    t = top2v_merge(t, u);
  }
  return t;
}

// lm_head GEMV (one workgroup per 64-row panel) -> logits + per-panel top-2
syn_status_t launch_lmhead_top2(const void *W, const float *ws, int N, int C, const int8_t *xq,
                                const float *sx, float *logits, float *pv, int *pi, float *pv2,
                                hipStream_t s);
// zero n int32 (the step's split-K accumulators; a kernel, not a memset
// node, so the step can be captured in a graph)
syn_status_t launch_zero_i32(int *p, size_t n, hipStream_t s);
// merge the per-panel top-2 -> token, margin, history; pos += 1, step += 1
syn_status_t launch_argmax_advance(const float *pv, const int *pi, const float *pv2, int np,
                                   StepState *st, uint32_t *history, float *mhist,
                                   hipStream_t s);

}  // namespace syn
