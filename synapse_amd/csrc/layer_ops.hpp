// Small device-resident kernels of the decoder layer.  Each one computes in
// the reference's floating-point order so that the whole decode step is
// bit-identical to the cpu_simd path.
#pragma once

#include "common.hpp"

namespace syn {

// KV cache layout (per layer), laid out for the decode attention's loads:
//  K: [kv_head][position tile of 64][d/4][64 positions][4 d]  - a wave whose
//     lanes are positions reads 1 KiB contiguously per 16-byte load;
//  V: [kv_head][position/4][d][4 positions]                   - a wave whose
//     lanes are output columns d reads 4 positions per 16-byte load.
// head_dim is padded to a multiple of 4 in K (the pad is never read as data)
// and max_seq to multiples of 64 (K) and 4 (V).
__host__ __device__ __forceinline__ size_t kv_k_index(int p, int g, int d, int hd, int max_seq) {
  const int hd4 = (hd + 3) >> 2, tiles = (max_seq + 63) >> 6;
  return ((((size_t)g * tiles + (p >> 6)) * hd4 + (d >> 2)) * 64 + (p & 63)) * 4 + (d & 3);
}
__host__ __device__ __forceinline__ size_t kv_v_index(int p, int g, int d, int hd, int max_seq) {
  const int s4 = (max_seq + 3) >> 2;
  return (((size_t)g * s4 + (p >> 2)) * hd + d) * 4 + (p & 3);
}
inline size_t kv_k_elems(int nkv, int hd, int max_seq) {
  return (size_t)nkv * ((max_seq + 63) / 64) * 64 * (((hd + 3) / 4) * 4);
}
inline size_t kv_v_elems(int nkv, int hd, int max_seq) {
  return (size_t)nkv * ((max_seq + 3) / 4) * 4 * hd;
}

struct StepState {  // device-resident decode state (read by kernels in a graph)
  int pos;          // tokens already in the KV cache
  uint32_t token;   // last sampled token
  int step;         // decode steps taken since the last reset of the counter
  float margin;     // top1 - top2 logit of the last argmax
  int nhist = -1;   // tokens of the history the sampler's repetition penalty
                    // reads (-1: all `step` sampled so far)
};

// x[r] = embed[ids[r]] (zero row for ids >= vocab), ids on device
syn_status_t launch_embed(const float *embed, const uint32_t *ids, int rows, int hidden,
                          int vocab, float *x, hipStream_t s);
// per row: x += delta (if delta); normed = rmsnorm(x, w, eps); quantize(normed)
// (xq == nullptr: no quantization, normed must be given)
syn_status_t launch_rmsnorm_quant(float *x, const float *delta, const float *w, float eps,
                                  int rows, int hidden, int8_t *xq, int ldq, float *sx,
                                  float *normed, hipStream_t s);
// headwise q/k RMSNorm + RoPE (rotate-half) + KV-cache append for `rows` tokens
// at positions pos0 + r (pos0 = *d_pos if d_pos else pos_static), written to
// cache rows pos0 + r + cache_off.
syn_status_t launch_qk_norm_rope_kv(const float *qkv, int ldqkv, int rows, int n_heads,
                                    int n_kv, int head_dim, const float *q_norm,
                                    const float *k_norm, float eps, const float *rope_cos,
                                    const float *rope_sin, const int *d_pos, int pos_static,
                                    float *q_out, float *kcache, float *vcache, int max_seq,
                                    hipStream_t s, int cache_off = 0);
// single-query GQA attention over positions [0, *d_pos] (cache already holds
// the new token), ops/attention.rs:24-147
syn_status_t launch_attention_decode(const float *q, const float *kcache, const float *vcache,
                                     const int *d_pos, int n_heads, int n_kv, int head_dim,
                                     float *scores, int max_seq, float *out, hipStream_t s);
// causal attention over `t` prompt tokens (cache rows cache_off ..),
// exports.zig:1364-1478 per head
syn_status_t launch_attention_prefill(const float *q, const float *kcache, const float *vcache,
                                      int t, int n_heads, int n_kv, int head_dim, int max_seq,
                                      float *scores, float *out, hipStream_t s, int cache_off = 0);
// the same attention without the reference's float order (parallel chains,
// tree reductions), for the decoders graded to a tolerance; prompts whose
// scores do not fit LDS run launch_attention_prefill
syn_status_t launch_attention_prefill_tol(const float *q, const float *kcache,
                                          const float *vcache, int t, int n_heads, int n_kv,
                                          int head_dim, int max_seq, float *out, hipStream_t s,
                                          int cache_off = 0);
// h = silu(gate) * up (int8.rs:500-503), then quantize rows of h
syn_status_t launch_swiglu_quant(const float *gu, int ldgu, int rows, int inter, int8_t *hq,
                                 int ldq, float *sh, hipStream_t s);
// f32-path SwiGLU (Zig swigluFused order) from [gate | up] rows
syn_status_t launch_swiglu_f32(const float *gu, int ldgu, int rows, int inter, float *h, int ldh,
                               hipStream_t s);
// greedy argmax (last maximum wins, sampler.rs:217-224) -> state->token,
// top1-top2 margin -> state->margin, token also stored to history[state->step]
syn_status_t launch_argmax(const float *logits, int n, float *part_v, int *part_i,
                           float *part_v2, StepState *state, uint32_t *history,
                           float *margin_hist, hipStream_t s);
// state->pos += add_pos; state->step += 1
syn_status_t launch_step_advance(StepState *state, int add_pos, hipStream_t s);
// zero K/V rows at position state->pos of `layers` layer caches (strides in floats)
syn_status_t launch_kv_zero_rows(float *kc, float *vc, size_t k_stride, size_t v_stride,
                                 int layers, int nkv, int hd, int max_seq, const StepState *st,
                                 hipStream_t s);
// state->pos = pos (if pos >= 0), state->nhist = nhist
syn_status_t launch_state_set(StepState *state, int pos, int nhist, hipStream_t s);
// elementwise residual: x += d
syn_status_t launch_add(float *x, const float *d, int n, hipStream_t s);

}  // namespace syn
