/*
 * CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference algorithms (eren23/synapse, Zig
 * cpu_simd kernels + the Rust glue around them).  Every function cites the
 * reference file:line it follows (paths relative to the reference's
 * `synapse/` directory).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker / the timed CPU baseline — never as part of the product path.
 *
 * Build: gcc -O3 -mavx2 -mfma -mf16c -ffp-contract=off -fno-fast-math
 *        (-ffp-contract=off keeps every `a*b + c` the reference writes
 *        unfused; explicit fmaf() calls stand for Zig's @mulAdd).
 */
#ifndef SYN_ORACLE_H
#define SYN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes: synapse.h:27-35 */
#define ORC_OK 0
#define ORC_ERR_NULL_PTR 1
#define ORC_ERR_INVALID_ARG 2
#define ORC_ERR_OUT_OF_MEMORY 3
#define ORC_ERR_SHAPE_MISMATCH 4

/* ---- harness input spec (not a reference algorithm) ---- */
void orc_fill_normal(float *dst, size_t n, uint64_t seed, float stddev);
void orc_fill_token_ids(uint32_t *dst, size_t n, uint64_t seed, uint32_t vocab);

/* ---- f16 conversions ---- */
uint16_t orc_f32_to_f16_trunc(float v);   /* q4_linear.rs:9-33 */
float orc_f16_to_f32_zig(uint16_t bits);  /* qmatmul.zig:346-371 */
float orc_f16_to_f32_rs(uint16_t bits);   /* weight_loading/converter.rs:12-40 */

/* ---- A1: activation quantizer ---- */
int orc_quantize_per_channel_int8(const float *data, size_t channels, size_t channel_size,
                                  int8_t *out, float *scales);

/* ---- A2: weight quantizer (QuantizedLinear::from_f32) ---- */
void orc_minmax_scales(const float *w, size_t channels, size_t channel_size, float *scales);
void orc_quantize_weights_int8(const float *w, const float *scales, size_t out_features,
                               size_t in_features, int8_t *out_kn);

/* ---- A3/A4: INT8 GEMM (int8GemmTiled) ---- */
int orc_qgemm_int8(size_t m, size_t n, size_t k, const int8_t *a, size_t lda, const int8_t *b,
                   size_t ldb, float *c, size_t ldc, const float *scales_a,
                   const float *scales_b);
void orc_naive_int8_gemm(size_t m, size_t n, size_t k, const int8_t *a, size_t lda,
                         const int8_t *b, size_t ldb, float *c, size_t ldc,
                         const float *scales_a, const float *scales_b);

/* ---- A6/A7: Q4_0 ---- */
size_t orc_q4_packed_bytes(size_t out_features, size_t in_features);
void orc_q4_from_f32_packed(const float *w, size_t out_features, size_t in_features,
                            uint8_t *packed);
int orc_q4_0_gemv(size_t n, size_t k, const float *a, const uint8_t *b_q4, float *c);

/* ---- A8..A11: GGUF dequantizers ---- */
int orc_dequant_q4_0(const uint8_t *data, size_t numel, float *out);
int orc_dequant_q8_0(const uint8_t *data, size_t numel, float *out);
int orc_dequant_q4_k(const uint8_t *data, size_t numel, float *out);
int orc_dequant_q6_k(const uint8_t *data, size_t numel, float *out);

/* ---- A12: f32 SGEMM (sgemmTiled semantics) ---- */
int orc_sgemm(size_t m, size_t n, size_t k, const float *a, size_t lda, int trans_a,
              const float *b, size_t ldb, int trans_b, float *c, size_t ldc);

/* ---- A14: per-layer ops ---- */
void orc_rmsnorm(const float *x, const float *w, float eps, size_t rows, size_t hidden,
                 float *out);
void orc_rope_tables(size_t max_pos, size_t head_dim, double base, float *cos_t,
                     float *sin_t);
void orc_rope_apply(float *qk, const float *cos_t, const float *sin_t, size_t seq_len,
                    size_t num_heads, size_t head_dim, size_t pos_offset);
float orc_expf(float x);
float orc_silu(float x);
void orc_softmax_slice(float *x, size_t n);
uint32_t orc_argmax(const float *logits, size_t n);
void orc_attention_decode(const float *q, const float *kcache, const float *vcache,
                          size_t seq_len, size_t num_heads, size_t num_kv_heads,
                          size_t head_dim, float *out);
int orc_fused_attention(size_t seq_q, size_t seq_k, size_t d_head, const float *q,
                        const float *k, const float *v, float *out);

/* ---- A15: INT8 W8A8 causal LM (QuantizedCausalLM) ---- */
typedef struct {
  size_t hidden, n_layers, n_heads, n_kv_heads, head_dim, inter, vocab, max_seq;
  float eps;
  double rope_theta;
} orc_lm_cfg;

typedef struct orc_qlm orc_qlm;
orc_qlm *orc_qlm_create(const orc_lm_cfg *cfg);
void orc_qlm_destroy(orc_qlm *m);
int orc_qlm_set_embed(orc_qlm *m, const float *embed);
int orc_qlm_set_layer(orc_qlm *m, size_t layer, const float *wq, const float *wk,
                      const float *wv, const float *wo, const float *wg, const float *wu,
                      const float *wd);
int orc_qlm_init_synthetic(orc_qlm *m, uint64_t seed_base, float stddev);
/* RMSNorm gains (all 1.0 until set; NULL leaves one as it is), head norms
   on/off, untied lm_head f32 [vocab, h] (quantized at finalize) */
int orc_qlm_set_norms(orc_qlm *m, size_t layer, const float *attn, const float *ffn,
                      const float *q, const float *k);
int orc_qlm_set_final_norm(orc_qlm *m, const float *w);
void orc_qlm_set_qk_norm(orc_qlm *m, int enabled);
int orc_qlm_set_lm_head(orc_qlm *m, const float *w);
int orc_qlm_finalize(orc_qlm *m);
void orc_qlm_reset(orc_qlm *m);
size_t orc_qlm_cur_len(const orc_qlm *m);
int orc_qlm_prefill(orc_qlm *m, const uint32_t *ids, size_t n, float *logits);
int orc_qlm_prefill_append(orc_qlm *m, const uint32_t *ids, size_t n, float *logits);
void orc_qlm_truncate(orc_qlm *m, size_t new_len);
int orc_qlm_forward_one(orc_qlm *m, uint32_t token, float *logits);
int orc_qlm_generate(orc_qlm *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                     uint32_t *out_tokens, float *margins);
const int8_t *orc_qlm_lm_head_weights(const orc_qlm *m); /* [K,N] reference layout */
const float *orc_qlm_lm_head_scales(const orc_qlm *m);

/* ---- f32 CausalLM over GGUF-dequantized weights (models/lm/causal_lm.rs,
 *      decoder_layer.rs): the reference path for Q4_K / Q6_K / Q8_0 models ---- */
#define ORC_FMT_Q8_0 3
#define ORC_FMT_Q4_K 4
#define ORC_FMT_Q6_K 5
typedef struct orc_flm orc_flm;
/* qk_norm: 1 = Qwen3-style q/k RMSNorm (gains 1.0), 0 = none (LLaMA) */
orc_flm *orc_flm_create(const orc_lm_cfg *cfg, int qk_norm);
void orc_flm_destroy(orc_flm *m);
int orc_flm_set_embed(orc_flm *m, const float *embed);
/* one projection of one layer from GGUF bytes: proj 0..6 = q,k,v,o,gate,up,down */
int orc_flm_set_proj(orc_flm *m, size_t layer, int proj, int fmt, const uint8_t *bytes);
int orc_flm_set_lm_head(orc_flm *m, int fmt, const uint8_t *bytes);
/* RMSNorm gains (all 1.0 until set); NULL leaves one as it is */
int orc_flm_set_norms(orc_flm *m, size_t layer, const float *attn, const float *ffn,
                      const float *q, const float *k);
int orc_flm_set_final_norm(orc_flm *m, const float *w);
void orc_flm_reset(orc_flm *m);
int orc_flm_prefill(orc_flm *m, const uint32_t *ids, size_t n, float *logits);
int orc_flm_prefill_append(orc_flm *m, const uint32_t *ids, size_t n, float *logits);
void orc_flm_truncate(orc_flm *m, size_t new_len);
size_t orc_flm_cur_len(const orc_flm *m);
int orc_flm_forward_one_draft(orc_flm *m, uint32_t token, size_t n_draft, float *logits);
int orc_flm_forward_one(orc_flm *m, uint32_t token, float *logits);
int orc_flm_generate(orc_flm *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                     uint32_t *out_tokens, float *margins);
void orc_swiglu_fused(float *dst, const float *gate, const float *up, size_t n);

/* ---- INT8 Mamba (quantization/ssm/int8_mamba.rs): in_proj/out_proj W8A8,
 *      x_proj/dt_proj/lm_head f32, selective scan zig/src/ops/selective_scan.zig ---- */
typedef struct {
  size_t d_model, d_inner, d_state, d_conv, dt_rank, n_layers, vocab;
  float eps;
} orc_mamba_cfg;
typedef struct orc_mamba orc_mamba;
orc_mamba *orc_mamba_create(const orc_mamba_cfg *cfg);
void orc_mamba_destroy(orc_mamba *m);
/* synthetic weights (seed spec documented in oracle.c) */
int orc_mamba_init_synthetic(orc_mamba *m, uint64_t seed_base);
int orc_mamba_init_synthetic_std(orc_mamba *m, uint64_t seed_base, float std);
/* BASELINE config 5's variant: x_proj and dt_proj as W8A8 QuantizedLinears */
int orc_mamba_set_int8_xdt(orc_mamba *m);
void orc_mamba_reset(orc_mamba *m);
int orc_mamba_prefill(orc_mamba *m, const uint32_t *ids, size_t n, float *logits);
int orc_mamba_decode_one(orc_mamba *m, uint32_t token, float *logits);
int orc_mamba_generate(orc_mamba *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                       uint32_t *out_tokens, float *margins);
float orc_softplus(float x);
void orc_conv1d_step(const float *x, const float *w, const float *bias, float *state,
                     size_t d_inner, size_t d_conv, float *out);
void orc_rmsnorm_seq(const float *x, const float *w, float eps, size_t hidden, float *out);
void orc_selective_scan_step(const float *x, const float *delta, const float *a_log,
                             const float *b, const float *c, const float *d, float *state,
                             float *y, size_t d_inner, size_t d_state);

/* OpenMP threads of the large f32 products (results do not depend on it) */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- sampling (generation/sampler.rs) ---- */
void orc_repetition_penalty(float *logits, size_t n, const uint32_t *hist, size_t nh,
                            float penalty);
void orc_softmax_inplace(float *x, size_t n);
void orc_top_k_filter(float *logits, size_t n, size_t k);
void orc_top_p_filter(float *logits, size_t n, float p);
uint32_t orc_sample_combined(float *logits, size_t n, const uint32_t *hist, size_t nh,
                             float temperature, size_t top_k, float top_p, float rep_penalty,
                             float u);
void orc_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds,
                      uint32_t out[16]);
void orc_stdrng_f32(uint64_t seed, size_t n, float *out);
uint64_t orc_pcg32_step(uint64_t state, uint64_t inc);
uint32_t orc_pcg32_xsh_rr(uint64_t state);

/* ---- ternary linear (quantization/primitives/ternary_linear.rs) ---- */
void orc_ternary_from_f32(const float *w, size_t n, size_t k, uint8_t *blocks);
void orc_ternary_forward(const uint8_t *blocks, size_t n, size_t k, const float *x, size_t m,
                         float *y);


/* ---- Hybrid LFM2.5 decoder, Q4 decode path (models/ssm/hybrid): layer
 * kinds 0 = LIV conv (double-gated), 1 = GQA; every projection a Q4 GEMV,
 * the lm_head tied to the f32 embedding. ---- */
typedef struct {
  size_t hidden, n_layers, vocab, n_heads, n_kv_heads, head_dim, inner, conv_kernel, inter,
      max_seq;
  float eps, rope_theta;
  int conv_bias;
  uint8_t layer_kinds[64];
} orc_hlm_cfg;
typedef struct orc_hlm orc_hlm;
orc_hlm *orc_hlm_create(const orc_hlm_cfg *cfg);
void orc_hlm_destroy(orc_hlm *m);
int orc_hlm_init_synthetic(orc_hlm *m, uint64_t seed_base, float std);
void orc_hlm_reset(orc_hlm *m);
size_t orc_hlm_pos(const orc_hlm *m);
void orc_hlm_conv_step(const float *proj, size_t inner, size_t ck, float *state,
                       const float *w, const float *bias, float *out);
int orc_hlm_decode_one(orc_hlm *m, uint32_t token, float *logits);
int orc_hlm_generate(orc_hlm *m, const uint32_t *prompt, size_t n_prompt, size_t max_new,
                     uint32_t *out_tokens, float *out_margins);

#ifdef __cplusplus
}
#endif
#endif
