/*
 * synapse_hip.h — C ABI of the MI355X (gfx950) `hip` backend for Synapse's
 * quantized-linear hot path.
 *
 * Style follows the reference C header (synapse.h): every entry point returns
 * a syn_status_t, no exception or abort crosses the boundary, all buffers are
 * caller-owned unless a *_create / *_destroy pair says otherwise, and handles
 * are opaque.  Signatures use plain pointers and sizes only.
 *
 * Two layers:
 *   1. Reference-signature entry points (host pointers, synchronous): the
 *      exact functions the reference's Rust FFI binds for this path
 *      (crates/synapse-sys/src/lib.rs), so a build can link this library in
 *      place of libsynapse_zig for them.  Each call uploads its operands.
 *   2. Device-resident API (syn_hip_*): weights repacked once into HBM behind
 *      a handle; activations stay on the device; calls are asynchronous on a
 *      stream (NULL = the library's stream for the current device).
 *
 * Handles are not thread-safe (as the reference's Q4Linear cache and Metal
 * state are not).  Reference paths below are relative to `synapse/`.
 */
#ifndef SYNAPSE_HIP_H
#define SYNAPSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: synapse.h:27-35, same values and meaning ---- */
typedef int32_t syn_status_t;
#define SYN_OK 0
#define SYN_ERR_NULL_PTR 1
#define SYN_ERR_INVALID_ARG 2
#define SYN_ERR_OUT_OF_MEMORY 3
#define SYN_ERR_SHAPE_MISMATCH 4
#define SYN_ERR_NOT_CONTIGUOUS 5
#define SYN_ERR_INVALID_AXIS 6
#define SYN_ERR_INVALID_DIMENSIONS 7
#define SYN_ERR_INTERNAL 8
/* device-side codes (new; >= 100 so the reference's check_status maps them to
 * SynapseError::Unknown, crates/synapse-core/src/lib.rs:50-62) */
#define SYN_ERR_NO_DEVICE 100
#define SYN_ERR_HIP 101
#define SYN_ERR_LAUNCH 102

/* =====================================================================
 * 1. Reference-signature entry points (host pointers, synchronous)
 * =================================================================== */

/* Replaces syn_quantize_per_channel_int8 (synapse.h:341-345,
 * zig/src/ffi/exports.zig:1275-1288).  Zero dims -> SYN_ERR_INVALID_ARG. */
syn_status_t syn_quantize_per_channel_int8(const float *data, size_t channels,
                                           size_t channel_size, int8_t *out,
                                           float *scales);

/* Replaces syn_qgemm_int8 (synapse.h:363-368, exports.zig:1313-1350):
 * C[m,n] = diag(scales_a) (A_i8[m,k] B_i8[k,n]) diag(scales_b), B in the
 * reference's [K,N] layout.  Zero dims -> SYN_OK no-op. */
syn_status_t syn_qgemm_int8(size_t m, size_t n, size_t k, const int8_t *a, size_t lda,
                            const int8_t *b, size_t ldb, float *c, size_t ldc,
                            const float *scales_a, const float *scales_b);

/* Replaces syn_q4_0_gemv (crates/synapse-sys/src/lib.rs:413-419,
 * exports.zig:1614-1628): c[n] = a[k] . dequant(B_q4[n,k]), B in the
 * reference's pack_for_zig format.  k % 32 != 0 -> SYN_ERR_SHAPE_MISMATCH. */
syn_status_t syn_q4_0_gemv(size_t n, size_t k, const float *a, const uint8_t *b_q4,
                           float *c);

/* Replaces syn_sgemm (synapse.h:176-184, exports.zig:725-761): C = op(A) op(B),
 * row-major, trans != 0 uses the transpose; M <= 16 with A as is overwrites C
 * (one f32GemvRow per row), otherwise C accumulates (zero it first), with the
 * reference's per-element chain order (matmul.zig:125-184).  Zero dims ->
 * SYN_OK no-op; null pointers -> SYN_ERR_NULL_PTR. */
syn_status_t syn_sgemm(size_t m, size_t n, size_t k, const float *a, size_t lda, int trans_a,
                       const float *b, size_t ldb, int trans_b, float *c, size_t ldc);

/* The four entry points above under names the reference's static Zig archive
 * (libsynapse_zig.a, which defines the unprefixed ones) does not define, so a
 * binary can link both and reach these. */
syn_status_t syn_hip_quantize_per_channel_int8(const float *data, size_t channels,
                                               size_t channel_size, int8_t *out,
                                               float *scales);
syn_status_t syn_hip_qgemm_int8(size_t m, size_t n, size_t k, const int8_t *a, size_t lda,
                                const int8_t *b, size_t ldb, float *c, size_t ldc,
                                const float *scales_a, const float *scales_b);
syn_status_t syn_hip_q4_0_gemv(size_t n, size_t k, const float *a, const uint8_t *b_q4,
                               float *c);
syn_status_t syn_hip_sgemm(size_t m, size_t n, size_t k, const float *a, size_t lda,
                           int trans_a, const float *b, size_t ldb, int trans_b, float *c,
                           size_t ldc);

/* =====================================================================
 * 2. Device-resident API
 * =================================================================== */

/* -- runtime (no reference counterpart: device bookkeeping) -- */
syn_status_t syn_hip_init(int device);
syn_status_t syn_hip_device_count(int *count);
const char *syn_hip_last_error(void);
syn_status_t syn_hip_malloc(void **dptr, size_t bytes);
syn_status_t syn_hip_free(void *dptr);
syn_status_t syn_hip_memcpy_h2d(void *dst, const void *src, size_t bytes);
syn_status_t syn_hip_memcpy_d2h(void *dst, const void *src, size_t bytes);
syn_status_t syn_hip_memcpy_d2d(void *dst, const void *src, size_t bytes);
syn_status_t syn_hip_memset(void *dst, int value, size_t bytes);
syn_status_t syn_hip_synchronize(void);
syn_status_t syn_hip_stream_create(void **stream);
syn_status_t syn_hip_stream_destroy(void *stream);
syn_status_t syn_hip_stream_synchronize(void *stream);

/* hipEvent pair timing on a stream: elapsed ms between start and stop. */
typedef struct syn_hip_timer_s syn_hip_timer_t;
syn_status_t syn_hip_timer_create(syn_hip_timer_t **timer);
syn_status_t syn_hip_timer_start(syn_hip_timer_t *timer, void *stream);
syn_status_t syn_hip_timer_stop(syn_hip_timer_t *timer, void *stream);
syn_status_t syn_hip_timer_elapsed_ms(syn_hip_timer_t *timer, float *ms);
syn_status_t syn_hip_timer_destroy(syn_hip_timer_t *timer);

/* -- activation quantizer on device: zig/src/ops/quantize.zig:12-47 --
 * x f32 [m, k] (row stride ldx) -> q i8 [m, k] (row stride ldq) + scales[m]. */
syn_status_t syn_hip_quantize_rows(const float *d_x, size_t m, size_t k, size_t ldx,
                                   int8_t *d_q, size_t ldq, float *d_scales, void *stream);

/* -- quantized linear handles --
 * Formats:  INT8 = W8A8 per-row symmetric (QuantizedLinear,
 * quantization/primitives/int8_linear.rs:10-170); Q4_0 = Q4Linear
 * (q4_linear.rs:52-150, pack_for_zig byte format). */
#define SYN_HIP_FMT_INT8 1
#define SYN_HIP_FMT_Q4_0 2
/* GGUF block formats (values defined by weight_loading/gguf.rs:255-487); the
 * reference dequantizes them to f32 at load and runs f32 matmul_t. */
#define SYN_HIP_FMT_Q8_0 3
#define SYN_HIP_FMT_Q4_K 4
#define SYN_HIP_FMT_Q6_K 5
/* TernaryLinear (quantization/primitives/ternary_linear.rs): blocks of 16
 * weights, each an f32 scale and four code bytes (0b00 -1, 0b01 0, 0b10 +1,
 * 0b11 0; weight 4b+j at bits 2j of byte b); f32 activations. */
#define SYN_HIP_FMT_TERNARY 6
/* host weight layouts accepted by syn_hip_qlinear_create for INT8 */
#define SYN_HIP_LAYOUT_KN 0 /* reference QuantizedLinear::weights_int8 [K,N] */
#define SYN_HIP_LAYOUT_NK 1 /* row per output feature [N,K] */
/* Q4_0 block scales read as the reference's dequantize_q4_0 reads them
 * (weight_loading/gguf.rs:294-326 with converter.rs:12-40: subnormal f16
 * deltas come out halved), the f32 map load_gguf_with_raw_q4 builds for the
 * reference's f32 prefill (gguf.rs:59-64).  Any other layout value for Q4_0
 * reads them as the Zig Q4 GEMV does (IEEE f16ToF32, qmatmul.zig:346-371),
 * the path of the raw-block map (RawQ4Tensor) and of Q4Linear. */
#define SYN_HIP_LAYOUT_GGUF_DEQUANT 2

typedef struct syn_hip_qlinear_s syn_hip_qlinear_t;

/* Repack already-quantized host weights once into HBM.
 *   INT8: host_weights int8 in `layout`, host_scales f32[n].
 *   Q4_0: host_weights = pack_for_zig bytes [n, k/32, 18] (= GGUF Q4_0 blocks);
 *         host_scales unused; layout SYN_HIP_LAYOUT_GGUF_DEQUANT or 0.
 *   Q8_0/Q4_K/Q6_K: GGUF block bytes of the row-major [n,k] tensor
 *   (k a multiple of 32 / 256); host_scales unused. */
syn_status_t syn_hip_qlinear_create(int fmt, size_t n, size_t k, const void *host_weights,
                                    const float *host_scales, int layout,
                                    syn_hip_qlinear_t **out);
/* Quantize f32 host weights [n,k] with the reference quantizer of `fmt`
 * (INT8: QuantizedLinear::from_f32, int8_linear.rs:35-70; Q4_0:
 * Q4Linear::from_f32 + pack_for_zig, q4_linear.rs:64-121), then repack. */
syn_status_t syn_hip_qlinear_from_f32(int fmt, size_t n, size_t k, const float *host_w,
                                      syn_hip_qlinear_t **out);
/* y[m,n] = x[m,k] W^T.  INT8 quantizes x per row first (forward,
 * int8_linear.rs:87-117); Q4_0 runs f32 activations (Q4Linear::forward). */
syn_status_t syn_hip_qlinear_forward(syn_hip_qlinear_t *h, size_t m, const float *d_x,
                                     float *d_y, void *stream);
/* No counterpart in the reference: syn_hip_qlinear_forward for INT8 handles
 * that allocates nothing, for callers that cannot call hipMalloc (code under
 * HIP graph capture, tight serving loops).  The quantized activation rows,
 * their scales and the split-K partials live in a fixed 4 MiB device array
 * of the library (one per GPU, held until the process ends); a call whose
 * rows need more returns SYN_ERR_INVALID_ARG.  Every call on a GPU shares
 * that array, so calls that overlap on one GPU (different streams or host
 * threads) race.  Results are bit-identical to syn_hip_qlinear_forward. */
syn_status_t syn_hip_qlinear_forward_noalloc(syn_hip_qlinear_t *h, size_t m, const float *d_x,
                                             float *d_y, void *stream);
/* INT8 only: forward_pre_quantized (int8_linear.rs:139-165). */
syn_status_t syn_hip_qlinear_forward_pre_quantized(syn_hip_qlinear_t *h, size_t m,
                                                   const int8_t *d_xq, size_t ldxq,
                                                   const float *d_sx, float *d_y,
                                                   void *stream);
syn_status_t syn_hip_qlinear_info(const syn_hip_qlinear_t *h, size_t *n, size_t *k, int *fmt,
                                  size_t *weight_bytes);
syn_status_t syn_hip_qlinear_destroy(syn_hip_qlinear_t *h);
/* Benchmark helper: average ms per forward of `iters` launches on the
 * library stream (hipEvents around the batch), activations from d_x/d_xq.
 * INT8 times forward_pre_quantized (d_xq, ldxq, d_sx); other formats time
 * forward (d_x). */
syn_status_t syn_hip_qlinear_time(syn_hip_qlinear_t *h, size_t m, const float *d_x,
                                  const int8_t *d_xq, size_t ldxq, const float *d_sx, float *d_y,
                                  size_t iters, float *avg_ms);
/* Benchmark helper: as syn_hip_qlinear_time, launching round-robin over
 * `count` handles (copies of one matrix in distinct memory, so that a
 * working set larger than the 256 MB Infinity Cache is streamed from HBM)
 * for `rounds` rounds; average ms per launch. */
syn_status_t syn_hip_qlinear_time_set(syn_hip_qlinear_t *const *hs, size_t count, size_t m,
                                      const float *d_x, const int8_t *d_xq, size_t ldxq,
                                      const float *d_sx, float *d_y, size_t rounds,
                                      float *avg_ms);

/* -- INT8 W8A8 causal LM: QuantizedCausalLM (quantization/lm/int8.rs),
 *    device-resident like MetalModelBuffers + gpu_forward_all_layers
 *    (metal/gpu_buffers.rs:79-433, metal/gpu_forward.rs:429-839). -- */
typedef struct {
  uint32_t hidden, n_layers, n_heads, n_kv_heads, head_dim, inter, vocab, max_seq;
  float eps;
  double rope_theta;
} syn_hip_lm_config;

/* -- Sampling (generation/sampler.rs) -------------------------------------- */
/* CombinedSampler (sampler.rs:152-157): repetition penalty -> temperature ->
 * top-k -> top-p -> softmax + categorical draw.  temperature <= 0 or
 * top_k == 1: argmax; top_k == 0 or >= vocab: no top-k; top_p outside
 * (0, 1): no top-p; repetition_penalty within f32::EPSILON of 1: none. */
typedef struct {
  float temperature;
  uint32_t top_k;
  float top_p;
  float repetition_penalty;
} syn_hip_sampler;
/* CombinedSampler::sample_with_history (sampler.rs:161-201) on the device:
 * d_logits f32 [vocab] (not modified), d_history the generated tokens
 * [n_history], u the draw rng.gen::<f32>() the reference would take.  The
 * token goes to d_token (device), asynchronously on `stream`.  d_status
 * (device, nullable) gets 0, or 1 when top-p would have to sort more than
 * 4096 candidates (top-p without top-k over a large vocabulary; the token is
 * then 0).  No counterpart in the reference's C ABI (sampling runs in Rust
 * there). */
syn_status_t syn_hip_sample(const float *d_logits, size_t vocab, const uint32_t *d_history,
                            size_t n_history, const syn_hip_sampler *params, float u,
                            uint32_t *d_token, int *d_status, void *stream);
/* The first n draws of StdRng::seed_from_u64(seed).gen::<f32>() (rand 0.8.5;
 * host computation). */
syn_status_t syn_hip_stdrng_f32(uint64_t seed, size_t n, float *out);


typedef struct syn_hip_qlm_s syn_hip_qlm_t;
syn_status_t syn_hip_qlm_create(const syn_hip_lm_config *cfg, syn_hip_qlm_t **out);
/* embed_tokens [vocab, hidden] f32 (tied: the lm_head is quantized from it) */
syn_status_t syn_hip_qlm_set_embed(syn_hip_qlm_t *m, const float *embed);
/* f32 [out,in] projections of one layer, quantized like quantize_model
 * (int8.rs:78-152). */
syn_status_t syn_hip_qlm_set_layer(syn_hip_qlm_t *m, uint32_t layer, const float *wq,
                                   const float *wk, const float *wv, const float *wo,
                                   const float *wg, const float *wu, const float *wd);
/* Untied lm_head, f32 [vocab, hidden] (int8.rs:125-130); without it the
 * lm_head is quantized from embed_tokens (int8.rs:132-139). */
syn_status_t syn_hip_qlm_set_lm_head(syn_hip_qlm_t *m, const float *w);
/* RMSNorm gains (int8.rs:33-56, applied as apply_norm / apply_headwise_rmsnorm,
 * ops/norm.rs:64-93); all 1.0 until set, NULL leaves a gain as it is.  Per
 * layer: attention and FFN norms [hidden], q/k head norms [head_dim]; final
 * norm [hidden]. */
syn_status_t syn_hip_qlm_set_norms(syn_hip_qlm_t *m, uint32_t layer, const float *attn_norm,
                                   const float *ffn_norm, const float *q_norm,
                                   const float *k_norm);
syn_status_t syn_hip_qlm_set_final_norm(syn_hip_qlm_t *m, const float *norm);
/* Per-head q/k RMSNorm on (1, the default: Qwen3) or off (models whose layers
 * have no q/k norm weights, where the reference skips it, norm.rs:86-88).
 * Before finalize. */
syn_status_t syn_hip_qlm_set_qk_norm(syn_hip_qlm_t *m, int enabled);
/* Synthetic weights: SplitMix64(seed_base + tensor_id) + Box-Muller, tensor
 * id 0 = embed, 1 + 8*layer + {0..6} = q,k,v,o,gate,up,down. */
syn_status_t syn_hip_qlm_init_synthetic(syn_hip_qlm_t *m, uint64_t seed_base, float stddev);
/* Quantize the lm_head, upload RoPE tables; call once after weights. */
syn_status_t syn_hip_qlm_finalize(syn_hip_qlm_t *m);
syn_status_t syn_hip_qlm_reset(syn_hip_qlm_t *m);
/* forward_prefill (int8.rs:593-635) into an empty cache (a fresh ModelState):
 * logits of the last prompt token. */
syn_status_t syn_hip_qlm_forward_prefill(syn_hip_qlm_t *m, const uint32_t *ids, size_t n,
                                         float *host_logits);
/* forward_prefill into the cache as it stands (int8.rs:593-635 with
 * cached_attention_prefill, ops/attention.rs:153-247): the n rows are
 * appended after the cached ones, rotated at positions 0..n-1 and attend
 * among themselves, as in the reference. */
syn_status_t syn_hip_qlm_forward_prefill_append(syn_hip_qlm_t *m, const uint32_t *ids,
                                                size_t n, float *host_logits);
/* KVCache::truncate_to -> syn_kvcache_truncate (kv_cache/cache.rs:307-312,
 * exports.zig:1935-1939, kvcache.zig:109-113): the cache length becomes
 * new_len if that is shorter; contents are kept. */
syn_status_t syn_hip_qlm_truncate(syn_hip_qlm_t *m, size_t new_len);
/* KVCache::current_len (kv_cache/cache.rs:301-304). */
syn_status_t syn_hip_qlm_cache_len(syn_hip_qlm_t *m, size_t *out_len);
/* forward_one (int8.rs:638-709) for `token` at the current cache length. */
syn_status_t syn_hip_qlm_forward_one(syn_hip_qlm_t *m, uint32_t token, float *host_logits);
/* Greedy generate (generation/pipeline.rs:197-278): max_new tokens from one
 * prefill and max_new-1 decode steps, all on device (HIP graph per step);
 * only the tokens are read back.  margins (nullable) gets top1-top2. */
syn_status_t syn_hip_qlm_generate(syn_hip_qlm_t *m, const uint32_t *prompt, size_t n_prompt,
                                  size_t max_new, uint32_t *out_tokens, float *out_margins);
/* Speculative generate (generation/pipeline.rs:281-395, speculative_k = k,
 * max_new_tokens = max_new, the model's sampler settings): per round k draft
 * tokens from forward_one (QuantizedCausalLM has no draft forward,
 * int8.rs:739), truncate to the round's start, verify forward_prefill of
 * [last accepted, drafts], accept all drafts, then a bonus token from
 * forward_one of the last draft when all k were accepted.  The whole loop is
 * enqueued without a host round trip; k = 0 is generate. */
syn_status_t syn_hip_qlm_generate_speculative(syn_hip_qlm_t *m, const uint32_t *prompt,
                                              size_t n_prompt, size_t max_new, size_t k,
                                              uint32_t *out_tokens, float *out_margins);
/* Timed decode: `steps` greedy decode steps after the current state, on the
 * model stream; returns elapsed milliseconds measured with hipEvents. */
syn_status_t syn_hip_qlm_decode_timed(syn_hip_qlm_t *m, size_t steps, float *elapsed_ms);
/* Average duration of the lm_head GEMV launch (the largest decode matvec),
 * timed with a hipEvent pair around each of `iters` launches on the model
 * stream; between launches `flush_bytes` of device memory are overwritten so
 * the 256 MB Infinity Cache does not hold the weights (as in a real step,
 * where the layer weights stream through it in between). */
syn_status_t syn_hip_qlm_time_lm_head(syn_hip_qlm_t *m, size_t iters, size_t flush_bytes,
                                      float *avg_ms);
/* Average duration of the fused decode step's lm_head kernel over `iters`
 * back-to-back launches alternating between the model's weights and a
 * temporary device copy (2 x the weights exceed the Infinity Cache, so every
 * launch streams from HBM); one hipEvent pair around the batch. */
syn_status_t syn_hip_qlm_time_lm_head_rotating(syn_hip_qlm_t *m, size_t iters, float *avg_ms);
/* Benchmark helper: `steps` fused decode steps launched eagerly, every kernel
 * through hipExtLaunchKernelGGL with a start/stop event pair (the dispatch's
 * own start and end timestamps); per kernel kind the average microseconds per
 * launch and the launch count (arrays of SYN_HIP_STEP_KINDS).  The steps
 * advance the model like any decode. */
#define SYN_HIP_STEP_ZERO 0       /* accumulator zeroing */
#define SYN_HIP_STEP_QKV 1        /* residual + RMSNorm + quantize + QKV GEMV */
#define SYN_HIP_STEP_ATTENTION 2  /* head norms, RoPE, KV append, attention */
#define SYN_HIP_STEP_O 3          /* quantize + O GEMV */
#define SYN_HIP_STEP_GATE_UP 4    /* residual + RMSNorm + quantize + gate|up (+ SwiGLU) */
#define SYN_HIP_STEP_DOWN 5       /* (SwiGLU +) quantize + down GEMV */
#define SYN_HIP_STEP_FINAL_NORM 6
#define SYN_HIP_STEP_LM_HEAD 7
#define SYN_HIP_STEP_SELECT 8     /* argmax (or sampling) and state advance */
#define SYN_HIP_STEP_KINDS 9
syn_status_t syn_hip_qlm_time_step_kernels(syn_hip_qlm_t *m, size_t steps, float *avg_us,
                                           uint32_t *launches);
/* Decode-step options (no reference counterpart; both settings compute the
 * same bits).  fused_decode = 1 (default when the shape fits the fused
 * kernels' LDS rows): five kernels per layer, each a split-K GEMV whose
 * prologue forms its own input activation; 0: one kernel per reference op.
 * graph_replay = 1 (default): each decode step is a replayed HIP graph; 0:
 * kernels are launched eagerly (for profilers that cannot follow graphs). */
syn_status_t syn_hip_qlm_set_options(syn_hip_qlm_t *m, int fused_decode, int graph_replay);
/* Sampling for generate / decode steps: the CombinedSampler of
 * generation/sampler.rs:152-201 (NULL params: greedy, the default), with the
 * draws of StdRng::seed_from_u64(seed) (pipeline.rs:162-165).  The draws are
 * generated on the host at this call and uploaded once; every step samples
 * on the device.  The margin history then holds the chosen token's
 * probability (0 on the greedy route). */
syn_status_t syn_hip_qlm_set_sampler(syn_hip_qlm_t *m, const syn_hip_sampler *params,
                                     uint64_t seed);
syn_status_t syn_hip_qlm_destroy(syn_hip_qlm_t *m);

/* -- GGUF files (weight_loading/gguf.rs:49-151, 551-591): a read-only
 *    mapping and its tensor table, so block bytes go to the device without
 *    being dequantized on the host.  Versions 2 and 3; tensor data aligned to
 *    32 bytes as the reference assumes.  dims[0] is the fastest axis (a
 *    weight of N rows over K inputs has dims {K, N}).  Pointers returned
 *    point into the mapping and stay valid until syn_hip_gguf_close. -- */
#define SYN_HIP_GGML_F32 0
#define SYN_HIP_GGML_F16 1
#define SYN_HIP_GGML_Q4_0 2
#define SYN_HIP_GGML_Q4_1 3
#define SYN_HIP_GGML_Q8_0 8
#define SYN_HIP_GGML_Q4_K 12
#define SYN_HIP_GGML_Q6_K 14
#define SYN_HIP_GGML_BF16 30 /* read here; the reference rejects it */
/* metadata value types */
#define SYN_HIP_GGUF_UINT8 0
#define SYN_HIP_GGUF_INT8 1
#define SYN_HIP_GGUF_UINT16 2
#define SYN_HIP_GGUF_INT16 3
#define SYN_HIP_GGUF_UINT32 4
#define SYN_HIP_GGUF_INT32 5
#define SYN_HIP_GGUF_FLOAT32 6
#define SYN_HIP_GGUF_BOOL 7
#define SYN_HIP_GGUF_STRING 8
#define SYN_HIP_GGUF_ARRAY 9
#define SYN_HIP_GGUF_UINT64 10
#define SYN_HIP_GGUF_INT64 11
#define SYN_HIP_GGUF_FLOAT64 12
typedef struct syn_hip_gguf_s syn_hip_gguf_t;
/* parse_gguf (gguf.rs:75-151): bad magic, version, shapes, unsupported types
 * or tensors outside the file -> SYN_ERR_INVALID_ARG */
syn_status_t syn_hip_gguf_open(const char *path, syn_hip_gguf_t **out);
syn_status_t syn_hip_gguf_tensor_count(const syn_hip_gguf_t *g, size_t *n);
syn_status_t syn_hip_gguf_find(const syn_hip_gguf_t *g, const char *name, size_t *index);
/* any output pointer may be NULL; dims4 receives 4 values (unused = 1) */
syn_status_t syn_hip_gguf_tensor_info(const syn_hip_gguf_t *g, size_t index, const char **name,
                                      uint32_t *ggml_type, uint32_t *n_dims, uint64_t *dims4,
                                      uint64_t *nbytes, const void **data);
/* scalar metadata (integers of any width as u64, floats as double) */
syn_status_t syn_hip_gguf_meta_u64(const syn_hip_gguf_t *g, const char *key, uint64_t *value);
syn_status_t syn_hip_gguf_meta_f64(const syn_hip_gguf_t *g, const char *key, double *value);
syn_status_t syn_hip_gguf_meta_str(const syn_hip_gguf_t *g, const char *key, const char **value);
syn_status_t syn_hip_gguf_close(syn_hip_gguf_t *g);
/* numel f32 values of tensor `index` as the reference's parse_gguf returns
 * them (gguf.rs:208-233): F32, F16 (converter.rs:12-40), Q4_0 (element 2i =
 * low nibble, 2i+1 = high), Q4_1, Q8_0, Q4_K, Q6_K; also BF16 (type 30). */
syn_status_t syn_hip_gguf_to_f32(const syn_hip_gguf_t *g, size_t index, float *out);

/* -- safetensors (weight_loading/safetensors.rs:21-302): a file, or a
 *    directory holding model.safetensors.index.json (the shards it lists,
 *    only the tensors in its weight_map, each from its named shard) or one
 *    .safetensors file.  dtypes as the reference: F32, F16, BF16, I64, I32,
 *    U8 (others -> SYN_ERR_INVALID_ARG at open).  shape8 is row-major
 *    (slowest axis first, unused = 0); pointers point into the mapping and
 *    stay valid until syn_hip_safetensors_close. -- */
#define SYN_HIP_ST_F32 0
#define SYN_HIP_ST_F16 1
#define SYN_HIP_ST_BF16 2
#define SYN_HIP_ST_I64 3
#define SYN_HIP_ST_I32 4
#define SYN_HIP_ST_U8 5
typedef struct syn_hip_safetensors_s syn_hip_safetensors_t;
syn_status_t syn_hip_safetensors_open(const char *path, syn_hip_safetensors_t **out);
syn_status_t syn_hip_safetensors_tensor_count(const syn_hip_safetensors_t *st, size_t *n);
syn_status_t syn_hip_safetensors_find(const syn_hip_safetensors_t *st, const char *name,
                                      size_t *index);
syn_status_t syn_hip_safetensors_tensor_info(const syn_hip_safetensors_t *st, size_t index,
                                             const char **name, uint32_t *dtype,
                                             uint32_t *n_dims, uint64_t *shape8,
                                             uint64_t *nbytes, const void **data);
/* a string of the header's __metadata__ */
syn_status_t syn_hip_safetensors_meta(const syn_hip_safetensors_t *st, const char *key,
                                      const char **value);
/* numel f32 values as parse_safetensors converts them (F16 and BF16 by
 * converter.rs:12-46, integers cast) */
syn_status_t syn_hip_safetensors_to_f32(const syn_hip_safetensors_t *st, size_t index,
                                        float *out);
/* The Q4_0 triple expand_q4_tensors reads (safetensors.rs:80-170:
 * <base>.q4_nibbles U8 [rows, bpr, 16], <base>.q4_scales F16 [rows, bpr],
 * <base>.q4_orig_cols I64 [1]) as pack_for_zig bytes [rows, bpr, 18] without
 * dequantizing.  packed may be NULL to query rows and cols (orig_cols). */
syn_status_t syn_hip_safetensors_q4_pack(const syn_hip_safetensors_t *st, const char *base,
                                         uint8_t *packed, size_t *rows, size_t *cols);
syn_status_t syn_hip_safetensors_close(syn_hip_safetensors_t *st);

/* Linear layers straight from file bytes (no dequantization):
 * a 2-D GGUF tensor of type Q4_0 (the reference's RawQ4Tensor, gguf.rs:49-57),
 * Q8_0, Q4_K or Q6_K, dims {K, N}; or a safetensors Q4_0 triple whose
 * orig_cols is a multiple of 32. */
syn_status_t syn_hip_qlinear_from_gguf(const syn_hip_gguf_t *g, const char *name,
                                       syn_hip_qlinear_t **out);
syn_status_t syn_hip_qlinear_from_safetensors_q4(const syn_hip_safetensors_t *st,
                                                 const char *base, syn_hip_qlinear_t **out);

/* -- f32 causal LM over GGUF-block weights: CausalLM (models/lm/causal_lm.rs:
 *    195-278, decoder_layer.rs:51-138, 590-730), the reference path for models
 *    whose weights are Q8_0 / Q4_K / Q6_K (dequantized at load there, decoded
 *    in the kernels here).  Projections 0..6 = q,k,v,o,gate,up,down. -- */
typedef struct {
  syn_hip_lm_config base;
  int32_t fmt_qkv, fmt_o, fmt_gate_up, fmt_down, fmt_lm_head; /* SYN_HIP_FMT_Q* */
  int32_t qk_norm; /* 1: per-head q/k RMSNorm (Qwen3), 0: none (LLaMA) */
} syn_hip_klm_config;

typedef struct syn_hip_klm_s syn_hip_klm_t;
syn_status_t syn_hip_klm_create(const syn_hip_klm_config *cfg, syn_hip_klm_t **out);
syn_status_t syn_hip_klm_set_embed(syn_hip_klm_t *m, const float *embed);
syn_status_t syn_hip_klm_set_proj(syn_hip_klm_t *m, uint32_t layer, int proj,
                                  const uint8_t *gguf_bytes);
syn_status_t syn_hip_klm_set_lm_head(syn_hip_klm_t *m, const uint8_t *gguf_bytes);
/* RMSNorm gains (decoder_layer.rs:590-730, causal_lm.rs:262-270); every gain
 * is 1.0 until set.  Per layer: attention and FFN norms [hidden], q/k head
 * norms [head_dim] (used when qk_norm = 1); a NULL pointer leaves that gain
 * as it is.  The final norm is [hidden]. */
syn_status_t syn_hip_klm_set_norms(syn_hip_klm_t *m, uint32_t layer, const float *attn_norm,
                                   const float *ffn_norm, const float *q_norm,
                                   const float *k_norm);
syn_status_t syn_hip_klm_set_final_norm(syn_hip_klm_t *m, const float *norm);
/* Every weight of the model from an open GGUF file (engine/loading.rs:55-80
 * with load_gguf, gguf.rs:43-151): projections, norms, embedding and lm_head
 * by llama.cpp names (blk.N.attn_q.weight, token_embd.weight, output.weight,
 * ...) or the HuggingFace names of the reference's weight map
 * (model.layers.N.self_attn.q_proj.weight, ...).  Projection and lm_head
 * tensors must hold the configured block format with dims {K, N}; they are
 * uploaded as stored.  Norms and the embedding may be F32, F16, Q8_0, Q4_K
 * or Q6_K (converted to f32 as the reference does).  Missing norms stay 1.0;
 * a missing lm_head is tied to token_embd (which must then hold the lm_head
 * format).  Call syn_hip_klm_finalize afterwards. */
syn_status_t syn_hip_klm_load_gguf(syn_hip_klm_t *m, const syn_hip_gguf_t *g);
/* INT8 decoder weights from a file (engine/loading.rs:29-130 with
 * quantize_model, int8.rs:78-152): HuggingFace names
 * (model.layers.N.self_attn.q_proj.weight, ..., fused qkv_proj / gate_up_proj
 * split by the q/k/v widths, weight_map.rs:780-829) or llama.cpp GGUF names
 * (blk.N.attn_q.weight, ...); any tensor type the container's to_f32 reads,
 * converted as the reference does, then quantized.  Head norms are on when
 * layer 0 has q_norm weights; lm_head is tied when the file has none.  Call
 * syn_hip_qlm_finalize afterwards. */
syn_status_t syn_hip_qlm_load_gguf(syn_hip_qlm_t *m, const syn_hip_gguf_t *g);
syn_status_t syn_hip_qlm_load_safetensors(syn_hip_qlm_t *m, const syn_hip_safetensors_t *st);
/* Synthetic weights (seed spec as syn_hip_qlm_init_synthetic; untied lm_head
 * is tensor id 1 + 8*n_layers), encoded with the library's block encoder. */
syn_status_t syn_hip_klm_init_synthetic(syn_hip_klm_t *m, uint64_t seed_base, float stddev);
syn_status_t syn_hip_klm_finalize(syn_hip_klm_t *m);
syn_status_t syn_hip_klm_reset(syn_hip_klm_t *m);
syn_status_t syn_hip_klm_forward_prefill(syn_hip_klm_t *m, const uint32_t *ids, size_t n,
                                         float *host_logits);
syn_status_t syn_hip_klm_forward_one(syn_hip_klm_t *m, uint32_t token, float *host_logits);
syn_status_t syn_hip_klm_generate(syn_hip_klm_t *m, const uint32_t *prompt, size_t n_prompt,
                                  size_t max_new, uint32_t *out_tokens, float *out_margins);
/* forward_prefill into the cache as it stands (causal_lm.rs:195-239 with
 * cached_attention_prefill, ops/attention.rs:153-247); truncate_to and
 * current_len of the cache (kv_cache/cache.rs:301-312, kvcache.zig:109-113). */
syn_status_t syn_hip_klm_forward_prefill_append(syn_hip_klm_t *m, const uint32_t *ids,
                                                size_t n, float *host_logits);
syn_status_t syn_hip_klm_truncate(syn_hip_klm_t *m, size_t new_len);
syn_status_t syn_hip_klm_cache_len(syn_hip_klm_t *m, size_t *out_len);
/* CausalLM::forward_one_draft (causal_lm.rs:283-323): the first n_layers
 * layers, zero K/V rows appended to the others, final norm, lm_head. */
syn_status_t syn_hip_klm_forward_one_draft(syn_hip_klm_t *m, uint32_t token, size_t n_layers,
                                           float *host_logits);
/* Greedy speculative generate (generation/pipeline.rs:281-395): k drafts per
 * round from forward_one_draft with draft_layers layers (0: n_layers / 3,
 * pipeline.rs:28, 295-299), truncate, verify forward_prefill, accept all,
 * bonus token; enqueued without a host round trip.  k = 0 is generate. */
syn_status_t syn_hip_klm_generate_speculative(syn_hip_klm_t *m, const uint32_t *prompt,
                                              size_t n_prompt, size_t max_new, size_t k,
                                              size_t draft_layers, uint32_t *out_tokens,
                                              float *out_margins);
/* hipEvent timing of one prefill of `prompt` and `steps` greedy decode steps. */
syn_status_t syn_hip_klm_time(syn_hip_klm_t *m, const uint32_t *prompt, size_t n_prompt,
                              size_t steps, float *prefill_ms, float *decode_ms);
/* Decode-step form: fused != 0 (the default) runs five kernels per layer
 * with tree-ordered sums (models whose shapes the fused step supports;
 * others keep the op-by-op step), fused == 0 one kernel per reference op;
 * graph != 0 (the default) replays a captured HIP graph, graph == 0 launches
 * the same kernels eagerly (for profilers that do not follow graph launches). */
syn_status_t syn_hip_klm_set_options(syn_hip_klm_t *m, int fused, int graph);
syn_status_t syn_hip_klm_destroy(syn_hip_klm_t *m);

/* -- INT8 Mamba: QuantizedMambaModel (quantization/ssm/int8_mamba.rs:21-224).
 *    in_proj/out_proj W8A8 INT8, x_proj/dt_proj/lm_head f32 (tied to the
 *    embedding), selective scan as in zig/src/ops/selective_scan.zig:30-90.
 *    int8_xdt = 1 also runs x_proj and dt_proj as INT8 W8A8 (no reference
 *    counterpart; BASELINE config 5's variant).  max_tokens bounds prompt +
 *    generated tokens of one sequence. -- */
typedef struct {
  uint32_t d_model, d_inner, d_state, d_conv, dt_rank, n_layers, vocab, max_tokens;
  float eps;
  int32_t int8_xdt;
} syn_hip_mamba_config;

typedef struct syn_hip_mamba_s syn_hip_mamba_t;
syn_status_t syn_hip_mamba_create(const syn_hip_mamba_config *cfg, syn_hip_mamba_t **out);
syn_status_t syn_hip_mamba_init_synthetic(syn_hip_mamba_t *m, uint64_t seed_base, float stddev);
/* QuantizedMambaModel::prefill (per-token recurrence, :177-203) */
syn_status_t syn_hip_mamba_prefill(syn_hip_mamba_t *m, const uint32_t *ids, size_t n,
                                   float *host_logits);
/* QuantizedMambaModel::decode_one (:205-224) */
syn_status_t syn_hip_mamba_decode_one(syn_hip_mamba_t *m, uint32_t token, float *host_logits);
syn_status_t syn_hip_mamba_generate(syn_hip_mamba_t *m, const uint32_t *prompt, size_t n_prompt,
                                    size_t max_new, uint32_t *out_tokens, float *out_margins);
syn_status_t syn_hip_mamba_decode_timed(syn_hip_mamba_t *m, size_t steps, float *elapsed_ms);
/* Token step form: fused split-K GEMV kernels whose prologues form their own
 * inputs (fused != 0, the default when the shapes fit) or one kernel per
 * reference op; HIP graph replay (graph != 0, the default) or eager launches.
 * Both forms compute the same float operations. */
syn_status_t syn_hip_mamba_set_options(syn_hip_mamba_t *m, int fused, int graph);
syn_status_t syn_hip_mamba_destroy(syn_hip_mamba_t *m);

/* -- Hybrid LFM2.5 decoder, Q4 decode path: HybridModel::decode_one
 *    (models/ssm/hybrid/model.rs:240-290) over LIV conv and GQA layers
 *    (layer.rs:593-654, 878-954, 1055-1078) after quantize_for_decode: every
 *    projection a Q4_0 GEMV (q4_0GemvRow), the lm_head tied to the f32
 *    embedding.  layer_kinds[l]: 0 = LIV conv (double-gated, in_proj rows
 *    [B | C | x]), 1 = GQA with q/k head norms.  The reference's Metal decode
 *    counterpart is metal/hybrid_gpu_forward.rs:16 (hybrid_forward_all_layers);
 *    its prompt goes through the CPU f32 forward first, this decoder feeds a
 *    prompt through the decode step.  max_seq bounds prompt + generated
 *    tokens (<= 32768). -- */
typedef struct {
  uint32_t hidden, n_layers, vocab, n_heads, n_kv_heads, head_dim, inner, conv_kernel, inter,
      max_seq;
  float eps, rope_theta;
  int32_t conv_bias;
  uint8_t layer_kinds[64];
} syn_hip_hlm_config;

typedef struct syn_hip_hlm_s syn_hip_hlm_t;
syn_status_t syn_hip_hlm_create(const syn_hip_hlm_config *cfg, syn_hip_hlm_t **out);
/* synthetic weights (the oracle's orc_hlm_init_synthetic spec) */
syn_status_t syn_hip_hlm_init_synthetic(syn_hip_hlm_t *m, uint64_t seed_base, float stddev);
/* conv states to zero, position 0 */
syn_status_t syn_hip_hlm_reset(syn_hip_hlm_t *m);
syn_status_t syn_hip_hlm_position(syn_hip_hlm_t *m, size_t *pos);
/* HybridModel::decode_one: logits of `token` at the current position */
syn_status_t syn_hip_hlm_decode_one(syn_hip_hlm_t *m, uint32_t token, float *host_logits);
/* decode_one over ids[0..n); host_logits (may be null) of the last */
syn_status_t syn_hip_hlm_prefill(syn_hip_hlm_t *m, const uint32_t *ids, size_t n,
                                 float *host_logits);
/* greedy: the prompt through decode_one, then max_new argmax tokens
 * (last maximum wins) with their top1 - top2 margins */
syn_status_t syn_hip_hlm_generate(syn_hip_hlm_t *m, const uint32_t *prompt, size_t n_prompt,
                                  size_t max_new, uint32_t *out_tokens, float *out_margins);
/* hipEvent time of `steps` greedy decode steps from the current state */
syn_status_t syn_hip_hlm_decode_timed(syn_hip_hlm_t *m, size_t steps, float *elapsed_ms);
/* fused != 0 (the default): four kernels per LIV conv layer and five per
 * GQA layer when the shapes fit
 * (hidden 256..2048 in whole 256s, inner, inter, n_heads * head_dim multiples
 * of 256, head_dim 16..128, n_heads / n_kv_heads <= 8, IEEE block scales):
 * the Q4_0 rows of split-K workgroups add into fixed-point accumulators,
 * RMSNorm, SwiGLU and the attention combine run in the GEMVs' prologues and
 * epilogues, the lm_head carries a per-panel top-2; else the op-by-op step.
 * Both are graded against the reference by tolerance.
 * graph != 0 (the default): replay a captured HIP graph of the step */
syn_status_t syn_hip_hlm_set_options(syn_hip_hlm_t *m, int fused, int graph);
/* *active = 1 when decode steps run the fused form */
syn_status_t syn_hip_hlm_fused_active(syn_hip_hlm_t *m, int *active);
syn_status_t syn_hip_hlm_destroy(syn_hip_hlm_t *m);

/* -- harness helpers (no reference counterpart) -- */
/* Encode f32 [n,k] into Q8_0 / Q4_K / Q6_K block bytes.  The reference has no
 * encoder for these formats (only dequantizers); any encoding is valid since
 * its dequantizer defines the values.  host_out holds n*(k/32)*34 (Q8_0),
 * n*(k/256)*144 (Q4_K) or n*(k/256)*210 (Q6_K) bytes. */
syn_status_t syn_hip_kquant_encode(int fmt, size_t n, size_t k, const float *host_w,
                                   uint8_t *host_out);
/* Host dequantizer of the same formats, as the reference converts them at
 * load (gguf.rs:255-288 Q8_0, 375-438 Q4_K, 440-487 Q6_K): nblocks blocks ->
 * nblocks*32 (Q8_0) or nblocks*256 values.  The K-quant model's GGUF loader
 * uses it for embeddings stored in a block format. */
syn_status_t syn_hip_kquant_decode(int fmt, size_t nblocks, const uint8_t *host_blocks,
                                   float *host_out);
/* Diagnostic: y[i] = the device expf that SiLU and softmax use (bit-identical
 * to glibc expf, which Rust's f32::exp calls on Linux). */
syn_status_t syn_hip_eval_expf(const float *d_x, float *d_y, size_t n, void *stream);
/* Achievable-peak probes: kind 0 = dense v_mfma_f32_16x16x32_f16 loop,
 * 1 = dense v_mfma_i32_16x16x64_i8 loop, 2 = dense v_mfma_f32_32x32x16_f16
 * loop, 3 = dense v_mfma_i32_32x32x32_i8 loop (TFLOP/s or TOP/s, 8 waves per
 * SIMD);
 * HBM streaming read of `bytes` (best of 3 after a warm-up, GB/s). */
syn_status_t syn_hip_probe_mfma(int kind, size_t iters, double *tflops);
syn_status_t syn_hip_probe_hbm_read(size_t bytes, double *gb_s);
/* The device's reference-order sequential sum of n <= 16384 host values:
 * out5[0] = one lane's chain, out5[1] = the wave-cooperative chain of the
 * attention's softmax sum, out5[2] = that chain's clocks, out5[3] = the
 * long-row wave chain of the Mamba norms, out5[4] = its clocks (a check of
 * the summation order). */
syn_status_t syn_hip_probe_seq_sum(const float *host, size_t n, float *out5);
/* What ordering the decode step's dependency levels costs: the graph replay
   of n dependent tiny kernels of `wgs` workgroups (us per kernel), and nbar
   grid barriers among `wgs` <= CU-count co-resident workgroups of one
   cooperative launch (mode 0: one arrival counter; mode 1: eight counters
   and a top counter), us per barrier; every wait is bounded and a timed-out
   wait is counted in *timeouts instead of hanging.  No reference
   counterpart (harness measurements). */
syn_status_t syn_hip_probe_graph_floor(int n, int wgs, double *us_per_kernel);
syn_status_t syn_hip_probe_grid_barrier(int wgs, int mode, int nbar, double *us_per_barrier,
                                        int *timeouts);
/* SplitMix64 + Box-Muller (f64, cast to f32) into host memory. */
syn_status_t syn_hip_fill_normal(float *host_dst, size_t n, uint64_t seed, float stddev);

#ifdef __cplusplus
}
#endif
#endif /* SYNAPSE_HIP_H */
