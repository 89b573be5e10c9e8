// f32 causal LM over GGUF-block weights (Q8_0 / Q4_K / Q6_K) on the device:
// the reference's CausalLM (models/lm/causal_lm.rs:195-278,
// decoder_layer.rs:51-138, 590-730) for the formats it dequantizes at load,
// with the weights kept in their block format in HBM and decoded in the
// GEMV/GEMM kernels.  Same greedy loop and HIP-graph decode step as the INT8
// driver; activations stay f32 between layers (no activation quantization
// on this path, as in the reference).
#include <algorithm>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "decode_fused.hpp"
#include "klm_fused.hpp"
#include "kquant.hpp"
#include "layer_ops.hpp"

using namespace syn;

struct syn_hip_klm_s {
  syn_hip_klm_config c{};
  size_t h = 0, hd = 0, qd = 0, kvd = 0, inter = 0, L = 0, vocab = 0, S = 0, n_qkv = 0;
  struct Layer {
    QLinearKQ qkv, o, gu, down;
    std::vector<std::vector<uint8_t>> pending;  // q,k,v,gate,up bytes until stacked
    int have = 0;                               // bitmask of the 7 projections
  };
  std::vector<Layer> layers;
  QLinearKQ lm_head;
  bool have_lm = false, have_embed = false;
  DevBuf embed, rope_cos, rope_sin, kc, vc;
  // RMSNorm gains: attention and FFN norms [L][h], q/k head norms [L][hd],
  // final norm [h] (1.0 until set)
  DevBuf attn_nw, ffn_nw, q_nw, k_nw, final_nw;
  DevBuf x, normed, qkv, qrot, attn, o, gu, hbuf, down, logits, scores;
  DevBuf pv, pi, pv2, state, history, mhist, ids;
  hipStream_t stream = nullptr;
  hipGraphExec_t graph = nullptr;
  bool finalized = false;
  bool use_graph = true;  // replay the captured decode step, else launch eagerly
  bool use_fused = true;  // five-kernel decode layers (klm_fused.hip) when the model fits
  // fused decode step: split plans, the fixed-point residual r [h] and QKV
  // accumulator [n_qkv], attention chunk partials, lm_head per-panel top-2
  bool fused_ok = false;
  KqfPlan fp_qkv, fp_o, fp_gu, fp_down, fp_lm;
  DevBuf f_r, f_qkv, f_ao, f_aml, f_pv, f_pi, f_pv2;

  ~syn_hip_klm_s() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (draft_graph) (void)hipGraphExecDestroy(draft_graph);
    if (stream) (void)hipStreamDestroy(stream);
  }
  // per-layer KV caches in the decode attention's tiled layout (layer_ops.hpp)
  size_t k_elems() const { return kv_k_elems((int)(kvd / hd), (int)hd, (int)S); }
  size_t v_elems() const { return kv_v_elems((int)(kvd / hd), (int)hd, (int)S); }
  float *kc_l(size_t l) { return kc.as<float>() + l * k_elems(); }
  float *vc_l(size_t l) { return vc.as<float>() + l * v_elems(); }
  StepState *st() { return state.as<StepState>(); }
  int fmt_of(int proj) const {
    if (proj <= 2) return c.fmt_qkv;
    if (proj == 3) return c.fmt_o;
    if (proj <= 5) return c.fmt_gate_up;
    return c.fmt_down;
  }
  void proj_shape(int proj, size_t *n, size_t *k) const {
    const size_t rows[7] = {qd, kvd, kvd, h, inter, inter, h};
    const size_t cols[7] = {h, h, h, qd, h, h, inter};
    *n = rows[proj];
    *k = cols[proj];
  }
  size_t proj_bytes(int proj) const {
    size_t n, k;
    proj_shape(proj, &n, &k);
    const int f = fmt_of(proj);
    return n * (k / kq_block_elems(f)) * kq_block_bytes(f);
  }

  syn_status_t alloc_all() {
    const size_t T = S;
    SYN_TRY(rope_cos.alloc(S * (hd / 2) * 4));
    SYN_TRY(rope_sin.alloc(S * (hd / 2) * 4));
    SYN_TRY(kc.alloc(L * k_elems() * 4));
    SYN_TRY(vc.alloc(L * v_elems() * 4));
    SYN_TRY(x.alloc(T * h * 4));
    SYN_TRY(normed.alloc(T * h * 4));
    SYN_TRY(qkv.alloc(T * n_qkv * 4));
    SYN_TRY(qrot.alloc(T * qd * 4));
    SYN_TRY(attn.alloc(T * qd * 4));
    SYN_TRY(o.alloc(T * h * 4));
    SYN_TRY(gu.alloc(T * 2 * inter * 4));
    SYN_TRY(hbuf.alloc(T * inter * 4));
    SYN_TRY(down.alloc(T * h * 4));
    SYN_TRY(logits.alloc(vocab * 4));
    SYN_TRY(scores.alloc(c.base.n_heads * S * 4));
    SYN_TRY(pv.alloc(256 * 4));
    SYN_TRY(pi.alloc(256 * 4));
    SYN_TRY(pv2.alloc(256 * 4));
    SYN_TRY(state.alloc(sizeof(StepState)));
    SYN_TRY(history.alloc((S + 1) * 4));
    SYN_TRY(mhist.alloc((S + 1) * 4));
    SYN_TRY(ids.alloc(S * 4));
    std::vector<float> one(std::max(h, hd), 1.0f);
    SYN_TRY(attn_nw.alloc(L * h * 4));
    SYN_TRY(ffn_nw.alloc(L * h * 4));
    SYN_TRY(q_nw.alloc(L * hd * 4));
    SYN_TRY(k_nw.alloc(L * hd * 4));
    SYN_TRY(final_nw.alloc(h * 4));
    for (size_t l = 0; l < L; l++) {
      SYN_HIP(hipMemcpy(attn_nw.as<float>() + l * h, one.data(), h * 4, hipMemcpyHostToDevice));
      SYN_HIP(hipMemcpy(ffn_nw.as<float>() + l * h, one.data(), h * 4, hipMemcpyHostToDevice));
      SYN_HIP(hipMemcpy(q_nw.as<float>() + l * hd, one.data(), hd * 4, hipMemcpyHostToDevice));
      SYN_HIP(hipMemcpy(k_nw.as<float>() + l * hd, one.data(), hd * 4, hipMemcpyHostToDevice));
    }
    SYN_HIP(hipMemcpy(final_nw.p, one.data(), h * 4, hipMemcpyHostToDevice));
    SYN_HIP(hipMemset(kc.p, 0, kc.bytes));
    SYN_HIP(hipMemset(vc.p, 0, vc.bytes));
    return SYN_OK;
  }

  syn_status_t set_proj(size_t l, int proj, const uint8_t *bytes) {
    Layer &Ly = layers[l];
    const size_t nbytes = proj_bytes(proj);
    if (proj == 3) {
      SYN_TRY(Ly.o.upload(fmt_of(3), bytes, h, qd));
    } else if (proj == 6) {
      SYN_TRY(Ly.down.upload(fmt_of(6), bytes, h, inter));
    } else {
      const int slot = proj <= 2 ? proj : proj - 1;  // q,k,v,gate,up -> 0..4
      Ly.pending[slot].assign(bytes, bytes + nbytes);
    }
    Ly.have |= 1 << proj;
    if ((Ly.have & 7) == 7 && !Ly.pending[0].empty()) {  // stack q|k|v rows
      std::vector<uint8_t> cat;
      for (int t = 0; t < 3; t++) cat.insert(cat.end(), Ly.pending[t].begin(), Ly.pending[t].end());
      SYN_TRY(Ly.qkv.upload(fmt_of(0), cat.data(), n_qkv, h));
      for (int t = 0; t < 3; t++) std::vector<uint8_t>().swap(Ly.pending[t]);
    }
    if ((Ly.have & 0x30) == 0x30 && !Ly.pending[3].empty()) {  // stack gate|up rows
      std::vector<uint8_t> cat(Ly.pending[3]);
      cat.insert(cat.end(), Ly.pending[4].begin(), Ly.pending[4].end());
      SYN_TRY(Ly.gu.upload(fmt_of(4), cat.data(), 2 * inter, h));
      for (int t = 3; t < 5; t++) std::vector<uint8_t>().swap(Ly.pending[t]);
    }
    return SYN_OK;
  }

  // cache_off (prefill only): cache row of the first of `rows` tokens
  syn_status_t layer(size_t l, int rows, bool prefill, hipStream_t s, int cache_off = 0) {
    Layer &Ly = layers[l];
    const float eps = c.base.eps;
    const int nh = (int)c.base.n_heads, nkv = (int)c.base.n_kv_heads;
    const float *qn = c.qk_norm ? q_nw.as<float>() + l * hd : nullptr;
    const float *kn = c.qk_norm ? k_nw.as<float>() + l * hd : nullptr;
    SYN_TRY(launch_rmsnorm_quant(x.as<float>(), l == 0 ? nullptr : down.as<float>(),
                                 attn_nw.as<float>() + l * h, eps, rows, (int)h, nullptr, 0,
                                 nullptr, normed.as<float>(), s));
    SYN_TRY(Ly.qkv.gemv(rows, normed.as<float>(), h, qkv.as<float>(), n_qkv, s));
    if (!prefill && fused_attention_fits((int)hd, (int)S)) {
      // one kernel per query head: head norms, RoPE, KV append and attention
      RowSrc src;
      src.f = qkv.as<float>();
      SYN_TRY(launch_fused_attention(src, nh, nkv, (int)hd, qn, kn, eps, rope_cos.as<float>(),
                                     rope_sin.as<float>(), st(), kc_l(l), vc_l(l), (int)S,
                                     scores.as<float>(), attn.as<float>(), s));
    } else {
      SYN_TRY(launch_qk_norm_rope_kv(qkv.as<float>(), (int)n_qkv, rows, nh, nkv, (int)hd, qn, kn,
                                     eps, rope_cos.as<float>(), rope_sin.as<float>(),
                                     prefill ? nullptr : &st()->pos, 0, qrot.as<float>(),
                                     kc_l(l), vc_l(l), (int)S, s, prefill ? cache_off : 0));
      if (prefill)
        SYN_TRY(launch_attention_prefill_tol(qrot.as<float>(), kc_l(l), vc_l(l), rows, nh, nkv,
                                             (int)hd, (int)S, attn.as<float>(), s, cache_off));
      else
        SYN_TRY(launch_attention_decode(qrot.as<float>(), kc_l(l), vc_l(l), &st()->pos, nh, nkv,
                                        (int)hd, scores.as<float>(), (int)S, attn.as<float>(),
                                        s));
    }
    SYN_TRY(Ly.o.gemv(rows, attn.as<float>(), qd, o.as<float>(), h, s));
    SYN_TRY(launch_rmsnorm_quant(x.as<float>(), o.as<float>(), ffn_nw.as<float>() + l * h, eps,
                                 rows, (int)h, nullptr, 0, nullptr, normed.as<float>(), s));
    SYN_TRY(Ly.gu.gemv(rows, normed.as<float>(), h, gu.as<float>(), 2 * inter, s));
    SYN_TRY(launch_swiglu_f32(gu.as<float>(), (int)(2 * inter), rows, (int)inter,
                              hbuf.as<float>(), (int)inter, s));
    SYN_TRY(Ly.down.gemv(rows, hbuf.as<float>(), inter, down.as<float>(), h, s));
    return SYN_OK;
  }

  syn_status_t head(int row, int add_pos, hipStream_t s) {
    float *xr = x.as<float>() + (size_t)row * h;
    const float *dr = down.as<float>() + (size_t)row * h;
    SYN_TRY(launch_rmsnorm_quant(xr, dr, final_nw.as<float>(), c.base.eps, 1, (int)h, nullptr, 0,
                                 nullptr, normed.as<float>(), s));
    SYN_TRY(lm_head.gemv(1, normed.as<float>(), h, logits.as<float>(), vocab, s));
    SYN_TRY(launch_argmax(logits.as<float>(), (int)vocab, pv.as<float>(), pi.as<int>(),
                          pv2.as<float>(), st(), history.as<uint32_t>(), mhist.as<float>(), s));
    return launch_step_advance(st(), add_pos, s);
  }

  // n_layers < L: CausalLM::forward_one_draft (causal_lm.rs:283-323), the
  // first n_layers layers, zero K/V rows appended to the others
  // the fused step's buffers and launch plans (all layers share shapes and formats)
  syn_status_t setup_fused() {
    fused_ok = false;
    const int fm[5] = {c.fmt_qkv, c.fmt_o, c.fmt_gate_up, c.fmt_down, c.fmt_lm_head};
    if (!kqf_fits((int)h, (int)qd, (int)inter, (int)c.base.n_heads, (int)c.base.n_kv_heads,
                  (int)hd, (int)S, fm, 5))
      return SYN_OK;
    const Layer &L0 = layers[0];
    fp_qkv = kqf_plan(L0.qkv, false);
    fp_o = kqf_plan(L0.o, false);
    fp_gu = kqf_plan(L0.gu, true);
    fp_down = kqf_plan(L0.down, false);
    fp_lm = kqf_plan(lm_head, false);
    fp_lm.bs = fp_lm.units;  // the top-2 epilogue needs whole dot products
    fp_lm.ks = 1;
    // workgroups that each loop over 64-row panels (one prologue per
    // workgroup); the merge reads one top-2 per workgroup
    fp_lm.groups = std::min(fp_lm.groups, kKqfTop2Groups);
    const size_t nch = (size_t)kqf_chunks((int)S), nh = c.base.n_heads;
    SYN_TRY(f_r.alloc(h * 8));
    SYN_TRY(f_qkv.alloc(n_qkv * 8));
    SYN_HIP(hipMemset(f_qkv.p, 0, f_qkv.bytes));  // later steps leave it cleared
    SYN_TRY(f_ao.alloc(nh * nch * hd * 4));
    SYN_TRY(f_aml.alloc(nh * nch * 2 * 4));
    SYN_HIP(hipMemset(f_ao.p, 0, f_ao.bytes));
    SYN_HIP(hipMemset(f_aml.p, 0, f_aml.bytes));
    SYN_TRY(f_pv.alloc((size_t)fp_lm.groups * 4));
    SYN_TRY(f_pi.alloc((size_t)fp_lm.groups * 4));
    SYN_TRY(f_pv2.alloc((size_t)fp_lm.groups * 4));
    SYN_HIP(hipDeviceSynchronize());  // the memsets ran on the null stream, not the model's
    fused_ok = true;
    return SYN_OK;
  }

  // fused decode step (klm_fused.hip): five kernels per layer, then the
  // lm_head with per-panel top-2 and the merge that advances the state
  syn_status_t decode_step_fused(hipStream_t s, size_t n) {
    const float eps = c.base.eps;
    const int nh = (int)c.base.n_heads, nkv = (int)c.base.n_kv_heads;
    long long *r = f_r.as<long long>(), *aq = f_qkv.as<long long>();
    for (size_t l = 0; l < n; l++) {
      Layer &Ly = layers[l];
      KqfIn a;  // K1: QKV rows of rmsnorm(r) (layer 0: of the token's embedding row)
      a.r = r;
      a.embed = embed.as<float>();
      a.vocab = (int)vocab;
      a.r_out = r;
      a.st = st();
      a.gain = attn_nw.as<float>() + l * h;
      a.eps = eps;
      a.H = (int)h;
      SYN_TRY(kqf_gemv(Ly.qkv, fp_qkv, l == 0 ? KQF_PRO_EMBED : KQF_PRO_NORM, a, aq, nullptr, 0,
                       s));
      SYN_TRY(kqf_attention(aq, nh, nkv, (int)hd, c.qk_norm ? q_nw.as<float>() + l * hd : nullptr,
                            c.qk_norm ? k_nw.as<float>() + l * hd : nullptr, eps,
                            rope_cos.as<float>(), rope_sin.as<float>(), st(), kc_l(l), vc_l(l),
                            (int)S, f_ao.as<float>(), f_aml.as<float>(), s));
      KqfIn b;  // K3: combine of the attention chunks; r += o; the QKV accumulator cleared
      b.ao = f_ao.as<float>();
      b.aml = f_aml.as<float>();
      b.hd = (int)hd;
      b.nch = kqf_chunks((int)S);
      b.st = st();
      SYN_TRY(kqf_gemv(Ly.o, fp_o, KQF_PRO_ATTN, b, r, aq, (int)n_qkv, s));
      KqfIn g;  // K4: gate|up of rmsnorm(r), SwiGLU
      g.r = r;
      g.gain = ffn_nw.as<float>() + l * h;
      g.eps = eps;
      g.H = (int)h;
      SYN_TRY(kqf_gate_up(Ly.gu, fp_gu, g, (int)inter, hbuf.as<float>(), s));
      KqfIn d;  // K5: r += down(h)
      d.x = hbuf.as<float>();
      SYN_TRY(kqf_gemv(Ly.down, fp_down, KQF_PRO_NONE, d, r, nullptr, 0, s));
    }
    if (n < L)
      SYN_TRY(launch_kv_zero_rows(kc_l(n), vc_l(n), k_elems(), v_elems(), (int)(L - n),
                                  (int)c.base.n_kv_heads, (int)hd, (int)S, st(), s));
    KqfIn f;  // final norm of r
    f.r = r;
    f.gain = final_nw.as<float>();
    f.eps = eps;
    f.H = (int)h;
    SYN_TRY(kqf_lm_head(lm_head, fp_lm, f, logits.as<float>(), f_pv.as<float>(),
                        f_pi.as<int>(), f_pv2.as<float>(), s));
    return launch_argmax_advance(f_pv.as<float>(), f_pi.as<int>(), f_pv2.as<float>(),
                                 fp_lm.groups, st(), history.as<uint32_t>(), mhist.as<float>(),
                                 s);
  }

  syn_status_t decode_step(hipStream_t s, size_t n_layers = SIZE_MAX) {
    const size_t n = std::min(n_layers, L);
    if (use_fused && fused_ok && n > 0) return decode_step_fused(s, n);
    SYN_TRY(launch_embed(embed.as<float>(), &st()->token, 1, (int)h, (int)vocab, x.as<float>(), s));
    for (size_t l = 0; l < n; l++) SYN_TRY(layer(l, 1, false, s));
    if (n < L)
      SYN_TRY(launch_kv_zero_rows(kc_l(n), vc_l(n), k_elems(), v_elems(), (int)(L - n),
                                  (int)c.base.n_kv_heads, (int)hd, (int)S, st(), s));
    return head(0, 1, s);
  }

  // the draft step as its own graph (rebuilt when the layer count changes)
  hipGraphExec_t draft_graph = nullptr;
  size_t draft_layers = 0;
  syn_status_t run_draft(size_t n_layers) {
    if (!use_graph) return decode_step(stream, n_layers);
    if (draft_graph && draft_layers != n_layers) {
      SYN_HIP(hipStreamSynchronize(stream));
      (void)hipGraphExecDestroy(draft_graph);
      draft_graph = nullptr;
    }
    if (!draft_graph) {
      hipGraph_t g;
      SYN_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
      syn_status_t st_ = decode_step(stream, n_layers);
      hipError_t e = hipStreamEndCapture(stream, &g);
      if (st_ != SYN_OK) {
        if (e == hipSuccess) (void)hipGraphDestroy(g);
        return st_;
      }
      if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
      e = hipGraphInstantiate(&draft_graph, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (e != hipSuccess) {
        draft_graph = nullptr;
        return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
      }
      draft_layers = n_layers;
    }
    SYN_HIP(hipGraphLaunch(draft_graph, stream));
    return SYN_OK;
  }

  syn_status_t build_graph() {
    if (graph) return SYN_OK;
    hipGraph_t g;
    SYN_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    syn_status_t st_ = decode_step(stream);
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (st_ != SYN_OK) {
      if (e == hipSuccess) (void)hipGraphDestroy(g);
      return st_;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    e = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
      graph = nullptr;
      return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    }
    return SYN_OK;
  }

  // one decode step on `stream`: graph replay or the same kernels launched eagerly
  syn_status_t run_step() {
    if (!use_graph) return decode_step(stream);
    SYN_TRY(build_graph());
    SYN_HIP(hipGraphLaunch(graph, stream));
    return SYN_OK;
  }

  syn_status_t set_state(int pos, uint32_t token, int step) {
    StepState hs{pos, token, step, 0.0f};
    SYN_HIP(hipMemcpyAsync(state.p, &hs, sizeof(hs), hipMemcpyHostToDevice, stream));
    SYN_HIP(hipStreamSynchronize(stream));
    return SYN_OK;
  }

  syn_status_t get_state(StepState *out) {
    SYN_HIP(hipMemcpyAsync(out, state.p, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    SYN_HIP(hipStreamSynchronize(stream));
    return SYN_OK;
  }

  // the layers of CausalLM::forward_prefill (causal_lm.rs:195-224) over n
  // tokens whose ids are on the device, appended at cache rows cache_off ..
  syn_status_t prefill_rows(const uint32_t *d_ids, int n, int cache_off) {
    SYN_TRY(launch_embed(embed.as<float>(), d_ids, n, (int)h, (int)vocab, x.as<float>(), stream));
    for (size_t l = 0; l < L; l++) SYN_TRY(layer(l, n, true, stream, cache_off));
    return SYN_OK;
  }

  // forward_prefill into an empty cache (a fresh ModelState)
  syn_status_t prefill(const uint32_t *host_ids, size_t n) {
    if (n == 0 || n > S) {
      set_error("prefill length must be in [1, max_seq]");
      return SYN_ERR_INVALID_ARG;
    }
    SYN_HIP(hipMemcpyAsync(ids.p, host_ids, n * 4, hipMemcpyHostToDevice, stream));
    SYN_TRY(set_state(0, 0, 0));
    SYN_TRY(prefill_rows(ids.as<uint32_t>(), (int)n, 0));
    return head((int)n - 1, (int)n, stream);
  }

  // forward_prefill into the cache as it stands (rows appended after the
  // cached ones, rotated from position 0, attending among themselves)
  syn_status_t prefill_append(const uint32_t *host_ids, size_t n) {
    StepState cur;
    SYN_TRY(get_state(&cur));
    if (n == 0 || (size_t)cur.pos + n > S) {
      set_error("prefill rows must be in [1, max_seq - cached rows]");
      return SYN_ERR_INVALID_ARG;
    }
    SYN_HIP(hipMemcpyAsync(ids.p, host_ids, n * 4, hipMemcpyHostToDevice, stream));
    SYN_TRY(prefill_rows(ids.as<uint32_t>(), (int)n, cur.pos));
    return head((int)n - 1, (int)n, stream);
  }

  syn_status_t truncate(size_t new_len) {  // kvcache.zig:109-113
    StepState cur;
    SYN_TRY(get_state(&cur));
    if (new_len < (size_t)cur.pos) SYN_TRY(set_state((int)new_len, cur.token, cur.step));
    return SYN_OK;
  }

  // generate_speculative (pipeline.rs:281-395), greedy, max_new as the stop
  // condition; drafts from the first n_draft layers (forward_one_draft).
  // Same loop as the INT8 decoder's: k draft steps, the verify prefill of
  // [last accepted, drafts] at the round's start, every draft accepted, a
  // bonus full step after a full round; enqueued without host round trips.
  syn_status_t generate_speculative(const uint32_t *prompt, size_t n_prompt, size_t max_new,
                                    size_t k, size_t n_draft) {
    if (n_prompt == 0 || n_prompt > S) {
      set_error("prefill length must be in [1, max_seq]");
      return SYN_ERR_INVALID_ARG;
    }
    size_t pos = n_prompt, gen = 1, calls = 1, top = n_prompt;
    while (gen < max_new) {
      const size_t save = pos, acc = std::min(k, max_new - gen);
      top = std::max(top, save + k + 1);
      calls += k;
      gen += acc;
      pos = save + k + 1;
      if (acc == k && gen < max_new) {
        top = std::max(top, pos + 1);
        pos += 1;
        gen += 1;
        calls += 1;
      }
    }
    if (top > S || calls > S + 1) {
      set_error("speculative decode: rows or sample calls exceed max_seq");
      return SYN_ERR_INVALID_ARG;
    }
    if (use_graph) SYN_TRY(build_graph());
    SYN_TRY(prefill(prompt, n_prompt));
    pos = n_prompt;
    gen = 1;
    while (gen < max_new) {
      const size_t save = pos, s0 = gen;
      for (size_t i = 0; i < k; i++) SYN_TRY(run_draft(n_draft));
      SYN_TRY(prefill_rows(history.as<uint32_t>() + (s0 - 1), (int)(k + 1), (int)save));
      SYN_TRY(launch_state_set(st(), (int)(save + k + 1), -1, stream));
      const size_t acc = std::min(k, max_new - gen);
      gen += acc;
      pos = save + k + 1;
      if (acc == k && gen < max_new) {
        SYN_TRY(run_step());
        gen += 1;
        pos += 1;
      }
    }
    return SYN_OK;
  }
};

static bool kq_fmt_ok(int f) {
  return f == SYN_HIP_FMT_Q8_0 || f == SYN_HIP_FMT_Q4_K || f == SYN_HIP_FMT_Q6_K;
}

static syn_status_t check_klm(syn_hip_klm_t *m) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (!m->finalized) {
    set_error("model not finalized");
    return SYN_ERR_INVALID_ARG;
  }
  return SYN_OK;
}

extern "C" {

syn_status_t syn_hip_klm_create(const syn_hip_klm_config *cfg, syn_hip_klm_t **out) {
  if (!cfg || !out) return SYN_ERR_NULL_PTR;
  const syn_hip_lm_config &b = cfg->base;
  if (!b.hidden || !b.n_layers || !b.n_heads || !b.n_kv_heads || !b.head_dim || !b.inter ||
      !b.vocab || !b.max_seq || b.n_heads % b.n_kv_heads || b.head_dim % 2 || b.head_dim > 1024)
    return SYN_ERR_INVALID_ARG;
  const int fm[5] = {cfg->fmt_qkv, cfg->fmt_o, cfg->fmt_gate_up, cfg->fmt_down, cfg->fmt_lm_head};
  for (int f : fm)
    if (!kq_fmt_ok(f)) return SYN_ERR_INVALID_ARG;
  // K of every projection must be a whole number of blocks
  const size_t qd = (size_t)b.n_heads * b.head_dim;
  if (b.hidden % kq_block_elems(cfg->fmt_qkv) || b.hidden % kq_block_elems(cfg->fmt_gate_up) ||
      qd % kq_block_elems(cfg->fmt_o) || b.inter % kq_block_elems(cfg->fmt_down) ||
      b.hidden % kq_block_elems(cfg->fmt_lm_head))
    return SYN_ERR_SHAPE_MISMATCH;
  SYN_TRY(ensure_init());
  auto *m = new syn_hip_klm_s();
  m->c = *cfg;
  m->h = b.hidden;
  m->hd = b.head_dim;
  m->qd = qd;
  m->kvd = (size_t)b.n_kv_heads * b.head_dim;
  m->inter = b.inter;
  m->L = b.n_layers;
  m->vocab = b.vocab;
  m->S = b.max_seq;
  m->n_qkv = m->qd + 2 * m->kvd;
  m->layers.resize(m->L);
  for (auto &Ly : m->layers) Ly.pending.resize(5);
  hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    m->stream = nullptr;
    delete m;
    return hip_fail(e, "hipStreamCreate", __FILE__, __LINE__);
  }
  syn_status_t st = m->alloc_all();
  if (st != SYN_OK) {
    delete m;
    return st;
  }
  *out = m;
  return SYN_OK;
}

syn_status_t syn_hip_klm_set_embed(syn_hip_klm_t *m, const float *embed) {
  if (!m || !embed) return SYN_ERR_NULL_PTR;
  SYN_TRY(m->embed.alloc(m->vocab * m->h * 4));
  SYN_HIP(hipMemcpy(m->embed.p, embed, m->vocab * m->h * 4, hipMemcpyHostToDevice));
  m->have_embed = true;
  return SYN_OK;
}

syn_status_t syn_hip_klm_set_proj(syn_hip_klm_t *m, uint32_t layer, int proj,
                                  const uint8_t *gguf_bytes) {
  if (!m || !gguf_bytes) return SYN_ERR_NULL_PTR;
  if (layer >= m->L || proj < 0 || proj > 6) return SYN_ERR_INVALID_ARG;
  return m->set_proj(layer, proj, gguf_bytes);
}

syn_status_t syn_hip_klm_set_lm_head(syn_hip_klm_t *m, const uint8_t *gguf_bytes) {
  if (!m || !gguf_bytes) return SYN_ERR_NULL_PTR;
  SYN_TRY(m->lm_head.upload(m->c.fmt_lm_head, gguf_bytes, m->vocab, m->h));
  m->have_lm = true;
  return SYN_OK;
}

syn_status_t syn_hip_klm_init_synthetic(syn_hip_klm_t *m, uint64_t seed_base, float stddev) {
  if (!m) return SYN_ERR_NULL_PTR;
  const size_t h = m->h;
  {
    std::vector<float> emb(m->vocab * h);
    fill_normal_parallel(emb.data(), emb.size(), seed_base + 0, stddev);
    SYN_TRY(syn_hip_klm_set_embed(m, emb.data()));
  }
  for (size_t l = 0; l < m->L; l++) {
    std::vector<std::vector<uint8_t>> bytes(7);
    std::vector<std::thread> th;
    for (int t = 0; t < 7; t++)
      th.emplace_back([&, t] {
        size_t n, k;
        m->proj_shape(t, &n, &k);
        std::vector<float> w(n * k);
        fill_normal(w.data(), w.size(), seed_base + 1 + 8 * l + (uint64_t)t, stddev);
        bytes[t].resize(m->proj_bytes(t));
        kq_encode(m->fmt_of(t), w.data(), n, k, bytes[t].data());
      });
    for (auto &x : th) x.join();
    for (int t = 0; t < 7; t++) SYN_TRY(m->set_proj(l, t, bytes[t].data()));
  }
  {  // untied lm_head: tensor id 1 + 8 * n_layers, encoded in row chunks on threads
    const int f = m->c.fmt_lm_head;
    const size_t rb = (h / kq_block_elems(f)) * kq_block_bytes(f);
    std::vector<float> w(m->vocab * h);
    fill_normal_parallel(w.data(), w.size(), seed_base + 1 + 8 * m->L, stddev);
    std::vector<uint8_t> bytes(m->vocab * rb);
    const unsigned nt = 16;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++)
      th.emplace_back([&, t] {
        const size_t r0 = m->vocab * t / nt, r1 = m->vocab * (t + 1) / nt;
        kq_encode(f, w.data() + r0 * h, r1 - r0, h, bytes.data() + r0 * rb);
      });
    for (auto &x : th) x.join();
    SYN_TRY(syn_hip_klm_set_lm_head(m, bytes.data()));
  }
  return SYN_OK;
}

syn_status_t syn_hip_klm_finalize(syn_hip_klm_t *m) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (!m->have_embed || !m->have_lm) {
    set_error("embed_tokens or lm_head not set");
    return SYN_ERR_INVALID_ARG;
  }
  for (size_t l = 0; l < m->L; l++)
    if (m->layers[l].have != 0x7f) {
      set_error("layer " + std::to_string(l) + " incomplete");
      return SYN_ERR_INVALID_ARG;
    }
  const size_t half = m->hd / 2;
  std::vector<float> cs(m->S * half), sn(m->S * half);
  const float fb = (float)m->c.base.rope_theta;
  for (size_t pos = 0; pos < m->S; pos++)
    for (size_t i = 0; i < half; i++) {  // models/lm/builder.rs:121-129
      const float freq = 1.0f / powf(fb, 2.0f * (float)i / (float)m->hd);
      const float scaled = freq / 1.0f;
      const float angle = (float)pos * scaled;
      cs[pos * half + i] = cosf(angle);
      sn[pos * half + i] = sinf(angle);
    }
  SYN_HIP(hipMemcpy(m->rope_cos.p, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  SYN_HIP(hipMemcpy(m->rope_sin.p, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  for (auto &Ly : m->layers) {
    SYN_TRY(Ly.qkv.prepare(m->S));
    SYN_TRY(Ly.o.prepare(m->S));
    SYN_TRY(Ly.gu.prepare(m->S));
    SYN_TRY(Ly.down.prepare(m->S));
  }
  SYN_TRY(m->lm_head.prepare(1));
  SYN_TRY(m->setup_fused());
  m->finalized = true;
  SYN_TRY(m->set_state(0, 0, 0));
  return SYN_OK;
}

syn_status_t syn_hip_klm_reset(syn_hip_klm_t *m) {
  SYN_TRY(check_klm(m));
  return m->set_state(0, 0, 0);
}

syn_status_t syn_hip_klm_forward_prefill(syn_hip_klm_t *m, const uint32_t *ids, size_t n,
                                         float *host_logits) {
  SYN_TRY(check_klm(m));
  if (!ids) return SYN_ERR_NULL_PTR;
  SYN_TRY(m->prefill(ids, n));
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_klm_forward_prefill_append(syn_hip_klm_t *m, const uint32_t *ids,
                                                size_t n, float *host_logits) {
  SYN_TRY(check_klm(m));
  if (!ids) return SYN_ERR_NULL_PTR;
  SYN_TRY(m->prefill_append(ids, n));
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_klm_truncate(syn_hip_klm_t *m, size_t new_len) {
  SYN_TRY(check_klm(m));
  return m->truncate(new_len);
}

syn_status_t syn_hip_klm_cache_len(syn_hip_klm_t *m, size_t *out_len) {
  SYN_TRY(check_klm(m));
  if (!out_len) return SYN_ERR_NULL_PTR;
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  *out_len = (size_t)cur.pos;
  return SYN_OK;
}

syn_status_t syn_hip_klm_forward_one_draft(syn_hip_klm_t *m, uint32_t token, size_t n_layers,
                                           float *host_logits) {
  SYN_TRY(check_klm(m));
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos >= m->S) {
    set_error("KV cache full");
    return SYN_ERR_INVALID_ARG;
  }
  SYN_TRY(m->set_state(cur.pos, token, cur.step));
  SYN_TRY(m->run_draft(n_layers));
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_klm_generate_speculative(syn_hip_klm_t *m, const uint32_t *prompt,
                                              size_t n_prompt, size_t max_new, size_t k,
                                              size_t draft_layers, uint32_t *out_tokens,
                                              float *out_margins) {
  SYN_TRY(check_klm(m));
  if (!prompt || !out_tokens) return SYN_ERR_NULL_PTR;
  if (k == 0) return syn_hip_klm_generate(m, prompt, n_prompt, max_new, out_tokens, out_margins);
  if (max_new == 0) return SYN_OK;
  // speculative_draft_layers, else num_layers / DEFAULT_DRAFT_LAYER_FRACTION (pipeline.rs:295-299)
  const size_t n_draft = draft_layers > 0 ? draft_layers : m->L / 3;
  SYN_TRY(m->generate_speculative(prompt, n_prompt, max_new, k, n_draft));
  SYN_HIP(hipMemcpyAsync(out_tokens, m->history.p, max_new * 4, hipMemcpyDeviceToHost,
                         m->stream));
  if (out_margins)
    SYN_HIP(hipMemcpyAsync(out_margins, m->mhist.p, max_new * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_klm_forward_one(syn_hip_klm_t *m, uint32_t token, float *host_logits) {
  SYN_TRY(check_klm(m));
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos >= m->S) {
    set_error("KV cache full");
    return SYN_ERR_INVALID_ARG;
  }
  SYN_TRY(m->set_state(cur.pos, token, cur.step));
  SYN_TRY(m->run_step());
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_klm_generate(syn_hip_klm_t *m, const uint32_t *prompt, size_t n_prompt,
                                  size_t max_new, uint32_t *out_tokens, float *out_margins) {
  SYN_TRY(check_klm(m));
  if (!prompt || !out_tokens) return SYN_ERR_NULL_PTR;
  if (max_new == 0) return SYN_OK;
  if (n_prompt + max_new - 1 > m->S) {
    set_error("prompt + generated tokens exceed max_seq");
    return SYN_ERR_INVALID_ARG;
  }
  if (m->use_graph) SYN_TRY(m->build_graph());
  SYN_TRY(m->prefill(prompt, n_prompt));
  for (size_t i = 1; i < max_new; i++) SYN_TRY(m->run_step());
  SYN_HIP(hipMemcpyAsync(out_tokens, m->history.p, max_new * 4, hipMemcpyDeviceToHost,
                         m->stream));
  if (out_margins)
    SYN_HIP(hipMemcpyAsync(out_margins, m->mhist.p, max_new * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_klm_time(syn_hip_klm_t *m, const uint32_t *prompt, size_t n_prompt,
                              size_t steps, float *prefill_ms, float *decode_ms) {
  SYN_TRY(check_klm(m));
  if (!prompt || !prefill_ms || !decode_ms) return SYN_ERR_NULL_PTR;
  if (n_prompt + steps > m->S) {
    set_error("prompt + decode steps exceed max_seq");
    return SYN_ERR_INVALID_ARG;
  }
  if (m->use_graph) SYN_TRY(m->build_graph());
  hipEvent_t a, b, c;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  SYN_HIP(hipEventCreate(&c));
  SYN_HIP(hipMemcpyAsync(m->ids.p, prompt, n_prompt * 4, hipMemcpyHostToDevice, m->stream));
  SYN_TRY(m->set_state(0, 0, 0));
  SYN_HIP(hipEventRecord(a, m->stream));
  SYN_TRY(launch_embed(m->embed.as<float>(), m->ids.as<uint32_t>(), (int)n_prompt, (int)m->h,
                       (int)m->vocab, m->x.as<float>(), m->stream));
  for (size_t l = 0; l < m->L; l++) SYN_TRY(m->layer(l, (int)n_prompt, true, m->stream));
  SYN_TRY(m->head((int)n_prompt - 1, (int)n_prompt, m->stream));
  SYN_HIP(hipEventRecord(b, m->stream));
  for (size_t i = 0; i < steps; i++) SYN_TRY(m->run_step());
  SYN_HIP(hipEventRecord(c, m->stream));
  SYN_HIP(hipEventSynchronize(c));
  SYN_HIP(hipEventElapsedTime(prefill_ms, a, b));
  SYN_HIP(hipEventElapsedTime(decode_ms, b, c));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipEventDestroy(c);
  return SYN_OK;
}

syn_status_t syn_hip_klm_set_norms(syn_hip_klm_t *m, uint32_t layer, const float *attn_norm,
                                   const float *ffn_norm, const float *q_norm,
                                   const float *k_norm) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (layer >= m->L) return SYN_ERR_INVALID_ARG;
  const size_t h = m->h, hd = m->hd;
  if (attn_norm)
    SYN_HIP(hipMemcpy(m->attn_nw.as<float>() + layer * h, attn_norm, h * 4, hipMemcpyHostToDevice));
  if (ffn_norm)
    SYN_HIP(hipMemcpy(m->ffn_nw.as<float>() + layer * h, ffn_norm, h * 4, hipMemcpyHostToDevice));
  if (q_norm)
    SYN_HIP(hipMemcpy(m->q_nw.as<float>() + layer * hd, q_norm, hd * 4, hipMemcpyHostToDevice));
  if (k_norm)
    SYN_HIP(hipMemcpy(m->k_nw.as<float>() + layer * hd, k_norm, hd * 4, hipMemcpyHostToDevice));
  return SYN_OK;
}

syn_status_t syn_hip_klm_set_final_norm(syn_hip_klm_t *m, const float *norm) {
  if (!m || !norm) return SYN_ERR_NULL_PTR;
  SYN_HIP(hipMemcpy(m->final_nw.p, norm, m->h * 4, hipMemcpyHostToDevice));
  return SYN_OK;
}

// ------------------------------------------------------------------ GGUF
// Tensor names: llama.cpp's (blk.N.*) or the HuggingFace names the
// reference's weight map uses (weight_map.rs: model.layers.N.*).
namespace {

int ggml_of_fmt(int fmt) {
  return fmt == SYN_HIP_FMT_Q8_0 ? SYN_HIP_GGML_Q8_0
       : fmt == SYN_HIP_FMT_Q4_K ? SYN_HIP_GGML_Q4_K : SYN_HIP_GGML_Q6_K;
}

struct GgufTensor {
  uint32_t type = 0, n_dims = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  uint64_t nbytes = 0;
  const uint8_t *data = nullptr;
};

// first of `names` present in the file
bool gguf_get(const syn_hip_gguf_t *g, std::initializer_list<std::string> names, GgufTensor *t,
              std::string *found) {
  for (const std::string &n : names) {
    size_t idx = 0;
    if (syn_hip_gguf_find(g, n.c_str(), &idx) != SYN_OK) continue;
    const void *d = nullptr;
    syn_hip_gguf_tensor_info(g, idx, nullptr, &t->type, &t->n_dims, t->dims, &t->nbytes, &d);
    t->data = static_cast<const uint8_t *>(d);
    *found = n;
    return true;
  }
  return false;
}

// f32 values of an F32 / F16 / Q8_0 / Q4_K / Q6_K tensor (gguf.rs:115-139)
syn_status_t gguf_to_f32(const GgufTensor &t, size_t numel, const std::string &name,
                         std::vector<float> &out) {
  out.resize(numel);
  if (t.type == SYN_HIP_GGML_F32) {
    std::memcpy(out.data(), t.data, numel * 4);
  } else if (t.type == SYN_HIP_GGML_F16) {
    for (size_t i = 0; i < numel; i++) {
      uint16_t h;
      std::memcpy(&h, t.data + 2 * i, 2);
      out[i] = f16_to_f32_reference(h);
    }
  } else if (t.type == SYN_HIP_GGML_Q8_0 || t.type == SYN_HIP_GGML_Q4_K ||
             t.type == SYN_HIP_GGML_Q6_K) {
    const int fmt = t.type == SYN_HIP_GGML_Q8_0 ? SYN_HIP_FMT_Q8_0
                  : t.type == SYN_HIP_GGML_Q4_K ? SYN_HIP_FMT_Q4_K : SYN_HIP_FMT_Q6_K;
    kq_dequant(fmt, t.data, numel / kq_block_elems(fmt), out.data());
  } else {
    set_error("GGUF: tensor " + name + " has a type the loader cannot read as f32");
    return SYN_ERR_INVALID_ARG;
  }
  return SYN_OK;
}

}  // namespace

syn_status_t syn_hip_klm_load_gguf(syn_hip_klm_t *m, const syn_hip_gguf_t *g) {
  if (!m || !g) return SYN_ERR_NULL_PTR;
  const size_t h = m->h, hd = m->hd, L = m->L;
  GgufTensor t;
  std::string nm;
  auto expect = [&](size_t n, size_t k, int fmt) -> syn_status_t {
    const bool dims_ok = t.n_dims == 2 && t.dims[0] == k && t.dims[1] == n;
    if (!dims_ok || (int)t.type != ggml_of_fmt(fmt)) {
      set_error("GGUF: tensor " + nm + " has type " + std::to_string(t.type) + " and dims " +
                std::to_string(t.dims[0]) + "x" + std::to_string(t.dims[1]) + "; the model expects " +
                std::to_string(k) + "x" + std::to_string(n) + " of GGML type " +
                std::to_string(ggml_of_fmt(fmt)));
      return SYN_ERR_SHAPE_MISMATCH;
    }
    return SYN_OK;
  };
  auto missing = [&](const std::string &what) -> syn_status_t {
    set_error("GGUF: no tensor for " + what);
    return SYN_ERR_INVALID_ARG;
  };
  static const char *kLlama[7] = {"attn_q", "attn_k", "attn_v", "attn_output",
                                  "ffn_gate", "ffn_up", "ffn_down"};
  static const char *kHf[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                               "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                               "mlp.down_proj"};
  for (size_t l = 0; l < L; l++) {
    const std::string b = "blk." + std::to_string(l) + ".";
    const std::string hf = "model.layers." + std::to_string(l) + ".";
    for (int p = 0; p < 7; p++) {
      if (!gguf_get(g, {b + kLlama[p] + ".weight", hf + kHf[p] + ".weight"}, &t, &nm))
        return missing(b + kLlama[p]);
      size_t n, k;
      m->proj_shape(p, &n, &k);
      SYN_TRY(expect(n, k, m->fmt_of(p)));
      SYN_TRY(m->set_proj(l, p, t.data));
    }
    std::vector<float> an, fn, qn, kn;
    if (gguf_get(g, {b + "attn_norm.weight", hf + "input_layernorm.weight"}, &t, &nm)) {
      if (t.dims[0] != h) return missing(nm + " of the hidden size");
      SYN_TRY(gguf_to_f32(t, h, nm, an));
    }
    if (gguf_get(g, {b + "ffn_norm.weight", hf + "post_attention_layernorm.weight"}, &t, &nm)) {
      if (t.dims[0] != h) return missing(nm + " of the hidden size");
      SYN_TRY(gguf_to_f32(t, h, nm, fn));
    }
    if (m->c.qk_norm) {
      if (gguf_get(g, {b + "attn_q_norm.weight", hf + "self_attn.q_norm.weight"}, &t, &nm)) {
        if (t.dims[0] != hd) return missing(nm + " of the head size");
        SYN_TRY(gguf_to_f32(t, hd, nm, qn));
      }
      if (gguf_get(g, {b + "attn_k_norm.weight", hf + "self_attn.k_norm.weight"}, &t, &nm)) {
        if (t.dims[0] != hd) return missing(nm + " of the head size");
        SYN_TRY(gguf_to_f32(t, hd, nm, kn));
      }
    }
    SYN_TRY(syn_hip_klm_set_norms(m, (uint32_t)l, an.empty() ? nullptr : an.data(),
                                  fn.empty() ? nullptr : fn.data(),
                                  qn.empty() ? nullptr : qn.data(),
                                  kn.empty() ? nullptr : kn.data()));
  }
  GgufTensor emb;
  std::string emb_name;
  if (!gguf_get(g, {"token_embd.weight", "model.embed_tokens.weight"}, &emb, &emb_name))
    return missing("token_embd");
  if (emb.n_dims != 2 || emb.dims[0] != h || emb.dims[1] != m->vocab) {
    set_error("GGUF: " + emb_name + " is not [vocab, hidden]");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  {
    std::vector<float> e;
    SYN_TRY(gguf_to_f32(emb, m->vocab * h, emb_name, e));
    SYN_TRY(syn_hip_klm_set_embed(m, e.data()));
  }
  if (gguf_get(g, {"output_norm.weight", "model.norm.weight"}, &t, &nm)) {
    if (t.dims[0] != h) return missing(nm + " of the hidden size");
    std::vector<float> fnw;
    SYN_TRY(gguf_to_f32(t, h, nm, fnw));
    SYN_TRY(syn_hip_klm_set_final_norm(m, fnw.data()));
  }
  // lm_head: its own tensor, or tied to the embedding when the file has none
  if (!gguf_get(g, {"output.weight", "lm_head.weight"}, &t, &nm)) {
    t = emb;
    nm = emb_name + " (tied lm_head)";
  }
  SYN_TRY(expect(m->vocab, h, m->c.fmt_lm_head));
  return syn_hip_klm_set_lm_head(m, t.data);
}

syn_status_t syn_hip_klm_set_options(syn_hip_klm_t *m, int fused, int graph) {
  if (!m) return SYN_ERR_NULL_PTR;
  SYN_HIP(hipStreamSynchronize(m->stream));
  if (m->graph && (m->use_fused != (fused != 0))) {  // the captured step changes form
    (void)hipGraphExecDestroy(m->graph);
    m->graph = nullptr;
  }
  if (m->draft_graph && (m->use_fused != (fused != 0))) {
    (void)hipGraphExecDestroy(m->draft_graph);
    m->draft_graph = nullptr;
  }
  m->use_fused = fused != 0;
  m->use_graph = graph != 0;
  return SYN_OK;
}

syn_status_t syn_hip_klm_destroy(syn_hip_klm_t *m) {
  if (m) {
    (void)hipStreamSynchronize(m->stream);
    delete m;
  }
  return SYN_OK;
}

}  // extern "C"
