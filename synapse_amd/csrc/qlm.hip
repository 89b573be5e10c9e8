// INT8 W8A8 causal LM on the device: QuantizedCausalLM
// (quantization/lm/int8.rs:21-709) kept resident in HBM the way the Metal
// backend keeps MetalModelBuffers (metal/gpu_buffers.rs:79-433), with the
// whole greedy loop on the device (only token ids come back).
//
// Per layer (int8.rs:242-282, 429-505):
//   x += down(prev) ; q8(rmsnorm(x))          k_rmsnorm_quant
//   [q|k|v] = W_qkv q8                        fused GEMV (rows of Wq,Wk,Wv)
//   head norms, RoPE(pos), KV append          k_qk_norm_rope_kv
//   attention over the cache                  k_attn_decode
//   o = W_o q8(attn)                          quantize + GEMV
//   x += o ; q8(rmsnorm(x))                   k_rmsnorm_quant
//   [g|u] = W_gu q8                           fused GEMV (rows of Wgate,Wup)
//   q8(silu(g)*u)                             k_swiglu_quant
//   down = W_down q8                          GEMV
// Fusing weight rows of Q/K/V (and gate/up) is exact: each output row has its
// own scale and integer dot product.
#include <algorithm>
#include <thread>
#include <vector>

#include "sampler.hpp"
#include "decode_fused.hpp"
#include "layer_ops.hpp"
#include "linear.hpp"
#include "weights.hpp"

namespace syn {

struct QLayer {
  QLinearInt8 qkv, o, gu, down;
  SplitGemv f_qkv, f_o, f_gu, f_down;  // fused decode plans over these weights
  SplitGemv f_gup;                      // gate|up as pairs of panels (launch_gu_swiglu)
};

}  // namespace syn

using namespace syn;

struct syn_hip_qlm_s {
  syn_hip_lm_config c{};
  size_t h = 0, hd = 0, qd = 0, kvd = 0, inter = 0, L = 0, vocab = 0, S = 0;
  size_t ldh = 0, ldq = 0, ldi = 0, n_qkv = 0;
  std::vector<QLayer> layers;
  std::vector<int> have_layer;
  QLinearInt8 lm_head;
  std::vector<float> host_embed, host_lm_head;  // f32 until finalize quantizes them
  bool qk_norm = true;  // per-head q/k RMSNorm (Qwen3); off for models without the gains
  DevBuf embed, zeros_h, rope_cos, rope_sin, kc, vc;
  // RMSNorm gains (int8.rs:33-56): attention and FFN norms [L][h], q/k head
  // norms [L][hd], final norm [h]; 1.0 until set
  DevBuf attn_nw, ffn_nw, q_nw, k_nw, final_nw;
  DevBuf x, xq, sx, qkv, qrot, attn, aq, sa, o, gu, hq, sh, down, logits, scores;
  DevBuf pv, pi, pv2, state, history, mhist, ids;
  // fused decode step (decode_fused.hip): residual rows, activation scales
  // [qkv, o, gate|up, down, lm_head] and the split-K accumulators
  DevBuf xin, xmid, scal, acc;
  size_t acc_elems = 0;
  hipStream_t stream = nullptr;
  hipGraphExec_t graph = nullptr;
  bool finalized = false;
  // per-launch event pairs of an eager fused step (syn_hip_qlm_time_step_kernels)
  struct TraceEntry {
    int kind;
    hipEvent_t start, end;
  };
  std::vector<TraceEntry> *trace = nullptr;
  // the next SYN_LAUNCH records its kernel's own start and end on two events
  syn_status_t trace_begin(hipStream_t) {
    if (!trace) return SYN_OK;
    LaunchEvents &ev = launch_events();
    SYN_HIP(hipEventCreate(&ev.start));
    SYN_HIP(hipEventCreate(&ev.stop));
    trace->push_back(TraceEntry{-1, ev.start, ev.stop});
    return SYN_OK;
  }
  syn_status_t trace_end(int kind, hipStream_t) {
    if (!trace) return SYN_OK;
    LaunchEvents &ev = launch_events();
    if (ev.start) {  // the launcher did not go through SYN_LAUNCH
      ev.start = ev.stop = nullptr;
      set_error("time_step_kernels: a step kernel is not event-timed");
      return SYN_ERR_INTERNAL;
    }
    trace->back().kind = kind;
    return SYN_OK;
  }
  bool fused = true;      // fused five-kernel decode layer (else one kernel per op)
  bool use_graph = true;  // replay the decode step as a HIP graph (else launch eagerly)
  // sampling (sampler.hip): CombinedSampler settings, its scratch, and the
  // draws of the seeded StdRng, one per generated token (index = step)
  bool sampling = false;
  SampleArgs sargs;
  SampleScratch sscr;
  DevBuf u_draws;

  ~syn_hip_qlm_s() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (stream) (void)hipStreamDestroy(stream);
  }
  // per-layer KV caches in the decode attention's tiled layout (layer_ops.hpp)
  size_t k_elems() const { return kv_k_elems((int)(kvd / hd), (int)hd, (int)S); }
  size_t v_elems() const { return kv_v_elems((int)(kvd / hd), (int)hd, (int)S); }
  float *kc_l(size_t l) { return kc.as<float>() + l * k_elems(); }
  float *vc_l(size_t l) { return vc.as<float>() + l * v_elems(); }
  StepState *st() { return state.as<StepState>(); }
  const float *an(size_t l) { return attn_nw.as<float>() + l * h; }
  const float *fn(size_t l) { return ffn_nw.as<float>() + l * h; }
  const float *qn(size_t l) { return qk_norm ? q_nw.as<float>() + l * hd : nullptr; }
  const float *kn(size_t l) { return qk_norm ? k_nw.as<float>() + l * hd : nullptr; }

  syn_status_t alloc_all() {
    const size_t T = S;  // prefill rows
    SYN_TRY(zeros_h.alloc(h * 4));
    SYN_HIP(hipMemset(zeros_h.p, 0, h * 4));
    SYN_TRY(rope_cos.alloc(S * (hd / 2) * 4));
    SYN_TRY(rope_sin.alloc(S * (hd / 2) * 4));
    SYN_TRY(kc.alloc(L * k_elems() * 4));
    SYN_TRY(vc.alloc(L * v_elems() * 4));
    SYN_TRY(x.alloc(T * h * 4));
    SYN_TRY(xq.alloc(T * ldh));
    SYN_TRY(sx.alloc(T * 4));
    SYN_TRY(qkv.alloc(T * n_qkv * 4));
    SYN_TRY(qrot.alloc(T * qd * 4));
    SYN_TRY(attn.alloc(T * qd * 4));
    SYN_TRY(aq.alloc(T * ldq));
    SYN_TRY(sa.alloc(T * 4));
    SYN_TRY(o.alloc(T * h * 4));
    SYN_TRY(gu.alloc(T * 2 * inter * 4));
    SYN_TRY(hq.alloc(T * ldi));
    SYN_TRY(sh.alloc(T * 4));
    SYN_TRY(down.alloc(T * h * 4));
    SYN_TRY(logits.alloc(vocab * 4));
    SYN_TRY(scores.alloc(c.n_heads * S * 4));
    const size_t np = std::max<size_t>(256, cdiv(vocab, 64));
    SYN_TRY(pv.alloc(np * 4));
    SYN_TRY(pi.alloc(np * 4));
    SYN_TRY(pv2.alloc(np * 4));
    SYN_TRY(xin.alloc(h * 4));
    SYN_TRY(xmid.alloc(h * 4));
    SYN_TRY(scal.alloc(64));
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
    // zero padding columns of the activation rows once (kernels never write them)
    SYN_HIP(hipMemset(xq.p, 0, xq.bytes));
    SYN_HIP(hipMemset(aq.p, 0, aq.bytes));
    SYN_HIP(hipMemset(hq.p, 0, hq.bytes));
    SYN_HIP(hipMemset(kc.p, 0, kc.bytes));
    SYN_HIP(hipMemset(vc.p, 0, vc.bytes));
    return SYN_OK;
  }

  syn_status_t set_layer(size_t l, const float *wq, const float *wk, const float *wv,
                         const float *wo, const float *wg, const float *wu, const float *wd) {
    QLayer &Ly = layers[l];
    // q,k,v rows stacked: per-row scales make the fused GEMV exact
    {
      std::vector<float> sc(n_qkv);
      std::vector<int8_t> q(n_qkv * h);
      const float *srcs[3] = {wq, wk, wv};
      const size_t rows[3] = {qd, kvd, kvd};
      size_t r0 = 0;
      for (int t = 0; t < 3; t++) {
        host_minmax_scales(srcs[t], rows[t], h, sc.data() + r0);
        host_quantize_weights_nk(srcs[t], sc.data() + r0, rows[t], h, q.data() + r0 * h);
        r0 += rows[t];
      }
      SYN_TRY(Ly.qkv.upload_nk(q.data(), sc.data(), n_qkv, h));
    }
    SYN_TRY(Ly.o.from_f32(wo, h, qd));
    {
      std::vector<float> sc(2 * inter);
      std::vector<int8_t> q(2 * inter * h);
      host_minmax_scales(wg, inter, h, sc.data());
      host_quantize_weights_nk(wg, sc.data(), inter, h, q.data());
      host_minmax_scales(wu, inter, h, sc.data() + inter);
      host_quantize_weights_nk(wu, sc.data() + inter, inter, h, q.data() + inter * h);
      SYN_TRY(Ly.gu.upload_nk(q.data(), sc.data(), 2 * inter, h));
    }
    SYN_TRY(Ly.down.from_f32(wd, h, inter));
    have_layer[l] = 1;
    return SYN_OK;
  }

  // ---------------------------------------------------------- one layer
  // cache_off (prefill only): cache row of the first of `rows` tokens
  syn_status_t layer(size_t l, int rows, bool prefill, hipStream_t s, int cache_off = 0) {
    QLayer &Ly = layers[l];
    const float eps = c.eps;
    const int nh = (int)c.n_heads, nkv = (int)c.n_kv_heads;
    SYN_TRY(launch_rmsnorm_quant(x.as<float>(), l == 0 ? nullptr : down.as<float>(),
                                 an(l), eps, rows, (int)h, xq.as<int8_t>(), (int)ldh,
                                 sx.as<float>(), nullptr, s));
    SYN_TRY(Ly.qkv.gemv(rows, xq.as<int8_t>(), ldh, sx.as<float>(), qkv.as<float>(), n_qkv, s));
    SYN_TRY(launch_qk_norm_rope_kv(qkv.as<float>(), (int)n_qkv, rows, nh, nkv, (int)hd,
                                   qn(l), kn(l), eps, rope_cos.as<float>(),
                                   rope_sin.as<float>(), prefill ? nullptr : &st()->pos, 0,
                                   qrot.as<float>(), kc_l(l), vc_l(l), (int)S, s,
                                   prefill ? cache_off : 0));
    if (prefill)
      SYN_TRY(launch_attention_prefill(qrot.as<float>(), kc_l(l), vc_l(l), rows, nh, nkv,
                                       (int)hd, (int)S, nullptr, attn.as<float>(), s, cache_off));
    else
      SYN_TRY(launch_attention_decode(qrot.as<float>(), kc_l(l), vc_l(l), &st()->pos, nh, nkv,
                                      (int)hd, scores.as<float>(), (int)S, attn.as<float>(), s));
    SYN_TRY(launch_quantize_rows(attn.as<float>(), rows, qd, qd, aq.as<int8_t>(), ldq,
                                 sa.as<float>(), s));
    SYN_TRY(Ly.o.gemv(rows, aq.as<int8_t>(), ldq, sa.as<float>(), o.as<float>(), h, s));
    SYN_TRY(launch_rmsnorm_quant(x.as<float>(), o.as<float>(), fn(l), eps, rows,
                                 (int)h, xq.as<int8_t>(), (int)ldh, sx.as<float>(), nullptr, s));
    SYN_TRY(Ly.gu.gemv(rows, xq.as<int8_t>(), ldh, sx.as<float>(), gu.as<float>(), 2 * inter, s));
    SYN_TRY(launch_swiglu_quant(gu.as<float>(), (int)(2 * inter), rows, (int)inter,
                                hq.as<int8_t>(), (int)ldi, sh.as<float>(), s));
    SYN_TRY(Ly.down.gemv(rows, hq.as<int8_t>(), ldi, sh.as<float>(), down.as<float>(), h, s));
    return SYN_OK;
  }

  // final norm of row `row`, lm_head, greedy argmax, state advance
  syn_status_t head(int row, int add_pos, hipStream_t s) {
    float *xr = x.as<float>() + (size_t)row * h;
    const float *dr = down.as<float>() + (size_t)row * h;
    SYN_TRY(launch_rmsnorm_quant(xr, dr, final_nw.as<float>(), c.eps, 1, (int)h, xq.as<int8_t>(),
                                 (int)ldh, sx.as<float>(), nullptr, s));
    SYN_TRY(lm_head.gemv(1, xq.as<int8_t>(), ldh, sx.as<float>(), logits.as<float>(), vocab, s));
    if (sampling)
      return launch_sample(logits.as<float>(), (int)vocab, history.as<uint32_t>(), 0, sargs,
                           u_draws.as<float>(), st(), add_pos, history.as<uint32_t>(),
                           mhist.as<float>(), sscr, nullptr, s);
    SYN_TRY(launch_argmax(logits.as<float>(), (int)vocab, pv.as<float>(), pi.as<int>(),
                          pv2.as<float>(), st(), history.as<uint32_t>(), mhist.as<float>(), s));
    return launch_step_advance(st(), add_pos, s);
  }

  syn_status_t decode_step(hipStream_t s) {
    if (fused) return decode_step_fused(s);
    SYN_TRY(launch_embed(embed.as<float>(), &st()->token, 1, (int)h, (int)vocab, x.as<float>(), s));
    for (size_t l = 0; l < L; l++) SYN_TRY(layer(l, 1, false, s));
    return head(0, 1, s);
  }

  // Split-K plans for the fused step (one per layer: the weights differ, the
  // shapes do not) and their int32 accumulators, one set per layer so that a
  // single zeroing kernel at the start of the step resets all of them.
  syn_status_t prepare_fused() {
    int cus = 256;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
      (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // grids of about half a workgroup per CU: every workgroup repeats the
    // prologue (the RMSNorm chains read the whole row), and at the Qwen3
    // shape the QKV kernel measured 4.87 us on 256 workgroups against 5.68
    // on 512, gate|up 7.51 on 192 pairs' slices against 8.13 on 384 (a
    // quarter of the CUs: 5.39 and 7.83); O and down did not change
    const int target = std::max(1, cus / 2);
    size_t per_layer = 0;
    for (auto &Ly : layers) {
      Ly.f_qkv = plan_split_gemv(Ly.qkv.w.p, Ly.qkv.scales.as<float>(), (int)n_qkv,
                                 Ly.qkv.chunks, target, 256);
      // O on 512 threads (two waves per SIMD): 658.4 against 659.8 us per
      // token at positions 20-84; 512 measured slower for QKV (669 against
      // 660) and gate|up (663)
      Ly.f_o =
          plan_split_gemv(Ly.o.w.p, Ly.o.scales.as<float>(), (int)h, Ly.o.chunks, target, 512);
      Ly.f_gu = plan_split_gemv(Ly.gu.w.p, Ly.gu.scales.as<float>(), (int)(2 * inter),
                                Ly.gu.chunks, target, 256);
      Ly.f_down = plan_split_gemv(Ly.down.w.p, Ly.down.scales.as<float>(), (int)h,
                                  Ly.down.chunks, target, 512);
      per_layer = (size_t)Ly.f_qkv.N64 + Ly.f_o.N64 + Ly.f_gu.N64 + Ly.f_down.N64;
      if (gu_swiglu_fits((int)h, (int)inter))
        Ly.f_gup = plan_gu_pairs(Ly.gu.w.p, Ly.gu.scales.as<float>(), (int)inter, Ly.gu.chunks,
                                 target, 256);
    }
    // then one max |h| slot per layer for the gate|up SwiGLU kernel
    acc_elems = per_layer * L + round_up(L, 64);
    SYN_TRY(acc.alloc(acc_elems * 4));
    int *p = acc.as<int>();
    for (auto &Ly : layers) {
      SplitGemv *g[4] = {&Ly.f_qkv, &Ly.f_o, &Ly.f_gu, &Ly.f_down};
      for (int i = 0; i < 4; i++) {
        g[i]->acc = p;
        p += g[i]->N64;
      }
      // the gate|up pairs' inter packed 64-bit row accumulators take the
      // 2*inter int32 words (N64 is a multiple of 64: 256-byte aligned)
      if (gu_swiglu_fits((int)h, (int)inter)) Ly.f_gup.acc = Ly.f_gu.acc;
    }
    return SYN_OK;
  }

  bool fused_supported() const {
    return fused_attention_fits((int)hd, (int)S) && fused_gemv_fits((int)h) &&
           fused_gemv_fits((int)qd) && fused_gemv_fits((int)inter);
  }

  // one decode token in 5 kernels per layer + 3 (decode_fused.hip)
  syn_status_t decode_step_fused(hipStream_t s) {
    float *sc = scal.as<float>();
    float *s_qkv = sc + 0, *s_o = sc + 1, *s_gu = sc + 2, *s_down = sc + 3, *s_head = sc + 4;
    const float eps = c.eps;
    const int nh = (int)c.n_heads, nkv = (int)c.n_kv_heads;
    SYN_TRY(trace_begin(s));
    SYN_TRY(launch_zero_i32(acc.as<int>(), acc_elems, s));
    SYN_TRY(trace_end(SYN_HIP_STEP_ZERO, s));
    for (size_t l = 0; l < L; l++) {
      QLayer &Ly = layers[l];
      const RowSrc prev = l == 0 ? RowSrc{} : layers[l - 1].f_down.rows(s_down);
      SYN_TRY(trace_begin(s));
      SYN_TRY(launch_fused_norm_gemv(l == 0 ? nullptr : xmid.as<float>(), embed.as<float>(),
                                     st(), (int)vocab, zeros_h.as<float>(), prev, xin.as<float>(),
                                     an(l), eps, (int)h, s_qkv, Ly.f_qkv, s));
      SYN_TRY(trace_end(SYN_HIP_STEP_QKV, s));
      SYN_TRY(trace_begin(s));
      SYN_TRY(launch_fused_attention(Ly.f_qkv.rows(s_qkv), nh, nkv, (int)hd, qn(l), kn(l), eps,
                                     rope_cos.as<float>(),
                                     rope_sin.as<float>(), st(), kc_l(l), vc_l(l), (int)S,
                                     scores.as<float>(), attn.as<float>(), s));
      SYN_TRY(trace_end(SYN_HIP_STEP_ATTENTION, s));
      SYN_TRY(trace_begin(s));
      SYN_TRY(launch_fused_quant_gemv(attn.as<float>(), (int)qd, s_o, Ly.f_o, s));
      SYN_TRY(trace_end(SYN_HIP_STEP_O, s));
      if (gu_swiglu_fits((int)h, (int)inter)) {
        // gate|up split over K in pairs of panels with the SwiGLU epilogue in
        // each pair's last slice, then the down GEMV quantizes only its K
        // range of h with the published max
        unsigned *hmax = reinterpret_cast<unsigned *>(acc.as<int>() + acc_elems) -
                         round_up(L, 64) + l;
        SYN_TRY(trace_begin(s));
        SYN_TRY(launch_gu_swiglu(xin.as<float>(), Ly.f_o.rows(s_o), xmid.as<float>(), fn(l), eps,
                                 (int)h, s_gu, Ly.f_gup, Ly.gu.scales.as<float>(), (int)inter,
                                 gu.as<float>(), hmax, s));
        SYN_TRY(trace_end(SYN_HIP_STEP_GATE_UP, s));
        SYN_TRY(trace_begin(s));
        SYN_TRY(launch_fused_hq_gemv(gu.as<float>(), hmax, (int)inter, s_down, Ly.f_down, s));
        SYN_TRY(trace_end(SYN_HIP_STEP_DOWN, s));
      } else {
        SYN_TRY(trace_begin(s));
        SYN_TRY(launch_fused_norm_gemv(xin.as<float>(), nullptr, st(), (int)vocab, nullptr,
                                       Ly.f_o.rows(s_o), xmid.as<float>(), fn(l), eps,
                                       (int)h, s_gu, Ly.f_gu, s));
        SYN_TRY(trace_end(SYN_HIP_STEP_GATE_UP, s));
        SYN_TRY(trace_begin(s));
        SYN_TRY(launch_fused_swiglu_gemv(Ly.f_gu.rows(s_gu), (int)inter, s_down, Ly.f_down, s));
        SYN_TRY(trace_end(SYN_HIP_STEP_DOWN, s));
      }
    }
    SYN_TRY(trace_begin(s));
    SYN_TRY(launch_fused_final_norm(xmid.as<float>(), layers[L - 1].f_down.rows(s_down),
                                    final_nw.as<float>(), eps, (int)h, xq.as<int8_t>(), s_head, s));
    SYN_TRY(trace_end(SYN_HIP_STEP_FINAL_NORM, s));
    SYN_TRY(trace_begin(s));
    SYN_TRY(launch_lmhead_top2(lm_head.w.p, lm_head.scales.as<float>(), (int)vocab,
                               lm_head.chunks, xq.as<int8_t>(), s_head, logits.as<float>(),
                               pv.as<float>(), pi.as<int>(), pv2.as<float>(), s));
    SYN_TRY(trace_end(SYN_HIP_STEP_LM_HEAD, s));
    SYN_TRY(trace_begin(s));
    if (sampling)
      SYN_TRY(launch_sample(logits.as<float>(), (int)vocab, history.as<uint32_t>(), 0, sargs,
                            u_draws.as<float>(), st(), 1, history.as<uint32_t>(),
                            mhist.as<float>(), sscr, nullptr, s));
    else
      SYN_TRY(launch_argmax_advance(pv.as<float>(), pi.as<int>(), pv2.as<float>(),
                                    (int)cdiv(vocab, 64), st(), history.as<uint32_t>(),
                                    mhist.as<float>(), s));
    return trace_end(SYN_HIP_STEP_SELECT, s);
  }

  // sampler settings; the captured decode step changes with them
  syn_status_t set_sampler(const syn_hip_sampler *p, uint64_t seed) {
    SYN_HIP(hipStreamSynchronize(stream));
    if (graph) {
      (void)hipGraphExecDestroy(graph);
      graph = nullptr;
    }
    if (!p) {
      sampling = false;
      return SYN_OK;
    }
    if (!(p->temperature == p->temperature) || !(p->top_p == p->top_p) ||
        !(p->repetition_penalty == p->repetition_penalty)) {
      set_error("sampler parameters must not be NaN");
      return SYN_ERR_INVALID_ARG;
    }
    sargs = make_sample_args(*p);
    SYN_TRY(sscr.ensure(vocab));
    std::vector<float> u(S + 1);
    host_stdrng_f32(seed, u.size(), u.data());
    SYN_TRY(u_draws.alloc(u.size() * 4));
    SYN_HIP(hipMemcpy(u_draws.p, u.data(), u.size() * 4, hipMemcpyHostToDevice));
    sampling = true;
    return SYN_OK;
  }

  // one decode step on the model stream: graph replay or eager launches
  syn_status_t run_step() {
    if (!use_graph) return decode_step(stream);
    SYN_TRY(build_graph());
    SYN_HIP(hipGraphLaunch(graph, stream));
    return SYN_OK;
  }

  syn_status_t set_options(int fused_decode, int graph_replay) {
    const bool f = fused_decode != 0 && fused_supported();
    if (fused_decode && !f) {
      set_error("fused decode: shape outside the fused kernels' LDS limits");
      return SYN_ERR_INVALID_ARG;
    }
    if (f != fused && graph) {
      SYN_HIP(hipStreamSynchronize(stream));
      (void)hipGraphExecDestroy(graph);
      graph = nullptr;
    }
    fused = f;
    use_graph = graph_replay != 0;
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

  syn_status_t set_state(int pos, uint32_t token, int step) {
    StepState hs{pos, token, step, 0.0f};
    // synchronous: hs lives on this stack frame
    SYN_HIP(hipMemcpyAsync(state.p, &hs, sizeof(hs), hipMemcpyHostToDevice, stream));
    SYN_HIP(hipStreamSynchronize(stream));
    return SYN_OK;
  }

  syn_status_t get_state(StepState *out) {
    SYN_HIP(hipMemcpyAsync(out, state.p, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    SYN_HIP(hipStreamSynchronize(stream));
    return SYN_OK;
  }

  // the layers of QuantizedCausalLM::forward_prefill (int8.rs:593-618) over
  // n tokens whose ids are on the device, appended at cache rows cache_off ..
  syn_status_t prefill_rows(const uint32_t *d_ids, int n, int cache_off) {
    SYN_TRY(launch_embed(embed.as<float>(), d_ids, n, (int)h, (int)vocab, x.as<float>(), stream));
    for (size_t l = 0; l < L; l++) SYN_TRY(layer(l, n, true, stream, cache_off));
    return SYN_OK;
  }

  // forward_prefill into an empty cache (the pipeline's fresh ModelState)
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

  // forward_prefill into the cache as it stands: the n new rows are appended
  // after the cached ones, rotated at positions 0..n-1 and attending among
  // themselves (cached_attention_prefill, ops/attention.rs:153-247)
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

  // KvCache.truncateTo (kvcache.zig:109-113): only a shorter length applies
  syn_status_t truncate(size_t new_len) {
    StepState cur;
    SYN_TRY(get_state(&cur));
    if (new_len < (size_t)cur.pos) SYN_TRY(set_state((int)new_len, cur.token, cur.step));
    return SYN_OK;
  }

  // TextGenerator::generate_speculative (pipeline.rs:281-395) with max_new
  // as the only stop condition.  QuantizedCausalLM has no draft forward
  // (int8.rs:739), so a draft token is a full forward_one; the verify pass is
  // forward_prefill of [last accepted, drafts] after truncating the cache to
  // the round's start, its logits unused; every draft is accepted; when all k
  // were, a bonus token comes from forward_one of the last draft.  Drafts
  // sample with the penalty history as it stood at the round's start
  // (generated_tokens); draw i of the seeded stream goes to sample call i.
  // The loop runs on the stream without a host round trip: positions and
  // counts follow from k and max_new alone.
  syn_status_t generate_speculative(const uint32_t *prompt, size_t n_prompt, size_t max_new,
                                    size_t k) {
    if (n_prompt == 0 || n_prompt > S) {
      set_error("prefill length must be in [1, max_seq]");
      return SYN_ERR_INVALID_ARG;
    }
    // the rows and sample calls the loop will use
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
      // draft: k forward_one + sample, penalty history = the s0 generated tokens
      SYN_TRY(launch_state_set(st(), -1, (int)s0, stream));
      for (size_t i = 0; i < k; i++) SYN_TRY(run_step());
      // truncate to save, verify [history[s0-1], drafts] at cache rows save ..
      SYN_TRY(prefill_rows(history.as<uint32_t>() + (s0 - 1), (int)(k + 1), (int)save));
      SYN_TRY(launch_state_set(st(), (int)(save + k + 1), -1, stream));
      const size_t acc = std::min(k, max_new - gen);
      gen += acc;
      pos = save + k + 1;
      if (acc == k && gen < max_new) {  // bonus token
        SYN_TRY(run_step());
        gen += 1;
        pos += 1;
      }
    }
    return SYN_OK;
  }
};

static syn_status_t check_model(syn_hip_qlm_t *m) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (!m->finalized) {
    set_error("model not finalized");
    return SYN_ERR_INVALID_ARG;
  }
  return SYN_OK;
}

extern "C" {

syn_status_t syn_hip_qlm_create(const syn_hip_lm_config *cfg, syn_hip_qlm_t **out) {
  if (!cfg || !out) return SYN_ERR_NULL_PTR;
  if (!cfg->hidden || !cfg->n_layers || !cfg->n_heads || !cfg->n_kv_heads || !cfg->head_dim ||
      !cfg->inter || !cfg->vocab || !cfg->max_seq || cfg->n_heads % cfg->n_kv_heads ||
      cfg->head_dim % 2 || cfg->head_dim > 1024)
    return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  auto *m = new syn_hip_qlm_s();
  m->c = *cfg;
  m->h = cfg->hidden;
  m->hd = cfg->head_dim;
  m->qd = (size_t)cfg->n_heads * cfg->head_dim;
  m->kvd = (size_t)cfg->n_kv_heads * cfg->head_dim;
  m->inter = cfg->inter;
  m->L = cfg->n_layers;
  m->vocab = cfg->vocab;
  m->S = cfg->max_seq;
  m->ldh = round_up(m->h, 16);
  m->ldq = round_up(m->qd, 16);
  m->ldi = round_up(m->inter, 16);
  m->n_qkv = m->qd + 2 * m->kvd;
  m->layers.resize(m->L);
  m->have_layer.assign(m->L, 0);
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

syn_status_t syn_hip_qlm_set_embed(syn_hip_qlm_t *m, const float *embed) {
  if (!m || !embed) return SYN_ERR_NULL_PTR;
  const size_t n = m->vocab * m->h;
  m->host_embed.assign(embed, embed + n);
  SYN_TRY(m->embed.alloc(n * 4));
  SYN_HIP(hipMemcpy(m->embed.p, embed, n * 4, hipMemcpyHostToDevice));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_set_layer(syn_hip_qlm_t *m, uint32_t layer, const float *wq,
                                   const float *wk, const float *wv, const float *wo,
                                   const float *wg, const float *wu, const float *wd) {
  if (!m || !wq || !wk || !wv || !wo || !wg || !wu || !wd) return SYN_ERR_NULL_PTR;
  if (layer >= m->L) return SYN_ERR_INVALID_ARG;
  return m->set_layer(layer, wq, wk, wv, wo, wg, wu, wd);
}

syn_status_t syn_hip_qlm_set_lm_head(syn_hip_qlm_t *m, const float *w) {
  if (!m || !w) return SYN_ERR_NULL_PTR;
  if (m->finalized) {
    set_error("lm_head must be set before finalize");
    return SYN_ERR_INVALID_ARG;
  }
  m->host_lm_head.assign(w, w + m->vocab * m->h);
  return SYN_OK;
}

syn_status_t syn_hip_qlm_set_norms(syn_hip_qlm_t *m, uint32_t layer, const float *attn_norm,
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

syn_status_t syn_hip_qlm_set_final_norm(syn_hip_qlm_t *m, const float *norm) {
  if (!m || !norm) return SYN_ERR_NULL_PTR;
  SYN_HIP(hipMemcpy(m->final_nw.p, norm, m->h * 4, hipMemcpyHostToDevice));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_set_qk_norm(syn_hip_qlm_t *m, int enabled) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (m->finalized) {
    set_error("qk_norm must be chosen before finalize");
    return SYN_ERR_INVALID_ARG;
  }
  m->qk_norm = enabled != 0;
  return SYN_OK;
}

// --------------------------------------------------------- weight files
// Every tensor of the model by HuggingFace names (the reference's weight
// map, weight_map.rs; fused qkv_proj / gate_up_proj split as
// split_fused_projections does, weight_map.rs:780-829, by the q/k/v widths)
// or llama.cpp's GGUF names; converted to f32 as the reference's loaders do,
// then quantized like quantize_model (int8.rs:78-152).
static syn_status_t qlm_load(syn_hip_qlm_t *m, const WeightSource &src) {
  const size_t h = m->h, hd = m->hd, qd = m->qd, kvd = m->kvd, inter = m->inter;
  TensorView t;
  auto need = [&](bool ok, const std::string &what) -> syn_status_t {
    if (ok) return SYN_OK;
    set_error("weights: no tensor for " + what);
    return SYN_ERR_INVALID_ARG;
  };
  auto shape_err = [&](const TensorView &v, const std::string &want) -> syn_status_t {
    std::string got;
    for (int d = 0; d < v.n_dims; d++) got += (d ? "x" : "") + std::to_string(v.shape[d]);
    set_error("weights: tensor " + v.name + " is " + got + ", the model expects " + want);
    return SYN_ERR_SHAPE_MISMATCH;
  };
  auto matrix = [&](const TensorView &v, size_t rows, size_t cols,
                    std::vector<float> &out) -> syn_status_t {
    if (!v.is_matrix(rows, cols)) return shape_err(v, std::to_string(rows) + "x" + std::to_string(cols));
    out.resize(rows * cols);
    return tensor_to_f32(v, out.data());
  };
  auto vec = [&](const TensorView &v, size_t n, std::vector<float> &out) -> syn_status_t {
    if (!v.is_vector(n)) return shape_err(v, std::to_string(n));
    out.resize(n);
    return tensor_to_f32(v, out.data());
  };
  static const char *kHf[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                               "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                               "mlp.down_proj"};
  static const char *kLlama[7] = {"attn_q", "attn_k", "attn_v", "attn_output",
                                  "ffn_gate", "ffn_up", "ffn_down"};
  const size_t rows[7] = {qd, kvd, kvd, h, inter, inter, h};
  const size_t cols[7] = {h, h, h, qd, h, h, inter};
  // head norms: the reference applies them when the weights exist
  const bool qk = src.find_any({"model.layers.0.self_attn.q_norm.weight",
                                "blk.0.attn_q_norm.weight"}, &t);
  SYN_TRY(syn_hip_qlm_set_qk_norm(m, qk ? 1 : 0));
  std::vector<std::vector<float>> w(7);
  for (size_t l = 0; l < m->L; l++) {
    const std::string hf = "model.layers." + std::to_string(l) + ".";
    const std::string bl = "blk." + std::to_string(l) + ".";
    for (int p = 0; p < 7; p++) {
      if (src.find_any({hf + kHf[p] + ".weight", bl + kLlama[p] + ".weight"}, &t)) {
        SYN_TRY(matrix(t, rows[p], cols[p], w[p]));
      } else if (p <= 2 && src.find(hf + "self_attn.qkv_proj.weight", &t)) {
        std::vector<float> all;
        SYN_TRY(matrix(t, qd + 2 * kvd, h, all));
        const size_t r0 = p == 0 ? 0 : p == 1 ? qd : qd + kvd;
        w[p].assign(all.begin() + r0 * h, all.begin() + (r0 + rows[p]) * h);
      } else if ((p == 4 || p == 5) && src.find(hf + "mlp.gate_up_proj.weight", &t)) {
        std::vector<float> all;
        SYN_TRY(matrix(t, 2 * inter, h, all));
        const size_t r0 = p == 4 ? 0 : inter;
        w[p].assign(all.begin() + r0 * h, all.begin() + (r0 + inter) * h);
      } else {
        return need(false, hf + kHf[p] + ".weight");
      }
    }
    SYN_TRY(m->set_layer(l, w[0].data(), w[1].data(), w[2].data(), w[3].data(), w[4].data(),
                         w[5].data(), w[6].data()));
    std::vector<float> an, fn, qn, kn;
    if (src.find_any({hf + "input_layernorm.weight", bl + "attn_norm.weight"}, &t))
      SYN_TRY(vec(t, h, an));
    if (src.find_any({hf + "post_attention_layernorm.weight", bl + "ffn_norm.weight"}, &t))
      SYN_TRY(vec(t, h, fn));
    if (qk) {
      SYN_TRY(need(src.find_any({hf + "self_attn.q_norm.weight", bl + "attn_q_norm.weight"}, &t),
                   hf + "self_attn.q_norm.weight"));
      SYN_TRY(vec(t, hd, qn));
      SYN_TRY(need(src.find_any({hf + "self_attn.k_norm.weight", bl + "attn_k_norm.weight"}, &t),
                   hf + "self_attn.k_norm.weight"));
      SYN_TRY(vec(t, hd, kn));
    }
    SYN_TRY(syn_hip_qlm_set_norms(m, (uint32_t)l, an.empty() ? nullptr : an.data(),
                                  fn.empty() ? nullptr : fn.data(),
                                  qn.empty() ? nullptr : qn.data(),
                                  kn.empty() ? nullptr : kn.data()));
  }
  std::vector<float> v;
  SYN_TRY(need(src.find_any({"model.embed_tokens.weight", "token_embd.weight"}, &t),
               "model.embed_tokens.weight"));
  SYN_TRY(matrix(t, m->vocab, h, v));
  SYN_TRY(syn_hip_qlm_set_embed(m, v.data()));
  if (src.find_any({"model.norm.weight", "output_norm.weight"}, &t)) {
    SYN_TRY(vec(t, h, v));
    SYN_TRY(syn_hip_qlm_set_final_norm(m, v.data()));
  }
  if (src.find_any({"lm_head.weight", "output.weight"}, &t)) {
    SYN_TRY(matrix(t, m->vocab, h, v));
    SYN_TRY(syn_hip_qlm_set_lm_head(m, v.data()));
  }
  return SYN_OK;
}

syn_status_t syn_hip_qlm_load_gguf(syn_hip_qlm_t *m, const syn_hip_gguf_t *g) {
  if (!m || !g) return SYN_ERR_NULL_PTR;
  if (m->finalized) {
    set_error("weights must be loaded before finalize");
    return SYN_ERR_INVALID_ARG;
  }
  return qlm_load(m, *gguf_source(g));
}

syn_status_t syn_hip_qlm_load_safetensors(syn_hip_qlm_t *m, const syn_hip_safetensors_t *st) {
  if (!m || !st) return SYN_ERR_NULL_PTR;
  if (m->finalized) {
    set_error("weights must be loaded before finalize");
    return SYN_ERR_INVALID_ARG;
  }
  return qlm_load(m, *safetensors_source(st));
}

syn_status_t syn_hip_qlm_init_synthetic(syn_hip_qlm_t *m, uint64_t seed_base, float stddev) {
  if (!m) return SYN_ERR_NULL_PTR;
  const size_t h = m->h;
  {
    std::vector<float> emb(m->vocab * h);
    fill_normal_parallel(emb.data(), emb.size(), seed_base + 0, stddev);
    SYN_TRY(syn_hip_qlm_set_embed(m, emb.data()));
  }
  const size_t rows[7] = {m->qd, m->kvd, m->kvd, h, m->inter, m->inter, h};
  const size_t cols[7] = {h, h, h, m->qd, h, h, m->inter};
  std::vector<std::vector<float>> w(7);
  for (int t = 0; t < 7; t++) w[t].resize(rows[t] * cols[t]);
  for (size_t l = 0; l < m->L; l++) {
    std::vector<std::thread> th;
    for (int t = 0; t < 7; t++)
      th.emplace_back([&, t] {
        fill_normal(w[t].data(), w[t].size(), seed_base + 1 + 8 * l + (uint64_t)t, stddev);
      });
    for (auto &x : th) x.join();
    SYN_TRY(m->set_layer(l, w[0].data(), w[1].data(), w[2].data(), w[3].data(), w[4].data(),
                         w[5].data(), w[6].data()));
  }
  return SYN_OK;
}

syn_status_t syn_hip_qlm_finalize(syn_hip_qlm_t *m) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (m->host_embed.empty()) {
    set_error("embed_tokens not set");
    return SYN_ERR_INVALID_ARG;
  }
  for (size_t l = 0; l < m->L; l++)
    if (!m->have_layer[l]) {
      set_error("layer " + std::to_string(l) + " not set");
      return SYN_ERR_INVALID_ARG;
    }
  // lm_head quantized from its own weight, else tied to embed_tokens
  // (int8.rs:125-139)
  const std::vector<float> &lm = m->host_lm_head.empty() ? m->host_embed : m->host_lm_head;
  SYN_TRY(m->lm_head.from_f32(lm.data(), m->vocab, m->h));
  std::vector<float>().swap(m->host_embed);
  std::vector<float>().swap(m->host_lm_head);
  // RoPE tables, models/lm/builder.rs:88-133 (glibc powf/cosf/sinf, as Rust f32)
  const size_t half = m->hd / 2;
  std::vector<float> cs(m->S * half), sn(m->S * half);
  const float fb = (float)m->c.rope_theta;
  for (size_t pos = 0; pos < m->S; pos++)
    for (size_t i = 0; i < half; i++) {
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
  SYN_TRY(m->prepare_fused());
  m->fused = m->fused_supported();
  m->finalized = true;
  SYN_TRY(m->set_state(0, 0, 0));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_reset(syn_hip_qlm_t *m) {
  SYN_TRY(check_model(m));
  SYN_TRY(m->set_state(0, 0, 0));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_forward_prefill(syn_hip_qlm_t *m, const uint32_t *ids, size_t n,
                                         float *host_logits) {
  SYN_TRY(check_model(m));
  if (!ids) return SYN_ERR_NULL_PTR;
  SYN_TRY(m->prefill(ids, n));
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_forward_prefill_append(syn_hip_qlm_t *m, const uint32_t *ids,
                                                size_t n, float *host_logits) {
  SYN_TRY(check_model(m));
  if (!ids) return SYN_ERR_NULL_PTR;
  SYN_TRY(m->prefill_append(ids, n));
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_truncate(syn_hip_qlm_t *m, size_t new_len) {
  SYN_TRY(check_model(m));
  return m->truncate(new_len);
}

syn_status_t syn_hip_qlm_cache_len(syn_hip_qlm_t *m, size_t *out_len) {
  SYN_TRY(check_model(m));
  if (!out_len) return SYN_ERR_NULL_PTR;
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  *out_len = (size_t)cur.pos;
  return SYN_OK;
}

syn_status_t syn_hip_qlm_forward_one(syn_hip_qlm_t *m, uint32_t token, float *host_logits) {
  SYN_TRY(check_model(m));
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos >= m->S) {
    set_error("KV cache full");  // kvcache.zig:68-69 CacheFull
    return SYN_ERR_INVALID_ARG;
  }
  if (m->use_graph) SYN_TRY(m->build_graph());
  SYN_TRY(m->set_state(cur.pos, token, cur.step));
  SYN_TRY(m->run_step());
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->vocab * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_generate(syn_hip_qlm_t *m, const uint32_t *prompt, size_t n_prompt,
                                  size_t max_new, uint32_t *out_tokens, float *out_margins) {
  SYN_TRY(check_model(m));
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

syn_status_t syn_hip_qlm_generate_speculative(syn_hip_qlm_t *m, const uint32_t *prompt,
                                              size_t n_prompt, size_t max_new, size_t k,
                                              uint32_t *out_tokens, float *out_margins) {
  SYN_TRY(check_model(m));
  if (!prompt || !out_tokens) return SYN_ERR_NULL_PTR;
  if (k == 0) return syn_hip_qlm_generate(m, prompt, n_prompt, max_new, out_tokens, out_margins);
  if (max_new == 0) return SYN_OK;
  SYN_TRY(m->generate_speculative(prompt, n_prompt, max_new, k));
  SYN_HIP(hipMemcpyAsync(out_tokens, m->history.p, max_new * 4, hipMemcpyDeviceToHost,
                         m->stream));
  if (out_margins)
    SYN_HIP(hipMemcpyAsync(out_margins, m->mhist.p, max_new * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_qlm_decode_timed(syn_hip_qlm_t *m, size_t steps, float *elapsed_ms) {
  SYN_TRY(check_model(m));
  if (!elapsed_ms) return SYN_ERR_NULL_PTR;
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos + steps > m->S) {
    set_error("decode steps exceed max_seq");
    return SYN_ERR_INVALID_ARG;
  }
  if (m->use_graph) SYN_TRY(m->build_graph());
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  SYN_HIP(hipEventRecord(a, m->stream));
  for (size_t i = 0; i < steps; i++) SYN_TRY(m->run_step());
  SYN_HIP(hipEventRecord(b, m->stream));
  SYN_HIP(hipEventSynchronize(b));
  SYN_HIP(hipEventElapsedTime(elapsed_ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return SYN_OK;
}

syn_status_t syn_hip_qlm_time_lm_head(syn_hip_qlm_t *m, size_t iters, size_t flush_bytes,
                                      float *avg_ms) {
  SYN_TRY(check_model(m));
  if (!avg_ms) return SYN_ERR_NULL_PTR;
  if (iters == 0) return SYN_ERR_INVALID_ARG;
  DevBuf flush;
  if (flush_bytes) SYN_TRY(flush.alloc(flush_bytes));
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  double total = 0.0;
  syn_status_t st = SYN_OK;
  for (size_t i = 0; i < iters && st == SYN_OK; i++) {
    if (flush_bytes) SYN_HIP(hipMemsetAsync(flush.p, (int)(i & 0xff), flush_bytes, m->stream));
    SYN_HIP(hipEventRecord(a, m->stream));
    // the kernel the decode step runs: the fused step's lm_head with per-panel
    // top-2, or the plain GEMV of the one-kernel-per-op step
    if (m->fused)
      st = launch_lmhead_top2(m->lm_head.w.p, m->lm_head.scales.as<float>(), (int)m->vocab,
                              m->lm_head.chunks, m->xq.as<int8_t>(), m->sx.as<float>(),
                              m->logits.as<float>(), m->pv.as<float>(), m->pi.as<int>(),
                              m->pv2.as<float>(), m->stream);
    else
      st = m->lm_head.gemv(1, m->xq.as<int8_t>(), m->ldh, m->sx.as<float>(),
                           m->logits.as<float>(), m->vocab, m->stream);
    SYN_HIP(hipEventRecord(b, m->stream));
    SYN_HIP(hipEventSynchronize(b));
    float ms = 0.0f;
    SYN_HIP(hipEventElapsedTime(&ms, a, b));
    total += ms;
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  SYN_TRY(st);
  *avg_ms = (float)(total / (double)iters);
  return SYN_OK;
}

syn_status_t syn_hip_qlm_set_options(syn_hip_qlm_t *m, int fused_decode, int graph_replay) {
  SYN_TRY(check_model(m));
  return m->set_options(fused_decode, graph_replay);
}

syn_status_t syn_hip_qlm_set_sampler(syn_hip_qlm_t *m, const syn_hip_sampler *params,
                                     uint64_t seed) {
  SYN_TRY(check_model(m));
  return m->set_sampler(params, seed);
}

syn_status_t syn_hip_qlm_time_step_kernels(syn_hip_qlm_t *m, size_t steps, float *avg_us,
                                           uint32_t *launches) {
  SYN_TRY(check_model(m));
  if (!avg_us || !launches) return SYN_ERR_NULL_PTR;
  if (!m->fused) {
    set_error("time_step_kernels: the fused decode step only");
    return SYN_ERR_INVALID_ARG;
  }
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if (steps == 0 || (size_t)cur.pos + steps > m->S) {
    set_error("time_step_kernels: steps must be in [1, max_seq - cached rows]");
    return SYN_ERR_INVALID_ARG;
  }
  std::vector<syn_hip_qlm_s::TraceEntry> tr;
  tr.reserve(steps * (5 * m->L + 4));
  m->trace = &tr;
  syn_status_t st = SYN_OK;
  for (size_t i = 0; i < steps && st == SYN_OK; i++) st = m->decode_step(m->stream);
  m->trace = nullptr;
  launch_events() = LaunchEvents{};
  hipError_t e = hipStreamSynchronize(m->stream);
  double sum[SYN_HIP_STEP_KINDS] = {};
  uint32_t cnt[SYN_HIP_STEP_KINDS] = {};
  for (const auto &t : tr) {
    float ms = 0.0f;
    if (st == SYN_OK && e == hipSuccess && hipEventElapsedTime(&ms, t.start, t.end) == hipSuccess &&
        t.kind >= 0 && t.kind < SYN_HIP_STEP_KINDS) {
      sum[t.kind] += ms;
      cnt[t.kind]++;
    }
    (void)hipEventDestroy(t.start);
    (void)hipEventDestroy(t.end);
  }
  SYN_TRY(st);
  SYN_HIP(e);
  for (int k = 0; k < SYN_HIP_STEP_KINDS; k++) {
    launches[k] = cnt[k];
    avg_us[k] = cnt[k] ? (float)(sum[k] / cnt[k] * 1e3) : 0.0f;
  }
  return SYN_OK;
}

syn_status_t syn_hip_qlm_time_lm_head_rotating(syn_hip_qlm_t *m, size_t iters, float *avg_ms) {
  SYN_TRY(check_model(m));
  if (!avg_ms) return SYN_ERR_NULL_PTR;
  if (iters == 0) return SYN_ERR_INVALID_ARG;
  if (!m->fused) {
    set_error("rotating lm_head timing measures the fused decode step's kernel");
    return SYN_ERR_INVALID_ARG;
  }
  // a second copy of the weights: alternating launches stream 2 x 156 MB,
  // more than the Infinity Cache holds, so every launch reads HBM
  DevBuf w2, s2;
  SYN_TRY(w2.alloc(m->lm_head.w.bytes));
  SYN_TRY(s2.alloc(m->lm_head.scales.bytes));
  SYN_HIP(hipMemcpyAsync(w2.p, m->lm_head.w.p, w2.bytes, hipMemcpyDeviceToDevice, m->stream));
  SYN_HIP(hipMemcpyAsync(s2.p, m->lm_head.scales.p, s2.bytes, hipMemcpyDeviceToDevice,
                         m->stream));
  auto launch = [&](size_t i) -> syn_status_t {
    const void *W = (i & 1) ? w2.p : m->lm_head.w.p;
    const float *ws = (i & 1) ? s2.as<float>() : m->lm_head.scales.as<float>();
    return launch_lmhead_top2(W, ws, (int)m->vocab, m->lm_head.chunks, m->xq.as<int8_t>(),
                              m->sx.as<float>(), m->logits.as<float>(), m->pv.as<float>(),
                              m->pi.as<int>(), m->pv2.as<float>(), m->stream);
  };
  SYN_TRY(launch(0));
  SYN_TRY(launch(1));
  SYN_HIP(hipStreamSynchronize(m->stream));
  hipEvent_t a, b;
  SYN_HIP(hipEventCreate(&a));
  SYN_HIP(hipEventCreate(&b));
  SYN_HIP(hipEventRecord(a, m->stream));
  syn_status_t st = SYN_OK;
  for (size_t i = 0; i < iters && st == SYN_OK; i++) st = launch(i);
  SYN_HIP(hipEventRecord(b, m->stream));
  SYN_HIP(hipEventSynchronize(b));
  float ms = 0.0f;
  SYN_HIP(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  SYN_TRY(st);
  *avg_ms = ms / (float)iters;
  return SYN_OK;
}

syn_status_t syn_hip_qlm_destroy(syn_hip_qlm_t *m) {
  if (m) {
    (void)hipStreamSynchronize(m->stream);
    delete m;
  }
  return SYN_OK;
}

}  // extern "C"
