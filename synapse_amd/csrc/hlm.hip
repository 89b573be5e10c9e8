// Hybrid LFM2.5 decoder on the device, Q4 decode path: HybridModel::decode_one
// (models/ssm/hybrid/model.rs:240-290) over LIV conv and GQA decoder layers
// (layer.rs:593-654, 878-954, 1055-1078) after quantize_for_decode
// (layer.rs:570-581, 832-846): every projection is Q4_0 (f32 activations),
// q|k|v and gate|up stacked into one handle each (their rows are
// independent), the lm_head the tied f32 embedding.  Two forms of the step,
// both compared with the oracle by tolerance:
//
// - fused (the default when the shapes fit): four kernels per LIV conv layer
//   and five per GQA layer on the fused split-K GEMV of klm_fused.hip (the
//   Q4_0 planes as a fourth format; RMSNorm, the LIV conv step and the
//   attention chunk combine in GEMV prologues, SwiGLU in an epilogue,
//   fixed-point split-K atomics), the chunked attention of klm_fused.hip,
//   and head_f32.hip's tree-ordered f32 lm_head with per-panel top-2;
// - op-by-op: one kernel per op with the q4_0GemvRow GEMV of q4_0.hip, whose
//   split-K partials the consuming kernels sum (PartRows), the small ops in
//   the reference's float order except RMSNorm's sum of squares
//   (pure_rust_ops.rs:96-112's formula, tree-ordered sum): the double-gated
//   conv step (B*x, shift, sequential tap sum, C*y), head norms with
//   x * (w * s), rotate-half RoPE, attention with sequential dot products,
//   softmax_slice and a sequential P.V, SwiGLU silu(g) * u with glibc's
//   expf, and the lm_head in f32GemvRow order (the exact-order GEMV of
//   mamba.hip).
//
// The reference prefills on the CPU with f32 weights and then decodes on the
// GPU (examples/lfm25_inference.rs:86-99); this decoder feeds a prompt
// through the decode step (Q4 weights), one token at a time.
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "decode_fused.hpp"
#include "f32_ops.hpp"
#include "head_f32.hpp"
#include "klm_fused.hpp"
#include "layer_ops.hpp"
#include "linear.hpp"
#include "liv_conv.hpp"
#include "reduce_order.hpp"

namespace syn {

// Output row `row` of a Q4_0 GEMV from its split-K partials (PartRows):
// summed from 0.0f in slice order (deterministic: every consumer of a row
// sees the same value).
__device__ __forceinline__ float part_row(const PartRows &r, int row) {
  if (r.ks == 1) return r.p[row];
  float s = 0.0f;
  for (int k = 0; k < r.ks; k++) s += r.p[(size_t)k * r.stride + row];
  return s;
}

// The LIV conv step (liv_conv_channel) of the in_proj output, read from the
// Q4 GEMV's split-K partials: proj = [B | C | x], one thread per channel,
// the state half of the position read and the next one written.
__global__ void __launch_bounds__(256)
    k_hlm_conv(PartRows proj, int inner, int ck, const StepState *__restrict__ st,
               float *__restrict__ state, const float *__restrict__ w,
               const float *__restrict__ bias, float *__restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= inner) return;
  const int pos = st->pos;
  const size_t half = (size_t)inner * ck;
  const float *sold = state + (size_t)(pos & 1) * half + (size_t)i * ck;
  float *snew = state + (size_t)((pos + 1) & 1) * half + (size_t)i * ck;
  out[i] = liv_conv_channel(part_row(proj, i), part_row(proj, inner + i),
                            part_row(proj, 2 * inner + i), ck, sold, snew, w + (size_t)i * ck,
                            bias ? bias + i : nullptr);
}

// Heads of the stacked q|k|v row, one wave each: q heads [0, nh) get the
// q head norm and RoPE (-> q_out), k heads [nh, nh + nkv) the k norm and
// RoPE (-> K cache row pos), v heads are copied to the V cache row pos.
// Head norm layer.rs:865-876, RoPE layer.rs:848-863 at position pos.
__global__ void __launch_bounds__(64)
    k_hlm_qk(PartRows qkv, int nh, int nkv, int hd,
             const float *__restrict__ qn, const float *__restrict__ kn, float eps,
             const float *__restrict__ cosT, const float *__restrict__ sinT,
             const StepState *__restrict__ st, int S, float *__restrict__ q_out,
             float *__restrict__ kc, float *__restrict__ vc) {
  extern __shared__ __align__(16) float hv[];  // the head [hd] | its squares [hd]
  float *sq = hv + ((hd + 3) & ~3);
  const int h = blockIdx.x, lane = threadIdx.x;
  const int pos = st->pos, half = hd >> 1;
  const int src = h * hd;
  if (h >= nh + nkv) {  // v head
    const int g = h - nh - nkv;
    for (int d = lane; d < hd; d += 64) vc[kv_v_index(pos, g, d, hd, S)] = part_row(qkv, src + d);
    return;
  }
  for (int d = lane; d < hd; d += 64) {
    const float v = part_row(qkv, src + d);
    hv[d] = v;
    sq[d] = v * v;
  }
  __syncthreads();
  const float s = wave_seq_sum(sq, hd, -0.0f);
  const float scale = 1.0f / sqrtf(s / (float)hd + eps);
  const float *w = h < nh ? qn : kn;
  __syncthreads();
  for (int d = lane; d < hd; d += 64) {
    const float ws = w[d] * scale;
    hv[d] = hv[d] * ws;
  }
  __syncthreads();
  const float *cr = cosT + (size_t)pos * half, *sr = sinT + (size_t)pos * half;
  for (int i = lane; i < half; i += 64) {
    const float x1 = hv[i], x2 = hv[half + i], c = cr[i], sn = sr[i];
    const float a = x1 * c, b = x2 * sn, e = x2 * c, f = x1 * sn;
    if (h < nh) {
      q_out[(size_t)h * hd + i] = a - b;
      q_out[(size_t)h * hd + half + i] = e + f;
    } else {
      kc[kv_k_index(pos, h - nh, i, hd, S)] = a - b;
      kc[kv_k_index(pos, h - nh, half + i, hd, S)] = e + f;
    }
  }
}

// layer.rs:907-951 for one query head per workgroup over the seq = pos + 1
// cached positions: scores (sequential q.k) * scale, softmax_slice
// (activation.rs:117-129: max, exp in order with a sequential sum, divide),
// P.V as one sequential chain per output column.  The score row sits in
// dynamic LDS (max_seq rounded to 4 floats).
__global__ void __launch_bounds__(256)
    k_hlm_attn(const float *__restrict__ q, const float *__restrict__ kc,
               const float *__restrict__ vc, const StepState *__restrict__ st, int nh, int nkv,
               int hd, int S, float scale, float *__restrict__ out) {
  extern __shared__ __align__(16) float row[];
  __shared__ float qs[256];
  __shared__ float red[4];
  __shared__ float s_sum;
  const int qh = blockIdx.x, tid = threadIdx.x;
  const int kvh = qh / (nh / nkv), seq = st->pos + 1;
  for (int d = tid; d < hd; d += 256) qs[d] = q[(size_t)qh * hd + d];
  __syncthreads();
  float mx = -INFINITY;
  for (int p = tid; p < seq; p += 256) {
    float dot = 0.0f;
    for (int d = 0; d < hd; d++) {
      const float t = qs[d] * kc[kv_k_index(p, kvh, d, hd, S)];
      dot = dot + t;
    }
    const float sc = dot * scale;
    row[p] = sc;
    mx = fmaxf(mx, sc);
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  for (int p = tid; p < seq; p += 256) row[p] = syn_expf(row[p] - mx);
  __syncthreads();
  if (tid < 64) {
    const float s = wave_seq_sum(row, seq, 0.0f);
    if (tid == 0) s_sum = s;
  }
  __syncthreads();
  const float sum = s_sum;
  if (sum > 0.0f)
    for (int p = tid; p < seq; p += 256) row[p] = row[p] / sum;
  __syncthreads();
  for (int d = tid; d < hd; d += 256) {
    float val = 0.0f;
    for (int p = 0; p < seq; p++) {
      const float t = row[p] * vc[kv_v_index(p, kvh, d, hd, S)];
      val = val + t;
    }
    out[(size_t)qh * hd + d] = val;
  }
}

// x += delta (if delta.p); normed = (x * w) * (1 / sqrt(sum(x^2) / H + eps))
// (pure_rust_ops.rs:96-112's formula) with the sum of squares in tree order:
// one workgroup of 1024 threads, wave sums by shuffles, then the 16 wave
// sums in order.  The decoder is graded by tolerance (its Q4 GEMVs sum in
// their own order), and the sequential chain of the reference's order costs
// a 1024-deep dependent add chain per norm.
__global__ void __launch_bounds__(1024)
    k_hlm_norm(float *__restrict__ x, PartRows delta, const float *__restrict__ w, float eps,
               int H, float *__restrict__ normed) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  float ss = 0.0f;
  for (int j = tid; j < H; j += 1024) {
    float v = x[j];
    if (delta.p) {
      v = v + part_row(delta, j);
      x[j] = v;
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) tot += red[i];
  const float scale = 1.0f / sqrtf(tot / (float)H + eps);
  for (int j = tid; j < H; j += 1024) {
    const float t = x[j] * w[j];
    normed[j] = t * scale;
  }
}

// layer.rs:99: h = silu(gate) * up over the stacked [gate | up] row
__global__ void __launch_bounds__(256)
    k_hlm_swiglu(PartRows gu, int F, float *__restrict__ h) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < F) h[i] = syn_silu(part_row(gu, i)) * part_row(gu, F + i);
}

}  // namespace syn

using namespace syn;

static syn_status_t launch_hlm_norm(float *x, PartRows delta, const float *w, float eps, int H,
                                   float *normed, hipStream_t s) {
  hipLaunchKernelGGL(k_hlm_norm, dim3(1), dim3(1024), 0, s, x, delta, w, eps, H, normed);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

struct syn_hip_hlm_s {
  syn_hip_hlm_config c{};
  size_t H = 0, L = 0, V = 0, nh = 0, nkv = 0, hd = 0, I = 0, ck = 0, F = 0, S = 0;
  size_t qd = 0, kvd = 0, ldw = 0;
  struct Layer {
    int kind = 0;
    QLinearQ4_0 in, out, qkv, o, gu, down;
    DevBuf conv_w, conv_b, conv_state, q_nw, k_nw, attn_nw, ffn_nw, kc, vc;
  };
  std::vector<Layer> layers;
  DevBuf embed, lm_p, final_nw, rope_cos, rope_sin;
  DevBuf x, normed, proj, conv_out, qrot, attn, o, gu, hbuf, down, logits;
  DevBuf state, pv, pi, pv2, history, mhist;
  hipStream_t stream = nullptr;
  hipGraphExec_t graph = nullptr;
  bool ready = false, use_graph = true;
  // fused step (klm_fused.hip's GEMV over the Q4_0 planes): the fixed-point
  // residual r [H], the split-K accumulator of in_proj / q|k|v (cleared by
  // the projection after its reader), attention chunk partials, lm_head top-2
  bool use_fused = true, fused_ok = false;
  KqfPlan fp_in, fp_out, fp_qkv, fp_o, fp_gu, fp_down;
  DevBuf f_r, f_acc, f_ao, f_aml, f_pv, f_pi, f_pv2;
  size_t n_qkv = 0;

  ~syn_hip_hlm_s() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (stream) (void)hipStreamDestroy(stream);
  }
  StepState *st() { return state.as<StepState>(); }

  // HybridModel::decode_one for the token in st()->token at position
  // st()->pos; logits -> argmax -> st()->token, pos += 1
  // the fused step's plans and buffers, when every shape fits its kernels
  syn_status_t setup_fused() {
    fused_ok = false;
    const int fm[1] = {SYN_HIP_FMT_Q4_0};
    if (!kqf_fits((int)H, (int)qd, (int)F, (int)nh, (int)nkv, (int)hd, (int)S, fm, 1) ||
        I % 256 || !head_f32_fits((int)H))
      return SYN_OK;
    bool any_conv = false, any_gqa = false;
    for (auto &Ly : layers) {
      for (QLinearQ4_0 *q : {&Ly.in, &Ly.out, &Ly.qkv, &Ly.o, &Ly.gu, &Ly.down})
        if (q->n && !q->gemm_ok()) return SYN_OK;  // halved subnormal scales
      (Ly.kind == 0 ? any_conv : any_gqa) = true;
    }
    const Layer *conv = nullptr, *gqa = nullptr;
    for (auto &Ly : layers) (Ly.kind == 0 ? conv : gqa) = &Ly;
    if (conv) {
      fp_in = kqf_plan(conv->in, false);
      fp_out = kqf_plan(conv->out, false);
    }
    if (gqa) {
      fp_qkv = kqf_plan(gqa->qkv, false);
      fp_o = kqf_plan(gqa->o, false);
    }
    fp_gu = kqf_plan(layers[0].gu, true);
    fp_down = kqf_plan(layers[0].down, false);
    n_qkv = std::max(any_conv ? 3 * I : 0, any_gqa ? qd + 2 * kvd : 0);
    SYN_TRY(f_r.alloc(H * 8));
    SYN_TRY(f_acc.alloc(n_qkv * 8));
    SYN_HIP(hipMemset(f_acc.p, 0, f_acc.bytes));  // later steps leave it cleared
    if (any_gqa) {
      const size_t nch = (size_t)kqf_chunks((int)S);
      SYN_TRY(f_ao.alloc(nh * nch * hd * 4));
      SYN_TRY(f_aml.alloc(nh * nch * 2 * 4));
      SYN_HIP(hipMemset(f_ao.p, 0, f_ao.bytes));
      SYN_HIP(hipMemset(f_aml.p, 0, f_aml.bytes));
    }
    const size_t panels = cdiv(V, (size_t)64);
    SYN_TRY(f_pv.alloc(panels * 4));
    SYN_TRY(f_pi.alloc(panels * 4));
    SYN_TRY(f_pv2.alloc(panels * 4));
    SYN_HIP(hipDeviceSynchronize());  // the memsets ran on the null stream, not the model's
    fused_ok = true;
    return SYN_OK;
  }

  // fused step: per LIV conv layer in_proj of rmsnorm(r) (layer 0: of the
  // token's embedding row), out_proj of the conv step (in its prologue)
  // added into r, gate|up of rmsnorm(r) with SwiGLU, down added into r
  // (clearing the in_proj accumulator); per GQA layer q|k|v, the chunked attention with head norms, RoPE
  // and KV append, O of the chunk combine added into r, gate|up, down; then
  // the tied lm_head of rmsnorm(r) with per-panel top-2 and the merge.
  syn_status_t decode_step_fused(hipStream_t s) {
    const float eps = c.eps;
    long long *r = f_r.as<long long>(), *acc = f_acc.as<long long>();
    for (size_t l = 0; l < L; l++) {
      Layer &Ly = layers[l];
      KqfIn a;  // K1: in_proj or q|k|v rows of rmsnorm(r)
      a.r = r;
      a.embed = embed.as<float>();
      a.vocab = (int)V;
      a.r_out = r;
      a.st = st();
      a.gain = Ly.attn_nw.as<float>();
      a.eps = eps;
      a.H = (int)H;
      const int pro = l == 0 ? KQF_PRO_EMBED : KQF_PRO_NORM;
      long long *zero_after = nullptr;  // the accumulator the down projection clears
      int nzero = 0;
      if (Ly.kind == 0) {
        SYN_TRY(kqf_gemv(Ly.in, fp_in, pro, a, acc, nullptr, 0, s));
        KqfIn b;  // r += out_proj(conv step of the in_proj accumulator)
        b.cacc = acc;
        b.cstate = Ly.conv_state.as<float>();
        b.cw = Ly.conv_w.as<float>();
        b.cb = c.conv_bias ? Ly.conv_b.as<float>() : nullptr;
        b.inner = (int)I;
        b.ck = (int)ck;
        b.st = st();
        SYN_TRY(kqf_gemv(Ly.out, fp_out, KQF_PRO_CONV, b, r, nullptr, 0, s));
        zero_after = acc;  // every out_proj workgroup reads it in its prologue
        nzero = (int)(3 * I);
      } else {
        SYN_TRY(kqf_gemv(Ly.qkv, fp_qkv, pro, a, acc, nullptr, 0, s));
        SYN_TRY(kqf_attention(acc, (int)nh, (int)nkv, (int)hd, Ly.q_nw.as<float>(),
                              Ly.k_nw.as<float>(), eps, rope_cos.as<float>(),
                              rope_sin.as<float>(), st(), Ly.kc.as<float>(), Ly.vc.as<float>(),
                              (int)S, f_ao.as<float>(), f_aml.as<float>(), s));
        KqfIn b;  // r += O(combine of the chunks); the q|k|v accumulator cleared
        b.ao = f_ao.as<float>();
        b.aml = f_aml.as<float>();
        b.hd = (int)hd;
        b.nch = kqf_chunks((int)S);
        b.st = st();
        SYN_TRY(kqf_gemv(Ly.o, fp_o, KQF_PRO_ATTN, b, r, acc, (int)(qd + 2 * kvd), s));
      }
      KqfIn g;  // gate|up of rmsnorm(r), SwiGLU
      g.r = r;
      g.gain = Ly.ffn_nw.as<float>();
      g.eps = eps;
      g.H = (int)H;
      SYN_TRY(kqf_gate_up(Ly.gu, fp_gu, g, (int)F, hbuf.as<float>(), s));
      KqfIn d;  // r += down(h)
      d.x = hbuf.as<float>();
      SYN_TRY(kqf_gemv(Ly.down, fp_down, KQF_PRO_NONE, d, r, zero_after, nzero, s));
    }
    HeadIn hin;  // the tied f32 lm_head of rmsnorm(r)
    hin.fx = r;
    hin.gain = final_nw.as<float>();
    hin.eps = eps;
    SYN_TRY(launch_head_f32_top2(embed.as<float>(), (int)V, (int)H, hin, logits.as<float>(),
                                 f_pv.as<float>(), f_pi.as<int>(), f_pv2.as<float>(), s));
    return launch_argmax_advance(f_pv.as<float>(), f_pi.as<int>(), f_pv2.as<float>(),
                                 (int)cdiv(V, (size_t)64), st(), history.as<uint32_t>(),
                                 mhist.as<float>(), s);
  }

  syn_status_t decode_step(hipStream_t s) {
    if (use_fused && fused_ok) return decode_step_fused(s);
    const float eps = c.eps;
    // each Q4 GEMV leaves its split-K partials to the kernel that reads its
    // output (PartRows): no second launch per GEMV
    PartRows pin, pout, pgu, pdown;
    SYN_TRY(launch_embed(embed.as<float>(), &st()->token, 1, (int)H, (int)V, x.as<float>(), s));
    for (size_t l = 0; l < L; l++) {
      Layer &Ly = layers[l];
      SYN_TRY(launch_hlm_norm(x.as<float>(), l == 0 ? PartRows{} : pdown, Ly.attn_nw.as<float>(),
                              eps, (int)H, normed.as<float>(), s));
      if (Ly.kind == 0) {
        SYN_TRY(Ly.in.gemv_parts(normed.as<float>(), proj.as<float>(), &pin, s));
        hipLaunchKernelGGL(k_hlm_conv, dim3((unsigned)cdiv(I, 256)), dim3(256), 0, s, pin,
                           (int)I, (int)ck, st(), Ly.conv_state.as<float>(),
                           Ly.conv_w.as<float>(), c.conv_bias ? Ly.conv_b.as<float>() : nullptr,
                           conv_out.as<float>());
        SYN_LAUNCH_CHECK();
        SYN_TRY(Ly.out.gemv_parts(conv_out.as<float>(), o.as<float>(), &pout, s));
      } else {
        SYN_TRY(Ly.qkv.gemv_parts(normed.as<float>(), proj.as<float>(), &pin, s));
        hipLaunchKernelGGL(k_hlm_qk, dim3((unsigned)(nh + 2 * nkv)), dim3(64),
                           2 * round_up(hd, 4) * 4, s, pin, (int)nh, (int)nkv, (int)hd,
                           Ly.q_nw.as<float>(), Ly.k_nw.as<float>(), eps, rope_cos.as<float>(),
                           rope_sin.as<float>(), st(), (int)S, qrot.as<float>(),
                           Ly.kc.as<float>(), Ly.vc.as<float>());
        SYN_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_hlm_attn, dim3((unsigned)nh), dim3(256), ldw * 4, s,
                           qrot.as<float>(), Ly.kc.as<float>(), Ly.vc.as<float>(), st(), (int)nh,
                           (int)nkv, (int)hd, (int)S, 1.0f / sqrtf((float)hd), attn.as<float>());
        SYN_LAUNCH_CHECK();
        SYN_TRY(Ly.o.gemv_parts(attn.as<float>(), o.as<float>(), &pout, s));
      }
      SYN_TRY(launch_hlm_norm(x.as<float>(), pout, Ly.ffn_nw.as<float>(), eps, (int)H,
                              normed.as<float>(), s));
      SYN_TRY(Ly.gu.gemv_parts(normed.as<float>(), gu.as<float>(), &pgu, s));
      hipLaunchKernelGGL(k_hlm_swiglu, dim3((unsigned)cdiv(F, 256)), dim3(256), 0, s, pgu,
                         (int)F, hbuf.as<float>());
      SYN_LAUNCH_CHECK();
      SYN_TRY(Ly.down.gemv_parts(hbuf.as<float>(), down.as<float>(), &pdown, s));
    }
    SYN_TRY(launch_hlm_norm(x.as<float>(), pdown, final_nw.as<float>(), eps, (int)H,
                            normed.as<float>(), s));
    SYN_TRY(launch_gemv_f32_exact(lm_p.as<float>(), normed.as<float>(), normed.bytes / 4, (int)V,
                                  (int)H, n8_of((int)V), logits.as<float>(), s));
    SYN_TRY(launch_argmax(logits.as<float>(), (int)V, pv.as<float>(), pi.as<int>(),
                          pv2.as<float>(), st(), history.as<uint32_t>(), mhist.as<float>(), s));
    return launch_step_advance(st(), 1, s);
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
  // conv states to zero, position 0 (the KV rows past the position are never read)
  syn_status_t reset() {
    for (auto &Ly : layers)
      if (Ly.kind == 0)
        SYN_TRY(launch_zero_i32(Ly.conv_state.as<int>(), 2 * I * ck, stream));
    return set_state(0, 0, 0);
  }
};

static syn_status_t check_hlm(syn_hip_hlm_t *m) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (!m->ready) {
    set_error("hybrid LM: weights not initialised");
    return SYN_ERR_INVALID_ARG;
  }
  return SYN_OK;
}

extern "C" {

syn_status_t syn_hip_hlm_create(const syn_hip_hlm_config *cfg, syn_hip_hlm_t **out) {
  if (!cfg || !out) return SYN_ERR_NULL_PTR;
  *out = nullptr;
  const syn_hip_hlm_config &c = *cfg;
  if (c.n_layers == 0 || c.n_layers > 64 || c.hidden == 0 || c.vocab == 0 || c.max_seq == 0 ||
      c.hidden % 32 || c.inner % 32 || c.inter % 32 || c.n_kv_heads == 0 || c.n_heads == 0 ||
      c.n_heads % c.n_kv_heads || c.head_dim == 0 || c.head_dim % 2 || c.head_dim > 256 ||
      (c.n_heads * c.head_dim) % 32 || c.conv_kernel == 0 || c.conv_kernel > 64 ||
      c.max_seq > 32768) {
    set_error("hybrid LM: unsupported shape (K % 32 for every Q4 projection, head_dim even and "
              "<= 256, 1..64 layers, max_seq <= 32768 for the LDS score row)");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  for (uint32_t l = 0; l < c.n_layers; l++)
    if (c.layer_kinds[l] > 1) {
      set_error("hybrid LM: layer kind must be 0 (LIV conv) or 1 (GQA)");
      return SYN_ERR_INVALID_ARG;
    }
  SYN_TRY(ensure_init());
  auto *m = new (std::nothrow) syn_hip_hlm_t();
  if (!m) return SYN_ERR_OUT_OF_MEMORY;
  m->c = c;
  m->H = c.hidden, m->L = c.n_layers, m->V = c.vocab, m->nh = c.n_heads;
  m->nkv = c.n_kv_heads, m->hd = c.head_dim, m->I = c.inner, m->ck = c.conv_kernel;
  m->F = c.inter, m->S = c.max_seq;
  m->qd = m->nh * m->hd, m->kvd = m->nkv * m->hd, m->ldw = round_up(m->S, 4);
  if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
    delete m;
    set_error("hipStreamCreate failed");
    return SYN_ERR_HIP;
  }
  m->layers.resize(m->L);
  *out = m;
  return SYN_OK;
}

// Synthetic weights (harness spec, the same as the oracle's): embed (= tied
// lm_head) tensor 0 ~ N(0, std); layer l, seeds s = seed_base + 1 + 16 l:
// conv: in_proj s+0, conv taps s+1, out_proj s+2, conv bias s+3 (if
// enabled); GQA: q s+0, k s+1, v s+2, o s+3, q/k norm gains s+6, s+7; both:
// attn/ffn norm gains s+8, s+9, gate s+10, up s+11, down s+12 (projections
// ~ N(0, std), Q4-quantized by Q4Linear::from_f32; gains 1 + N(0, 0.1));
// final norm gain seed_base + 1 + 16 L.
syn_status_t syn_hip_hlm_init_synthetic(syn_hip_hlm_t *m, uint64_t seed_base, float stddev) {
  if (!m) return SYN_ERR_NULL_PTR;
  const size_t H = m->H, I = m->I, F = m->F, V = m->V, hd = m->hd, ck = m->ck;
  const size_t qd = m->qd, kvd = m->kvd, S = m->S, nkv_ = m->nkv;
  auto up = [](DevBuf &b, const std::vector<float> &v) -> syn_status_t {
    SYN_TRY(b.alloc(v.size() * 4));
    SYN_HIP(hipMemcpy(b.p, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return SYN_OK;
  };
  auto gain = [](size_t n, uint64_t seed) {
    std::vector<float> g(n);
    fill_normal(g.data(), n, seed, 0.1f);
    for (auto &v : g) v = 1.0f + v;
    return g;
  };
  // packed Q4 bytes of the stacked N(0, std) tensors (rows, seed) in order
  auto q4_stack = [&](QLinearQ4_0 &lin, std::vector<std::pair<size_t, uint64_t>> parts,
                      size_t k) -> syn_status_t {
    std::vector<std::vector<uint8_t>> packed(parts.size());
    std::vector<std::thread> th;
    for (size_t i = 0; i < parts.size(); i++)
      th.emplace_back([&, i] {
        std::vector<float> w(parts[i].first * k);
        fill_normal(w.data(), w.size(), parts[i].second, stddev);
        packed[i].resize(parts[i].first * (k / 32) * 18);
        host_q4_pack(w.data(), parts[i].first, k, packed[i].data());
      });
    for (auto &t : th) t.join();
    std::vector<uint8_t> all;
    size_t rows = 0;
    for (size_t i = 0; i < parts.size(); i++) {
      all.insert(all.end(), packed[i].begin(), packed[i].end());
      rows += parts[i].first;
    }
    SYN_TRY(lin.upload_packed(all.data(), rows, k));
    return lin.prepare(1);  // the step allocates nothing (graph capture)
  };
  {
    std::vector<float> emb(V * H);
    fill_normal_parallel(emb.data(), emb.size(), seed_base, stddev);
    SYN_TRY(up(m->embed, emb));
    SYN_TRY(up(m->lm_p, to_panels(emb.data(), V, H)));
  }
  for (size_t l = 0; l < m->L; l++) {
    auto &Ly = m->layers[l];
    const uint64_t s = seed_base + 1 + 16 * l;
    Ly.kind = m->c.layer_kinds[l];
    if (Ly.kind == 0) {
      SYN_TRY(q4_stack(Ly.in, {{3 * I, s + 0}}, H));
      std::vector<float> cw(I * ck);
      fill_normal(cw.data(), cw.size(), s + 1, stddev);
      SYN_TRY(up(Ly.conv_w, cw));
      SYN_TRY(q4_stack(Ly.out, {{H, s + 2}}, I));
      if (m->c.conv_bias) {
        std::vector<float> cb(I);
        fill_normal(cb.data(), I, s + 3, stddev);
        SYN_TRY(up(Ly.conv_b, cb));
      }
      SYN_TRY(up(Ly.conv_state, std::vector<float>(2 * I * ck, 0.0f)));  // two halves
    } else {
      SYN_TRY(q4_stack(Ly.qkv, {{qd, s + 0}, {kvd, s + 1}, {kvd, s + 2}}, H));
      SYN_TRY(q4_stack(Ly.o, {{H, s + 3}}, qd));
      SYN_TRY(up(Ly.q_nw, gain(hd, s + 6)));
      SYN_TRY(up(Ly.k_nw, gain(hd, s + 7)));
      // the attention kernels' tiled layouts (kv_k_index / kv_v_index)
      SYN_TRY(Ly.kc.alloc(kv_k_elems((int)nkv_, (int)hd, (int)S) * 4));
      SYN_TRY(Ly.vc.alloc(kv_v_elems((int)nkv_, (int)hd, (int)S) * 4));
      SYN_HIP(hipMemset(Ly.kc.p, 0, Ly.kc.bytes));
      SYN_HIP(hipMemset(Ly.vc.p, 0, Ly.vc.bytes));
    }
    SYN_TRY(up(Ly.attn_nw, gain(H, s + 8)));
    SYN_TRY(up(Ly.ffn_nw, gain(H, s + 9)));
    SYN_TRY(q4_stack(Ly.gu, {{F, s + 10}, {F, s + 11}}, H));
    SYN_TRY(q4_stack(Ly.down, {{H, s + 12}}, F));
  }
  SYN_TRY(up(m->final_nw, gain(H, seed_base + 1 + 16 * m->L)));
  // model.rs:708-720 RoPE tables (f32 powf / cosf / sinf on the host)
  {
    const size_t half = hd / 2;
    std::vector<float> cs(S * half), sn(S * half);
    const float theta = m->c.rope_theta;
    for (size_t p = 0; p < S; p++)
      for (size_t i = 0; i < half; i++) {
        const float freq = 1.0f / powf(theta, 2.0f * (float)i / (float)hd);
        const float ang = (float)p * freq;
        cs[p * half + i] = cosf(ang);
        sn[p * half + i] = sinf(ang);
      }
    SYN_TRY(up(m->rope_cos, cs));
    SYN_TRY(up(m->rope_sin, sn));
  }
  SYN_TRY(m->x.alloc(H * 4));
  SYN_TRY(m->normed.alloc(f32_exact_x_elems(H) * 4));  // padded for the f32 GEMV
  SYN_HIP(hipMemset(m->normed.p, 0, m->normed.bytes));
  SYN_TRY(m->proj.alloc(std::max(3 * I, qd + 2 * kvd) * 4));
  SYN_TRY(m->conv_out.alloc(I * 4));
  SYN_TRY(m->qrot.alloc(qd * 4));
  SYN_TRY(m->attn.alloc(qd * 4));
  SYN_TRY(m->o.alloc(H * 4));
  SYN_TRY(m->gu.alloc(2 * F * 4));
  SYN_TRY(m->hbuf.alloc(F * 4));
  SYN_TRY(m->down.alloc(H * 4));
  SYN_TRY(m->logits.alloc(V * 4));
  // the attention's score row: up to 128 KiB of dynamic LDS
  SYN_HIP(hipFuncSetAttribute((const void *)k_hlm_attn,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)(m->ldw * 4)));
  SYN_TRY(m->state.alloc(sizeof(StepState)));
  SYN_TRY(m->pv.alloc(256 * 4));
  SYN_TRY(m->pi.alloc(256 * 4));
  SYN_TRY(m->pv2.alloc(256 * 4));
  SYN_TRY(m->history.alloc((S + 1) * 4));
  SYN_TRY(m->mhist.alloc((S + 1) * 4));
  SYN_TRY(m->setup_fused());
  if (m->graph) {  // weights replaced: the captured step is stale
    (void)hipGraphExecDestroy(m->graph);
    m->graph = nullptr;
  }
  m->ready = true;
  return m->reset();
}

syn_status_t syn_hip_hlm_reset(syn_hip_hlm_t *m) {
  SYN_TRY(check_hlm(m));
  return m->reset();
}

syn_status_t syn_hip_hlm_position(syn_hip_hlm_t *m, size_t *pos) {
  SYN_TRY(check_hlm(m));
  if (!pos) return SYN_ERR_NULL_PTR;
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  *pos = (size_t)cur.pos;
  return SYN_OK;
}

syn_status_t syn_hip_hlm_decode_one(syn_hip_hlm_t *m, uint32_t token, float *host_logits) {
  SYN_TRY(check_hlm(m));
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos >= m->S) {
    set_error("hybrid LM: KV cache full");
    return SYN_ERR_INVALID_ARG;
  }
  SYN_TRY(m->set_state(cur.pos, token, cur.step));
  SYN_TRY(m->run_step());
  if (host_logits)
    SYN_HIP(hipMemcpyAsync(host_logits, m->logits.p, m->V * 4, hipMemcpyDeviceToHost, m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_hlm_prefill(syn_hip_hlm_t *m, const uint32_t *ids, size_t n,
                                 float *host_logits) {
  SYN_TRY(check_hlm(m));
  if (!ids) return SYN_ERR_NULL_PTR;
  for (size_t i = 0; i < n; i++)
    SYN_TRY(syn_hip_hlm_decode_one(m, ids[i], i + 1 == n ? host_logits : nullptr));
  return SYN_OK;
}

syn_status_t syn_hip_hlm_generate(syn_hip_hlm_t *m, const uint32_t *prompt, size_t n_prompt,
                                  size_t max_new, uint32_t *out_tokens, float *out_margins) {
  SYN_TRY(check_hlm(m));
  if (!prompt || !out_tokens) return SYN_ERR_NULL_PTR;
  if (max_new == 0 || n_prompt == 0) return SYN_OK;
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos + n_prompt + max_new - 1 > m->S) {
    set_error("hybrid LM: prompt + generated tokens exceed max_seq");
    return SYN_ERR_INVALID_ARG;
  }
  for (size_t i = 0; i + 1 < n_prompt; i++) SYN_TRY(syn_hip_hlm_decode_one(m, prompt[i], nullptr));
  // the last prompt token's argmax is the first generated token (step 0)
  SYN_TRY(m->set_state(cur.pos + (int)n_prompt - 1, prompt[n_prompt - 1], 0));
  for (size_t i = 0; i < max_new; i++) SYN_TRY(m->run_step());
  SYN_HIP(hipMemcpyAsync(out_tokens, m->history.p, max_new * 4, hipMemcpyDeviceToHost,
                         m->stream));
  if (out_margins)
    SYN_HIP(hipMemcpyAsync(out_margins, m->mhist.p, max_new * 4, hipMemcpyDeviceToHost,
                           m->stream));
  SYN_HIP(hipStreamSynchronize(m->stream));
  return SYN_OK;
}

syn_status_t syn_hip_hlm_decode_timed(syn_hip_hlm_t *m, size_t steps, float *elapsed_ms) {
  SYN_TRY(check_hlm(m));
  if (!elapsed_ms) return SYN_ERR_NULL_PTR;
  StepState cur;
  SYN_TRY(m->get_state(&cur));
  if ((size_t)cur.pos + steps > m->S) {
    set_error("hybrid LM: decode steps exceed max_seq");
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

syn_status_t syn_hip_hlm_set_options(syn_hip_hlm_t *m, int fused, int graph) {
  if (!m) return SYN_ERR_NULL_PTR;
  if (m->graph && m->use_fused != (fused != 0)) {  // the captured step changes form
    SYN_HIP(hipStreamSynchronize(m->stream));
    (void)hipGraphExecDestroy(m->graph);
    m->graph = nullptr;
  }
  m->use_fused = fused != 0;
  m->use_graph = graph != 0;
  return SYN_OK;
}

syn_status_t syn_hip_hlm_fused_active(syn_hip_hlm_t *m, int *active) {
  if (!m || !active) return SYN_ERR_NULL_PTR;
  *active = m->use_fused && m->fused_ok ? 1 : 0;
  return SYN_OK;
}

syn_status_t syn_hip_hlm_destroy(syn_hip_hlm_t *m) {
  if (!m) return SYN_OK;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  delete m;
  return SYN_OK;
}

}  // extern "C"
