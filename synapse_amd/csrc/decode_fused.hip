// Fused INT8 W8A8 decode step (one token, batch 1).
//
// The unfused step launches one kernel per reference op (13 per layer).  At
// batch 1 every one of them is latency-bound, so the step is rebuilt as five
// kernels per layer:
//
//   K1  x = x_mid + down(prev) ; q8(rmsnorm(x))       ; QKV rows (split K)
//   K2  per query head: q/k/v rows, head norms, RoPE, KV append, scores,
//       softmax, P.V (k_attn_head)
//   K3  q8(attn)                                       ; O rows (split K)
//   K4  x_mid = x + o ; q8(rmsnorm(x_mid)) ; gate and up rows over the whole
//       K, h = silu(gate) * up, max |h| (k_gu_swiglu)
//   K5  q8 of this split's K range of h with that max  ; down rows (split K)
//
// then the final norm, the lm_head GEMV with per-panel top-2, and one merge.
// A split-K GEMV adds its exact int32 partial dot products into per-layer
// accumulators with atomics (integer sums are exact in any order); the
// consumer applies the reference epilogue (f32(acc)*sx)*sw.  A prologue that
// needs a whole row (RMSNorm, a quantizer's max) is computed redundantly by
// every workgroup (it reads a few KB from L2), which removes all
// inter-workgroup synchronisation inside a kernel.  Each wave issues its
// weight loads before the prologue, so the HBM latency of the GEMV hides
// behind the prologue's dependency chains, and the prologue batches its own
// loads so that each thread has several in flight.  Dependent float chains
// run from registers (reduce_order.hpp pin_regs).
//
// Every float operation is the one of the unfused kernels (layer_ops.hip),
// which follow the reference's order: the fused step is bit-identical to it.
#include <algorithm>
#include <type_traits>

#include "fused_dev.hpp"
#include "linear.hpp"

namespace syn {

#ifdef SYN_PHASE_TIMING
static __device__ unsigned long long syn_phase_ts[256];
#define SYN_TS_FLUSH(base) SYN_TS_FLUSH_TO(syn_phase_ts, base)
// timeline of the step: workgroup (0, 0) of every kernel appends (kind,
// entry, exit) in s_memrealtime ticks (100 MHz)
static __device__ unsigned long long syn_tl[3 * 8192];
static __device__ unsigned syn_tl_n;
#define SYN_TL_ENTER() const unsigned long long syn_tl_e_ = __builtin_amdgcn_s_memrealtime()
#define SYN_TL_EXIT(kind)                                                          \
  do {                                                                             \
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {                  \
      const unsigned i_ = atomicAdd(&syn_tl_n, 1u);                                \
      if (i_ < 8192) {                                                             \
        syn_tl[3 * i_] = (kind);                                                   \
        syn_tl[3 * i_ + 1] = syn_tl_e_;                                            \
        syn_tl[3 * i_ + 2] = __builtin_amdgcn_s_memrealtime();                     \
      }                                                                            \
    }                                                                              \
  } while (0)
#else
#define SYN_TS_FLUSH(base) SYN_TS_FLUSH_TO(unused, base)
#define SYN_TL_ENTER() \
  do {                 \
  } while (0)
#define SYN_TL_EXIT(kind) \
  do {                    \
  } while (0)
#endif


// device address of the expf table (per device; resolved once)
const uint64_t *exp_table_address() {
  static const uint64_t *addr[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  if (!addr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(syn_exp2_tab)) != hipSuccess) return nullptr;
    addr[dev] = static_cast<const uint64_t *>(p);
  }
  return addr[dev];
}



// grid (panels, ks).  dynamic LDS: sq[round4(H)] floats (PRO_NORM) | xq[C*16].
// Everything a workgroup reads from memory is requested at entry: its weight
// chunks, then the prologue's inputs; the prologue then runs from registers.
// Loads are unconditional from clamped (in-bounds) addresses and the values
// of out-of-range lanes are ignored where they are used: a conditional load
// would make the compiler wait for it on the spot.
//
// GU (with PRO_NORM): the gate|up GEMV of the SwiGLU FFN.  A workgroup runs
// the same prologue, then the dot products of gate panel p and up panel
// pairs + p over its K slice.  Row j of the pair has one 64-bit accumulator
// holding its gate sum, its up sum and the number of slices added (gu_pack);
// each slice adds its two partial sums and one arrival with a single
// device-scope atomic and waits for the old value.  The slice whose add
// completes the count holds row j's exact totals: it applies the M <= 16
// epilogue (f32(acc)*sx)*sw to both, h[j] = silu(gate_j) * up_j
// (int8.rs:500-503), writes h and folds max |h| into hmax by an atomic max
// of the f32 bits (|h| >= 0, so the bit order is the value order; NaN is
// skipped as the reference quantizer's `if a > m` skips it).  Different
// rows of a pair may be completed by different slices.
template <int PRO, int NT, int U, bool GU, int R>
__global__ void __launch_bounds__(NT) k_fused_gemv(ProArgs a, GemvArgs g) {
  constexpr int NW = NT / 64;
  constexpr bool NORM = PRO == PRO_NORM || PRO == PRO_MNORM;
  static_assert(!GU || PRO == PRO_NORM, "gate|up pairs take the RMSNorm prologue");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float red[64];
  __shared__ int redi[(GU ? 2 : 1) * NW * 64];
  __shared__ uint64_t gu_tab[GU ? 32 : 1];  // GU: expf's table for the last slice's SiLU
  const int H = a.H;
  float *sq = reinterpret_cast<float *>(smem);
  int8_t *xq = reinterpret_cast<int8_t *>(smem) + (NORM ? ((H + 3) & ~3) * 4 : 0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int panel = blockIdx.x, ks = blockIdx.y;
  const int c0 = ks * g.cs, c1 = min(g.C, c0 + g.cs);  // c0 < c1 by the plan
  SYN_TS_DECL
  SYN_TS(0);
  SYN_TSR(14);
  SYN_TL_ENTER();

  // Vector loads retire in issue order, so the prologue's inputs (L2 hits)
  // are requested before the weight chunks (HBM): the prologue then waits
  // only for its own data while the weights stream in behind it.
  i32x4 w[U], w2[GU ? U : 1];
  const i32x4 *Wp = g.W + (size_t)panel * g.C * 64 + lane;
  const i32x4 *Wp2 = g.W + (size_t)(panel + g.pairs) * g.C * 64 + lane;
  // GU: the expf table word and the pair's row scales, for the last slice
  uint64_t gu_tv = 0;
  float gu_wsg = 0.0f, gu_wsu = 0.0f;
  if constexpr (GU) {
    gu_tv = g.exp_tab[tid & 31];
    gu_wsg = g.ws[panel * 64 + lane];
    gu_wsu = g.ws[(g.pairs + panel) * 64 + lane];
  }
  auto issue_weights = [&]() {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = min(c0 + wave + u * NW, c1 - 1);
      w[u] = __builtin_nontemporal_load(Wp + (size_t)c * 64);
      if constexpr (GU) w2[u] = __builtin_nontemporal_load(Wp2 + (size_t)c * 64);
    }
    asm volatile("" ::: "memory");  // keep the weight requests here, ahead of the prologue
    SYN_TS(1);
  };

  // 1. prologue inputs (element j = tid + u*NT, clamped to H-1), 2. the
  //    weight chunks, 3. the activation row x[] in registers
  float x[R];
  float nwv[R];
  float hq = 1.0f;
  if constexpr (NORM) {
    norm_prologue_load<NT, R>(a, H, x, nwv, issue_weights);
  } else if constexpr (PRO == PRO_HQ) {
    // element j = c0*16 + tid + u*NT of this split's K range
    const int k0 = c0 * 16, k1 = min(c1 * 16, H);
#pragma unroll
    for (int u = 0; u < R; u++) x[u] = a.vec[min(k0 + tid + u * NT, H - 1)];
    const float mx = __uint_as_float(a.hmax[0]);
    issue_weights();
    hq = quantize_range_with_max<NT, R>(x, k0, k1, mx, xq);
  } else if constexpr (PRO == PRO_QUANT) {
#pragma unroll
    for (int u = 0; u < R; u++) x[u] = a.vec[min(tid + u * NT, H - 1)];
    issue_weights();
  } else if constexpr (PRO == PRO_CONV) {
    // expf's table to LDS first (a global lookup would wait behind the weights)
    __shared__ uint64_t exp_tab[32];
    const uint64_t tv = a.exp_tab[tid & 31];
    int ra[R];
    float rw[R];
    float4 tp[R], cw[R];
    float cb[R];
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int j = min(tid + u * NT, H - 1);
      ra[u] = a.rows.acc[j];
      rw[u] = a.rows.ws[j];
      tp[u] = reinterpret_cast<const float4 *>(a.ring)[j];
      cw[u] = reinterpret_cast<const float4 *>(a.conv_w)[j];
      cb[u] = a.conv_b[j];
    }
    const float rsx = a.rows.sx[0];
    const int pos = a.st->pos;
    issue_weights();
    if (tid < 32) exp_tab[tid] = tv;
    bar<NT>();
    // taps oldest to newest: slots (pos+1)%4, (pos+2)%4, (pos+3)%4, then the input
    auto slot = [](const float4 &t, int k) {
      return k == 0 ? t.x : k == 1 ? t.y : k == 2 ? t.z : t.w;
    };
    const int k0 = (pos + 1) & 3, k1 = (pos + 2) & 3, k2 = (pos + 3) & 3;
#pragma unroll
    for (int u = 0; u < R; u++) {
      const float f = (float)ra[u] * rsx;
      const float xt = f * rw[u];
      float sum = 0.0f, t;
      t = slot(tp[u], k0) * cw[u].x;
      sum = sum + t;
      t = slot(tp[u], k1) * cw[u].y;
      sum = sum + t;
      t = slot(tp[u], k2) * cw[u].z;
      sum = sum + t;
      t = xt * cw[u].w;
      sum = sum + t;
      x[u] = syn_silu_tab(sum + cb[u], exp_tab);
      nwv[u] = xt;  // the new ring entry, published by workgroup 0
    }
  } else if constexpr (PRO == PRO_ROWS) {
    int ra[R];
    float rw[R];
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int j = min(tid + u * NT, H - 1);
      ra[u] = a.rows.acc[j];
      rw[u] = a.rows.ws[j];
    }
    const float rsx = a.rows.sx[0];
    issue_weights();
#pragma unroll
    for (int u = 0; u < R; u++) {
      const float f = (float)ra[u] * rsx;
      x[u] = f * rw[u];
    }
  } else {
    // expf's 2^(i/32) table goes to LDS first: a lookup in global memory
    // would wait behind the outstanding weight loads
    __shared__ uint64_t exp_tab[32];
    const uint64_t tv = a.exp_tab[tid & 31];
    int ga[R], ua[R];
    float gw[R], uw[R];
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int j = min(tid + u * NT, H - 1);
      ga[u] = a.gu.acc[j];
      ua[u] = a.gu.acc[H + j];
      gw[u] = a.gu.ws[j];
      uw[u] = a.gu.ws[H + j];
    }
    const float gsx = a.gu.sx[0];
    issue_weights();
    if (tid < 32) exp_tab[tid] = tv;
    bar<NT>();
#pragma unroll
    for (int u = 0; u < R; u++) {
      // silu(gate) * up (int8.rs:500-503), each factor the GEMV epilogue
      const float fg = (float)ga[u] * gsx, fu = (float)ua[u] * gsx;
      const float gv = fg * gw[u], uv = fu * uw[u];
      const float act = syn_silu_tab(gv, exp_tab);
      x[u] = act * uv;
    }
  }
  for (int j = H + tid; j < g.C * 16; j += NT) xq[j] = 0;
  SYN_TS(2);

  float sv;
  if constexpr (NORM) {
    sv = norm_quant<NT, R, PRO == PRO_MNORM>(a.eps, H, x, nwv, sq, xq, red SYN_TS_PASS);
  } else if constexpr (PRO == PRO_HQ) {
    sv = hq;
  } else {
    sv = quantize_regs<NT, R>(x, H, xq, red, 0);
  }
  SYN_TS(5);
  bar<NT>();
  SYN_TS(6);

  // 3. integer dot products of this wave's chunks, reduced over the waves
  int acc = 0, acc2 = 0;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int c = c0 + wave + u * NW;
    if (c < c1) {
      const i32x4 xv = *reinterpret_cast<const i32x4 *>(xq + c * 16);
      acc = __builtin_amdgcn_sdot4(w[u].x, xv.x, acc, false);
      acc = __builtin_amdgcn_sdot4(w[u].y, xv.y, acc, false);
      acc = __builtin_amdgcn_sdot4(w[u].z, xv.z, acc, false);
      acc = __builtin_amdgcn_sdot4(w[u].w, xv.w, acc, false);
      if constexpr (GU) {
        acc2 = __builtin_amdgcn_sdot4(w2[u].x, xv.x, acc2, false);
        acc2 = __builtin_amdgcn_sdot4(w2[u].y, xv.y, acc2, false);
        acc2 = __builtin_amdgcn_sdot4(w2[u].z, xv.z, acc2, false);
        acc2 = __builtin_amdgcn_sdot4(w2[u].w, xv.w, acc2, false);
      }
    }
  }
  SYN_TS(7);
  redi[wave * 64 + lane] = acc;
  if constexpr (GU) {
    redi[(NW + wave) * 64 + lane] = acc2;
    if (tid < 32) gu_tab[tid] = gu_tv;
  }
  bar<NT>();
  SYN_TS(8);
  if constexpr (GU) {
    if (wave == 0) {
      int sg = 0, su = 0;
#pragma unroll
      for (int i = 0; i < NW; i++) {
        sg += redi[i * 64 + lane];
        su += redi[(NW + i) * 64 + lane];
      }
      // row j's gate sum, up sum and one arrival in a single 64-bit add
      // (gu_pack); the returned value plus this add is the row's running
      // total, so the slice that completes the row knows it and has both
      // exact sums without another round trip
      const unsigned long long add = gu_pack(sg, su);
      const unsigned long long tot =
          __hip_atomic_fetch_add(g.acc64 + panel * 64 + lane, add, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) + add;
      int tg, tu, arrived;
      gu_unpack(tot, tg, tu, arrived);
      const bool last = arrived == (int)gridDim.y;
      const int j = panel * 64 + lane;
      float m = 0.0f;
      if (last && j < g.pairs * 64) {  // this row's SwiGLU and |h|
        const float fg = (float)tg * sv, fu = (float)tu * sv;
        const float gv = fg * gu_wsg, uv = fu * gu_wsu;
        const float act = syn_silu_tab(gv, gu_tab);
        const float hv = act * uv;
        g.h[j] = hv;
        const float av = fabsf(hv);
        if (av > m) m = av;
      }
      const bool any = __ballot(last) != 0;
      m = wave_max_nonneg(m);
      if (any && lane == 0) atomicMax(g.hmax, __float_as_uint(m));
    }
  } else if (wave == 0) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) s += redi[i * 64 + lane];
    atomicAdd(g.acc + panel * 64 + lane, s);
  }
  SYN_TS(9);

  // 4. workgroup 0 publishes the prologue's results for later kernels
  if (panel == 0 && ks == 0) {
    if constexpr (NORM) {
      if (a.res_out) {
#pragma unroll
        for (int u = 0; u < R; u++)
          if (tid + u * NT < H) a.res_out[tid + u * NT] = x[u];
      }
    }
    if constexpr (PRO == PRO_CONV) {
      const int ps = a.st->pos & 3;
#pragma unroll
      for (int u = 0; u < R; u++) {
        const int j = tid + u * NT;
        if (j < H) {
          a.conv_out[j] = x[u];
          a.ring[(size_t)j * 4 + ps] = nwv[u];
        }
      }
    }
    if (tid == 0) a.s_out[0] = sv;
  }
  SYN_TSR(15);
  SYN_TS_FLUSH(PRO * 16);
  SYN_TL_EXIT(PRO + (GU ? 10 : 0));
}

// threads per workgroup for a prologue row of H elements (RB rows each)
static int fused_nt_for(int H) { return H <= RB * 256 ? 256 : H <= RB * 512 ? 512 : 1024; }

// Each wave takes exactly U chunks of every K split (cs = U * waves), with U
// in {1, 2, 4, 8} chosen so the grid is closest to [target, 2*target]
// workgroups; only the last split can be partial.
SplitGemv plan_split_gemv(const void *W, const float *ws, int N, int C, int target_wg, int nt) {
  SplitGemv g;
  g.W = W;
  g.ws = ws;
  g.N = N;
  g.N64 = (int)round_up((size_t)N, 64);  // accumulator rows
  g.C = C;
  g.nt = std::max(nt, fused_nt_for(C * 16));
  const int panels = g.N64 / 64, nw = g.nt / 64;
  int best_u = 8;
  double best = 1e30;
  for (int u = 1; u <= 8; u *= 2) {
    const int cs = u * nw;
    const int ks = (int)cdiv((size_t)C, (size_t)cs);
    const double wg = (double)panels * ks;
    // distance from [target, 2*target] plus the waste of a partial last split
    double cost = wg < target_wg ? (target_wg - wg) / target_wg
                : wg > 2.0 * target_wg ? (wg - 2.0 * target_wg) / target_wg : 0.0;
    cost += (double)(ks * cs - C) / C;
    if (cost < best - 1e-9) {
      best = cost;
      best_u = u;
    }
  }
  g.u = best_u;
  g.cs = best_u * nw;
  g.ks = (int)cdiv((size_t)C, (size_t)g.cs);
  return g;
}

static size_t fused_lds_bytes(int H, int C) { return round_up((size_t)H, 4) * 4 + (size_t)C * 16; }

bool fused_gemv_fits(int H) {
  return H <= RB * 1024 && fused_lds_bytes(H, (int)cdiv((size_t)H, 16)) <= 60 * 1024;
}

template <int PRO, int NT, bool GU = false>
static syn_status_t launch_fused_nt(const ProArgs &a, const SplitGemv &g, hipStream_t s,
                                    const GemvArgs *gu = nullptr) {
  GemvArgs ga = gu ? *gu : GemvArgs{};
  ga.W = reinterpret_cast<const i32x4 *>(g.W);
  ga.C = g.C;
  ga.cs = g.cs;
  ga.acc = g.acc;
  const dim3 grid(g.N64 / 64, g.ks);
  const size_t shm = fused_lds_bytes(a.H, g.C);
  // R = prologue elements per thread: the fewest of {2, 4, 8} that cover H
  auto go = [&](auto rc) {
    constexpr int R = decltype(rc)::value;
    switch (g.u) {
      case 1: SYN_LAUNCH((k_fused_gemv<PRO, NT, 1, GU, R>), grid, dim3(NT), shm, s, a, ga); break;
      case 2: SYN_LAUNCH((k_fused_gemv<PRO, NT, 2, GU, R>), grid, dim3(NT), shm, s, a, ga); break;
      case 4: SYN_LAUNCH((k_fused_gemv<PRO, NT, 4, GU, R>), grid, dim3(NT), shm, s, a, ga); break;
      default: SYN_LAUNCH((k_fused_gemv<PRO, NT, 8, GU, R>), grid, dim3(NT), shm, s, a, ga); break;
    }
  };
  if (a.H <= 2 * NT) go(std::integral_constant<int, 2>{});
  else if (a.H <= 4 * NT) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, RB>{});
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

template <int PRO>
static syn_status_t launch_fused(const ProArgs &a, const SplitGemv &g, hipStream_t s) {
  if (!g.acc || !g.W) {
    set_error("fused decode GEMV: plan not prepared");
    return SYN_ERR_INTERNAL;
  }
  if (a.H > g.C * 16 || !fused_gemv_fits(a.H) || a.H > RB * g.nt) {
    set_error("fused decode GEMV: activation row does not fit the fused kernel");
    return SYN_ERR_INVALID_ARG;
  }
  if (PRO == PRO_ROWS && (!a.rows.acc || !a.rows.ws || !a.rows.sx)) {
    set_error("fused decode GEMV: row source must be GEMV accumulators");
    return SYN_ERR_INVALID_ARG;
  }
  if (g.nt == 1024) return launch_fused_nt<PRO, 1024>(a, g, s);
  if (g.nt == 512) return launch_fused_nt<PRO, 512>(a, g, s);
  return launch_fused_nt<PRO, 256>(a, g, s);
}

syn_status_t launch_fused_norm_gemv(const float *base, const float *embed, const StepState *st,
                                    int vocab, const float *zero_row, RowSrc delta,
                                    float *res_out, const float *nw, float eps, int H,
                                    float *s_out, const SplitGemv &g, hipStream_t s,
                                    bool sequential_sumsq) {
  ProArgs a{};
  a.base = base;
  a.embed = embed;
  a.st = st;
  a.vocab = vocab;
  a.delta = delta;
  a.res_out = res_out;
  a.nw = nw;
  a.zero_row = zero_row;
  a.eps = eps;
  a.H = H;
  a.s_out = s_out;
  return sequential_sumsq ? launch_fused<PRO_MNORM>(a, g, s) : launch_fused<PRO_NORM>(a, g, s);
}

syn_status_t launch_fused_rows_gemv(RowSrc rows, int H, float *s_out, const SplitGemv &g,
                                    hipStream_t s) {
  ProArgs a{};
  a.rows = rows;
  a.H = H;
  a.s_out = s_out;
  return launch_fused<PRO_ROWS>(a, g, s);
}

syn_status_t launch_fused_conv_gemv(RowSrc rows, const StepState *st, float *ring,
                                    const float *conv_w, const float *conv_b, float *conv_out,
                                    int H, float *s_out, const SplitGemv &g, hipStream_t s) {
  ProArgs a{};
  a.exp_tab = exp_table_address();
  if (!a.exp_tab) {
    set_error("fused decode: expf table address unavailable");
    return SYN_ERR_HIP;
  }
  a.rows = rows;
  a.st = st;
  a.ring = ring;
  a.conv_w = conv_w;
  a.conv_b = conv_b;
  a.conv_out = conv_out;
  a.H = H;
  a.s_out = s_out;
  if (!rows.acc || !rows.ws || !rows.sx) {
    set_error("fused conv GEMV: rows must be GEMV accumulators");
    return SYN_ERR_INTERNAL;
  }
  return launch_fused<PRO_CONV>(a, g, s);
}

syn_status_t launch_fused_quant_gemv(const float *vec, int H, float *s_out, const SplitGemv &g,
                                     hipStream_t s) {
  ProArgs a{};
  a.vec = vec;
  a.H = H;
  a.s_out = s_out;
  return launch_fused<PRO_QUANT>(a, g, s);
}

syn_status_t launch_fused_swiglu_gemv(RowSrc gu, int inter, float *s_out, const SplitGemv &g,
                                      hipStream_t s) {
  ProArgs a{};
  a.exp_tab = exp_table_address();
  if (!a.exp_tab) {
    set_error("fused decode: expf table address unavailable");
    return SYN_ERR_HIP;
  }
  a.gu = gu;
  a.H = inter;
  a.s_out = s_out;
  return launch_fused<PRO_SWIGLU>(a, g, s);
}

// ------------------------------------------------------------------ gate|up + SwiGLU
// x_mid = x + delta (res_out, workgroup 0), RMSNorm, quantize (the PRO_NORM
// prologue), then the gate|up GEMV split over K in pairs of panels (gate
// rows 64p.., up rows inter + 64p..), the slice that completes a row
// writing h = silu(gate) * up and max |h| (k_fused_gemv with GU).  The down GEMV
// then quantizes its K range of h with that max (PRO_HQ).
bool gu_swiglu_fits(int H, int inter) {
  return fused_gemv_fits(H) && H <= RB * 256 && inter > 0 && inter % 64 == 0;
}

SplitGemv plan_gu_pairs(const void *W, const float *ws, int inter, int C, int target_wg, int nt) {
  return plan_split_gemv(W, ws, inter, C, target_wg, nt);
}

syn_status_t launch_gu_swiglu(const float *base, RowSrc delta, float *res_out, const float *nw,
                              float eps, int H, float *s_out, const SplitGemv &g, const float *ws,
                              int inter, float *h, unsigned *hmax, hipStream_t s) {
  if (!gu_swiglu_fits(H, inter) || g.C != (int)cdiv((size_t)H, 16) || g.N64 != inter ||
      (g.nt != 256 && g.nt != 512) || g.ks > 255 || !g.acc ||
      reinterpret_cast<uintptr_t>(g.acc) % 8 || !h || !hmax || !ws) {
    set_error("gate|up SwiGLU GEMV: shapes outside the kernel's limits or plan not prepared");
    return SYN_ERR_INVALID_ARG;
  }
  ProArgs a{};
  a.base = base;
  a.delta = delta;
  a.res_out = res_out;
  a.nw = nw;
  a.eps = eps;
  a.H = H;
  a.s_out = s_out;
  GemvArgs gu{};
  gu.pairs = inter / 64;
  gu.acc64 = reinterpret_cast<unsigned long long *>(g.acc);
  gu.ws = ws;
  gu.h = h;
  gu.hmax = hmax;
  gu.exp_tab = exp_table_address();
  if (!gu.exp_tab) {
    set_error("fused decode: expf table address unavailable");
    return SYN_ERR_HIP;
  }
  if (g.nt == 512) return launch_fused_nt<PRO_NORM, 512, true>(a, g, s, &gu);
  return launch_fused_nt<PRO_NORM, 256, true>(a, g, s, &gu);
}

syn_status_t launch_fused_hq_gemv(const float *vec, const unsigned *hmax, int H, float *s_out,
                                  const SplitGemv &g, hipStream_t s) {
  if (!vec || !hmax) {
    set_error("fused decode GEMV: quantized-range prologue needs the vector and its max");
    return SYN_ERR_INVALID_ARG;
  }
  ProArgs a{};
  a.vec = vec;
  a.hmax = hmax;
  a.H = H;
  a.s_out = s_out;
  return launch_fused<PRO_HQ>(a, g, s);
}

// ------------------------------------------------------------------ attention
// One workgroup per query head.  Prologue = k_qk_norm_rope_kv for the head
// and its KV head (both query heads of a KV group write the same K/V values
// into the cache), and the new position's K/V rows are then taken from LDS.
// Attention = k_attn_decode (ops/attention.rs:24-147): the len >= 64 route
// uses fused multiply-add chains in f32GemvRow's 32/8-wide column blocks.

// shared prologue: q/k/v rows of this head from the QKV accumulators, head
// RMSNorms (norm.rs:78-93), rotate-half RoPE at pos (rope.rs:13-43) and the
// cache append.  qv/kv/vv/sq are LDS rows of hd floats.
template <int NT>
__device__ void attn_prologue(const RowSrc &qkv, int head, int kvh, int qd, int kvd, int hd,
                              const float *qn, const float *kn, float eps, const float *cosT,
                              const float *sinT, int pos, float *kc, float *vc, int max_seq,
                              float *qv, float *kv, float *vv, float *sq, float *red) {
  const int half = hd / 2;
  for (int d = threadIdx.x; d < hd; d += NT) {
    qv[d] = row_value(qkv, head * hd + d);
    kv[d] = row_value(qkv, qd + kvh * hd + d);
    vv[d] = row_value(qkv, qd + kvd + kvh * hd + d);
  }
  __syncthreads();
  if (qn) {
    const float ss = sumsq_lds<NT>(qv, hd, sq, red);
    const float scale = 1.0f / sqrtf(ss / (float)hd + eps);
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += NT) {
      const float t = qv[d] * qn[d];
      qv[d] = t * scale;
    }
    __syncthreads();
  }
  if (kn) {
    const float ss = sumsq_lds<NT>(kv, hd, sq, red);
    const float scale = 1.0f / sqrtf(ss / (float)hd + eps);
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += NT) {
      const float t = kv[d] * kn[d];
      kv[d] = t * scale;
    }
    __syncthreads();
  }
  const float *cr = cosT + (size_t)pos * half, *sr = sinT + (size_t)pos * half;
  for (int i = threadIdx.x; i < half; i += NT) {
    const float c = cr[i], sn = sr[i];
    {
      const float x1 = qv[i], x2 = qv[half + i];
      const float p = x1 * c, q = x2 * sn, r = x2 * c, t = x1 * sn;
      qv[i] = p - q;
      qv[half + i] = r + t;
    }
    {
      const float x1 = kv[i], x2 = kv[half + i];
      const float p = x1 * c, q = x2 * sn, r = x2 * c, t = x1 * sn;
      kv[i] = p - q;
      kv[half + i] = r + t;
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += NT) {
    kc[kv_k_index(pos, kvh, d, hd, max_seq)] = kv[d];
    vc[kv_v_index(pos, kvh, d, hd, max_seq)] = vv[d];
  }
}

// softmax_slice (activation.rs:117-129) over e[0..len): max, exp(x - max),
// sequential sum, divide when the sum is positive
template <int NT>
__device__ void attn_softmax(float *e, int len, float mx, float *red) {
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));  // scores may be negative
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; i++) mx = fmaxf(mx, red[i]);
  for (int sidx = threadIdx.x; sidx < len; sidx += NT) e[sidx] = syn_expf(e[sidx] - mx);
  __syncthreads();
  if (threadIdx.x == 0) red[40] = seq_sum(e, len);
  __syncthreads();
  const float sum = red[40];
  if (sum > 0.0f)
    for (int sidx = threadIdx.x; sidx < len; sidx += NT) e[sidx] = e[sidx] / sum;
  __syncthreads();
}

// Generic form (any head_dim): scores and P.V read the cache directly.
// dynamic LDS: qv[hd] | kv[hd] | vv[hd] | sq[hd] | e[max_seq rounded to 4]
__global__ void __launch_bounds__(256)
    k_fused_attention(RowSrc qkv, int nh, int nkv, int hd, const float *__restrict__ qn,
                      const float *__restrict__ kn, float eps, const float *__restrict__ cosT,
                      const float *__restrict__ sinT, const StepState *__restrict__ st,
                      float *__restrict__ kc, float *__restrict__ vc, int max_seq,
                      float *__restrict__ out) {
  constexpr int NT = 256;
  extern __shared__ __align__(16) float sm[];
  __shared__ float red[64];
  const int head = blockIdx.x;
  const int kvh = head / (nh / nkv);
  const int qd = nh * hd, kvd = nkv * hd;
  float *qv = sm, *kv = qv + hd, *vv = kv + hd, *sq = vv + hd, *e = sq + hd;
  const int pos = st->pos;
  const int len = pos + 1;
  attn_prologue<NT>(qkv, head, kvh, qd, kvd, hd, qn, kn, eps, cosT, sinT, pos, kc, vc, max_seq,
                    qv, kv, vv, sq, red);
  const float scale = 1.0f / sqrtf((float)hd);
  const bool simd = len >= 64;
  const int n32 = len - len % 32;
  const int n8 = n32 + ((len - n32) / 8) * 8;
  float mx = -__builtin_inff();
  for (int sidx = threadIdx.x; sidx < len; sidx += NT) {
    const bool fused = simd && sidx < n8;
    float acc = 0.0f;
    for (int d = 0; d < hd; d++) {
      const float kval = sidx == pos ? kv[d] : kc[kv_k_index(sidx, kvh, d, hd, max_seq)];
      if (fused) {
        acc = __builtin_fmaf(qv[d], kval, acc);
      } else {
        const float t = qv[d] * kval;
        acc = acc + t;
      }
    }
    const float sc = acc * scale;
    e[sidx] = sc;
    mx = fmaxf(mx, sc);
  }
  attn_softmax<NT>(e, len, mx, red);
  const int d32 = hd - hd % 32;
  for (int d = threadIdx.x; d < hd; d += NT) {
    const bool fused = simd && d < d32;
    float acc = 0.0f;
    for (int i = 0; i < len; i++) {
      const float vval = i == pos ? vv[d] : vc[kv_v_index(i, kvh, d, hd, max_seq)];
      if (fused) {
        acc = __builtin_fmaf(e[i], vval, acc);
      } else {
        const float t = e[i] * vval;
        acc = acc + t;
      }
    }
    out[head * hd + d] = acc;
  }
}


// ------------------------------------------------------------------ head attention
// Decode attention in one kernel: one workgroup per (query head, HD / CB
// column block), grouped by KV head (see the index decode below),
// 256 threads.  Every workgroup of a head computes the head's prologue (q/k/v
// rows, head RMSNorms, RoPE), all of its scores and the softmax, then the P.V
// chains of its CB columns; the workgroup of column block 0 of the first
// query head of a KV group appends the new K/V rows.  Compared with a scores
// kernel followed by a softmax + P.V kernel this removes one kernel boundary
// per layer, and every dependent chain runs from registers: q and the
// probabilities are read from LDS in blocks of 32 values that are issued
// before the previous block's arithmetic (pin_regs), the K row of a lane's
// position is loaded at kernel entry, and V reaches LDS through gfx950's
// direct global -> LDS loads, one 128-position chunk ahead of the chain.
// Every float operation and its order is the one of ops/attention.rs:24-147
// (scores: fused multiply-adds for positions below n8 when len >= 64, a
// rounded product and add otherwise; softmax_slice; P.V: fused multiply-adds
// over the positions when len >= 64 and the column lies in a whole 32-column
// block).

// dynamic LDS: e[round_up4(max_seq)] | V chunks [2][kPvGroups][CB] f32x4
template <bool F32, int HD>
__global__ void __launch_bounds__(kAttnNT)
    k_attn_head(RowSrc qkv, int nh, int nkv, const float *__restrict__ qn,
                const float *__restrict__ kn, float eps, const float *__restrict__ cosT,
                const float *__restrict__ sinT, const StepState *__restrict__ st,
                float *__restrict__ kc, float *__restrict__ vc, int max_seq,
                const uint64_t *__restrict__ exp_tab_g, float *__restrict__ out) {
  constexpr int CB = attn_cb<HD>(), HD4 = HD / 4, HALF = HD / 2;
  extern __shared__ __align__(16) float dsm[];
  __shared__ __align__(16) float qv[HD], kv[HD], sqq[HD], sqk[HD], vnew[HD];
  __shared__ float red[16];
  __shared__ uint64_t exp_tab[32];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup w: KV group w % nkv, then (query head of the group, column
  // block) from w / nkv.  Workgroups go to the XCDs round-robin by id, so
  // with nkv a multiple of 8 all workgroups of a KV group share an XCD and
  // its K and V rows come through that XCD's L2 once.
  const int grp = nh / nkv, wj = blockIdx.x / nkv;
  const int kvh = blockIdx.x % nkv, head = kvh * grp + wj / (HD / CB), cb0 = (wj % (HD / CB)) * CB;
  const int qd = nh * HD, kvd = nkv * HD;
  const int tiles = (max_seq + 63) >> 6, s4 = (max_seq + 3) >> 2;
  float *e = dsm;
  f32x4 *vbuf = reinterpret_cast<f32x4 *>(dsm + round_up4(max_seq));
  const f32x4 *V4 = reinterpret_cast<const f32x4 *>(vc) + (size_t)kvh * s4 * HD;
  const f32x4 *K4 = reinterpret_cast<const f32x4 *>(kc) + (size_t)kvh * tiles * HD4 * 64;
  SYN_TS_DECL
  SYN_TS(0);
  SYN_TSR(14);
  SYN_TL_ENTER();

  // 0. the decode position, requested first (waves 1-3 need it before they
  //    can issue their K rows); written by an earlier kernel of the stream,
  //    so a plain (scalar) load sees it
  const int pos = st->pos;
  // 1. what does not depend on the decode position, in the order it is
  //    needed last-first: wave 0's K rows (position tid) and the V of the
  //    first 64 positions of this block's columns (straight into LDS; every
  //    decode attends to position 0), then the q / k / v accumulator rows,
  //    their scales and gains and the expf table word.  Threads 0-127 own
  //    q[d], threads 128-255 own k[d] and v[d]; the rows' epilogue runs
  //    after the later loads are issued, so nothing waits here.  (Issuing
  //    the rows first, ahead of the K rows, measured slower.)
  f32x4 kr[HD4];
  auto load_k_rows = [&](int p) {
    const int pc = min(p, max_seq - 1);
    const f32x4 *src = K4 + (size_t)(pc >> 6) * HD4 * 64 + (pc & 63);
#pragma unroll
    for (int c = 0; c < HD4; c++) kr[c] = src[(size_t)c * 64];
  };
  if (wave == 0) {
    load_k_rows(tid);
    stage_v_chunk<CB>(V4, HD, s4, cb0, 0, vbuf, 0, 0, 1, lane, 16);
  }
  const bool is_q = tid < 128;
  const int d = tid & 127;
  const int dc = min(d, HD - 1), hc = min(d, HALF - 1);
  const int r0 = is_q ? head * HD + dc : qd + kvh * HD + dc;
  const int r1 = qd + kvd + kvh * HD + dc;
  float x0, x1;
  int a0 = 0, a1 = 0;
  float w0 = 0.0f, w1 = 0.0f, sx = 0.0f;
  if constexpr (F32) {
    x0 = qkv.f[r0];
    x1 = qkv.f[r1];
  } else {
    a0 = qkv.acc[r0];
    a1 = qkv.acc[r1];
    w0 = qkv.ws[r0];
    w1 = qkv.ws[r1];
    sx = qkv.sx[0];
  }
  const float *gn = is_q ? qn : kn;
  const float g = gn ? gn[dc] : 0.0f;
  const uint64_t tv = exp_tab_g[tid & 31];
  const int len = pos + 1;
  // score chain kinds (ops/attention.rs:24-147): fused multiply-adds for
  // positions below n8 when len >= 64, a rounded product and add for the
  // others.  The last len % 8 positions [n8, len) of a long decode need the
  // second kind; when wave 3 has no positions of its own in the last pass,
  // its lanes run those, so no wave runs both chains.
  const bool simd = len >= 64;
  const int n32 = len - len % 32;
  const int n8 = n32 + ((len - n32) / 8) * 8;
  const int last_base = (len - 1) / kAttnNT * kAttnNT;
  const bool tail_w3 = simd && n8 < len && len - last_base <= kAttnNT - 64;
  SYN_TS(1);
  // then the rest of the first pass of K rows and of the first V chunk,
  // for the positions the decode attends to
  if (wave != 0) {
    if (wave * 64 < len) load_k_rows(tid);
    else if (wave == 3 && tail_w3 && last_base == 0) load_k_rows(n8 + lane);
    if (len > 64) stage_v_chunk<CB>(V4, HD, s4, cb0, 16, vbuf + 16 * CB, wave, 1, 3, lane,
                                    min(kPvGroups, (len + 3) >> 2) - 16);
  }

  // 2. q and k: head RMSNorms (norm.rs:78-93; the q chains on wave 0 and
  //    the k chains on wave 2 at the same time) and rotate-half RoPE at pos
  //    (rope.rs:13-43)
  const float cs = cosT[(size_t)pos * HALF + hc], sn = sinT[(size_t)pos * HALF + hc];
  if constexpr (!F32) {  // the M <= 16 epilogue of the q / k / v rows
    float f;
    f = (float)a0 * sx; x0 = f * w0;
    f = (float)a1 * sx; x1 = f * w1;
  }
  float *myv = is_q ? qv : kv;
  float *mysq = is_q ? sqq : sqk;
  if (d < HD) {
    myv[d] = x0;
    mysq[sq_slot(d, HD)] = x0 * x0;
    if (!is_q) vnew[d] = x1;
  }
  if (tid < 32) exp_tab[tid] = tv;
  __syncthreads();
  SYN_TS(2);
  if (lane < 4) {
    if (wave == 0 && qn) red[lane] = sumsq_chain(sqq, HD, lane);
    if (wave == 2 && kn) red[4 + lane] = sumsq_chain(sqk, HD, lane);
  }
  __syncthreads();
  SYN_TS(3);
  if (gn && d < HD) {
    const float ss = sumsq_combine(red + (is_q ? 0 : 4), mysq, HD);
    const float scale = 1.0f / sqrtf(ss / (float)HD + eps);
    const float t = myv[d] * g;
    myv[d] = t * scale;
  }
  __syncthreads();
  if (d < HALF) {
    const float a = myv[d], b = myv[HALF + d];
    const float pp = a * cs, qq = b * sn, rr = b * cs, tt = a * sn;
    myv[d] = pp - qq;
    myv[HALF + d] = rr + tt;
  }
  __syncthreads();
  if (wj == 0 && !is_q && d < HD) {  // one writer per KV head
    kc[kv_k_index(pos, kvh, d, HD, max_seq)] = kv[d];
    vc[kv_v_index(pos, kvh, d, HD, max_seq)] = x1;
  }
  SYN_TS(4);

  // 3. scores, kAttnNT positions per pass (lane = position).  A wave runs
  //    the fused chain if any of its positions is below n8 and the plain
  //    one if any is not (unless wave 3 takes the tail, above); each lane
  //    keeps its own kind.  The lane of the new position takes the K row
  //    from LDS.
  const float scale = 1.0f / sqrtf((float)HD);
  const f32x4 *q4 = reinterpret_cast<const f32x4 *>(qv);
  float mx = -__builtin_inff();
  for (int base = 0; base < len; base += kAttnNT) {
    const bool last = base == last_base;
    const bool tw = last && tail_w3 && wave == 3;  // this wave runs the tail
    if (base > 0) load_k_rows(tw ? n8 + lane : base + tid);
    const int w0 = base + wave * 64;  // first position of this wave
    if (w0 < len || tw) {
      const int p = tw ? n8 + lane : base + tid;
      const int lim = last && tail_w3 && !tw ? n8 : len;  // positions this wave scores
      if (p == pos) {
        // only this lane reads the new row from LDS, straight into its K
        // registers: all HD/4 reads in flight at once (a select over every
        // lane needs a second row of registers, and the reads then go out
        // two at a time)
        const f32x4 *k4 = reinterpret_cast<const f32x4 *>(kv);
#pragma unroll
        for (int c = 0; c < HD4; c++) kr[c] = k4[c];
      }
      float sf = 0.0f, sp = 0.0f;
      if (!tw && simd && w0 < n8) sf = q_dot_chain<HD, true>(q4, kr);
      if (tw || !simd || (w0 + 63 >= n8 && !(last && tail_w3)))
        sp = q_dot_chain_plain<HD>(q4, kr);  // last: clobbers kr
      const float acc = simd && p < n8 ? sf : sp;
      if (p < lim) {
        const float sc = acc * scale;
        e[p] = sc;
        mx = fmaxf(mx, sc);
      }
    }
  }

  SYN_TS(5);
  // 4. softmax_slice (activation.rs:117-129): max, exp(x - max), the
  //    sequential sum (thread 0), the division when the sum is positive
  mx = wave_max_any(mx);
  if (lane == 0) red[8 + wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[8], red[9]), fmaxf(red[10], red[11]));
  SYN_TS(6);
  for (int i = tid; i < len; i += kAttnNT) e[i] = syn_expf_tab(e[i] - mx, exp_tab);
  __syncthreads();
  SYN_TS(7);
  if (wave == 0) {  // the sequential sum, run from registers by the whole wave
    const float r = wave_seq_sum(e, len, 0.0f);
    if (lane == 0) red[12] = r;
  }
  __syncthreads();
  SYN_TS(8);
  const float sum = red[12];
  if (sum > 0.0f)
    for (int i = tid; i < len; i += kAttnNT) e[i] = e[i] / sum;

  // 5. P.V: wave 0 runs the chains (lane = column; lanes >= CB repeat
  //    columns and store nothing) over 128-position chunks while waves 1-3
  //    stage the next chunk into the other buffer
  const bool fused_pv = simd && (HD % 32) == 0;
  const int col = lane % CB;
  const f32x4 *e4 = reinterpret_cast<const f32x4 *>(e);
  float acc = 0.0f;
  SYN_TS(9);
  for (int c = 0, cpos = 0; cpos < len; c++, cpos += kPvChunk) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    SYN_TS(10);
    f32x4 *buf = vbuf + (c & 1) * kPvGroups * CB;
    if (wave != 0) {
      if (cpos + kPvChunk < len)
        stage_v_chunk<CB>(V4, HD, s4, cb0, (c + 1) * kPvGroups,
                          vbuf + ((c + 1) & 1) * kPvGroups * CB, wave, 1, kAttnNT / 64 - 1, lane,
                          min(kPvGroups, (len - cpos - kPvChunk + 3) >> 2));
    } else {
      if (pos >= cpos && pos < cpos + kPvChunk && lane < CB) {  // this step's V row
        float *slot = reinterpret_cast<float *>(buf + ((pos - cpos) >> 2) * CB + col) + (pos & 3);
        *slot = vnew[cb0 + col];
      }
      const int clen = min(kPvChunk, len - cpos);
      const int ngf = clen >> 2, rem = clen & 3;
      const f32x4 *ec = e4 + c * kPvGroups;
      acc = fused_pv ? pv_chain<true, CB>(ec, buf + col, ngf, acc)
                     : pv_chain<false, CB>(ec, buf + col, ngf, acc);
      if (rem) {
        const f32x4 E = ec[ngf], Vv = buf[ngf * CB + col];
        auto one = [&](float ev, float v) {
          if (fused_pv) {
            acc = __builtin_fmaf(ev, v, acc);
          } else {
            const float t = ev * v;
            acc = acc + t;
          }
        };
        one(E.x, Vv.x);
        if (rem > 1) one(E.y, Vv.y);
        if (rem > 2) one(E.z, Vv.z);
      }
    }
  }
  if (wave == 0 && lane < CB) out[head * HD + cb0 + lane] = acc;
  SYN_TS(11);
  SYN_TSR(15);
  SYN_TS_FLUSH(48);
  SYN_TL_EXIT(20);
}

static size_t attn_head_lds_bytes(int hd, int max_seq) {
  const int cb = hd < 64 ? hd : 64;
  return (size_t)round_up4(max_seq) * 4 + 2 * (size_t)kPvGroups * cb * 16;
}
constexpr size_t kAttnHeadMaxLds = 152 * 1024;  // of 160 KiB, leaving the static rows

static bool attention_fast_ok(int hd) { return hd == 16 || hd == 32 || hd == 64 || hd == 128; }

static size_t attention_lds_bytes(int hd, int max_seq) {
  return ((size_t)4 * hd + round_up((size_t)max_seq, 4)) * sizeof(float);
}

bool fused_attention_fits(int hd, int max_seq) {
  if (attention_fast_ok(hd)) return attn_head_lds_bytes(hd, max_seq) <= kAttnHeadMaxLds;
  return attention_lds_bytes(hd, max_seq) <= 60 * 1024;
}

syn_status_t launch_fused_attention(RowSrc qkv, int nh, int nkv, int hd, const float *qn,
                                    const float *kn, float eps, const float *cosT,
                                    const float *sinT, const StepState *st, float *kc, float *vc,
                                    int max_seq, float *scores, float *out, hipStream_t s) {
  (void)scores;
  if (!fused_attention_fits(hd, max_seq)) {
    set_error("fused decode attention: max_seq too long for LDS");
    return SYN_ERR_INVALID_ARG;
  }
  if (attention_fast_ok(hd)) {
    const uint64_t *tab = exp_table_address();
    if (!tab) {
      set_error("fused decode: expf table address unavailable");
      return SYN_ERR_HIP;
    }
    const size_t shm = attn_head_lds_bytes(hd, max_seq);
    static bool attr[2][4] = {};
    auto run = [&](auto kern, int which) -> syn_status_t {
      bool &done = attr[qkv.f ? 1 : 0][which];
      if (!done) {  // more than the default 64 KiB of dynamic LDS
        SYN_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)kAttnHeadMaxLds));
        done = true;
      }
      const int cb = hd < 64 ? hd : 64;
      SYN_LAUNCH(kern, dim3((unsigned)(nh * (hd / cb))), dim3(kAttnNT), shm, s, qkv,
                         nh, nkv, qn, kn, eps, cosT, sinT, st, kc, vc, max_seq, tab, out);
      SYN_LAUNCH_CHECK();
      return SYN_OK;
    };
    auto pick = [&](auto f32c) -> syn_status_t {
      constexpr bool F = decltype(f32c)::value;
      switch (hd) {
        case 16: return run(k_attn_head<F, 16>, 0);
        case 32: return run(k_attn_head<F, 32>, 1);
        case 64: return run(k_attn_head<F, 64>, 2);
        default: return run(k_attn_head<F, 128>, 3);
      }
    };
    return qkv.f ? pick(std::true_type{}) : pick(std::false_type{});
  }
  const size_t shm = attention_lds_bytes(hd, max_seq);
  SYN_LAUNCH(k_fused_attention, dim3(nh), dim3(256), shm, s, qkv, nh, nkv, hd, qn, kn,
                     eps, cosT, sinT, st, kc, vc, max_seq, out);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ head
// final residual + RMSNorm + quantize, one workgroup of 1024 threads;
// dynamic LDS: sq[round4(H)]
__global__ void __launch_bounds__(1024)
    k_fused_final_norm(const float *__restrict__ base, RowSrc delta, const float *__restrict__ nw,
                       float eps, int H, int8_t *__restrict__ xq, float *__restrict__ s_out) {
  constexpr int NT = 1024;
  extern __shared__ __align__(16) float fsm[];
  __shared__ float red[64];
  SYN_TL_ENTER();
  const int tid = threadIdx.x;
  float x[RB], nwv[RB];
  int da[RB];
  float dw[RB];
  const bool has_delta = delta.acc != nullptr;
#pragma unroll
  for (int u = 0; u < RB; u++) {
    const int j = min(tid + u * NT, H - 1);
    x[u] = base[j];
    nwv[u] = nw[j];
    da[u] = has_delta ? delta.acc[j] : 0;
    dw[u] = has_delta ? delta.ws[j] : 0.0f;
  }
  if (has_delta) {
    const float dsx = delta.sx[0];
#pragma unroll
    for (int u = 0; u < RB; u++) {
      const float f = (float)da[u] * dsx;
      const float d = f * dw[u];
      x[u] = x[u] + d;
    }
  }
#pragma unroll
  for (int u = 0; u < RB; u++) {
    const int j = tid + u * NT;
    if (j < H) fsm[sq_slot(j, H)] = x[u] * x[u];
  }
  float t[RB];
#pragma unroll
  for (int u = 0; u < RB; u++) t[u] = x[u] * nwv[u];
  wg_max_post<NT>(local_absmax<NT, RB>(t, H), red, 0);
  __syncthreads();
  const float ss = sumsq_chains<NT>(fsm, H, red);
  const float scale = 1.0f / sqrtf(ss / (float)H + eps);
  float nv[RB];
#pragma unroll
  for (int u = 0; u < RB; u++) nv[u] = t[u] * scale;
  float mx = wg_max_get<NT>(red, 0) * scale;  // max|t*scale| = fl(max|t| * scale)
  if (!(mx <= 3.402823466e38f) || !(scale > 0.0f)) {
    wg_max_post<NT>(local_absmax<NT, RB>(nv, H), red, 16);
    __syncthreads();
    mx = wg_max_get<NT>(red, 16);
  }
  const float sv = quantize_regs_with_max<NT, RB>(nv, H, mx, xq);
  if (tid == 0) s_out[0] = sv;
  SYN_TL_EXIT(31);
}

syn_status_t launch_fused_final_norm(const float *base, RowSrc delta, const float *nw, float eps,
                                     int H, int8_t *xq, float *s_out, hipStream_t s) {
  if (H > RB * 1024) {
    set_error("fused final norm: hidden too large");
    return SYN_ERR_INVALID_ARG;
  }
  SYN_LAUNCH(k_fused_final_norm, dim3(1), dim3(1024), round_up((size_t)H, 4) * 4, s, base,
                     delta, nw, eps, H, xq, s_out);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

__global__ void __launch_bounds__(256) k_zero_i32(int *__restrict__ p, size_t n) {
  SYN_TL_ENTER();
  const size_t n4 = n / 4;
  i32x4 *p4 = reinterpret_cast<i32x4 *>(p);
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256)
    p4[i] = i32x4{0, 0, 0, 0};
  for (size_t i = n4 * 4 + (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (size_t)gridDim.x * 256)
    p[i] = 0;
  SYN_TL_EXIT(30);
}

syn_status_t launch_zero_i32(int *p, size_t n, hipStream_t s) {
  if (n == 0) return SYN_OK;
  if (reinterpret_cast<uintptr_t>(p) & 15) {
    set_error("launch_zero_i32: buffer must be 16-byte aligned");
    return SYN_ERR_INVALID_ARG;
  }
  const unsigned blocks = (unsigned)std::min<size_t>(512, cdiv(cdiv(n, 4), 256));
  SYN_LAUNCH(k_zero_i32, dim3(blocks), dim3(256), 0, s, p, n);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// one workgroup per 64-row panel; each wave takes every NW-th K chunk
template <int NW, int U>
__global__ void __launch_bounds__(NW * 64)
    k_lmhead_top2(const i32x4 *__restrict__ W, const float *__restrict__ ws, int N, int C,
                  const int8_t *__restrict__ xq, const float *__restrict__ sx,
                  float *__restrict__ logits, float *__restrict__ pv, int *__restrict__ pi,
                  float *__restrict__ pv2) {
  __shared__ int redi[NW * 64];
  SYN_TL_ENTER();
  const int panel = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const i32x4 *Wp = W + (size_t)panel * C * 64 + lane;
  int acc = 0;
  for (int c0 = 0; c0 < C; c0 += NW * U) {
    i32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = c0 + wave + u * NW;
      if (c < C) w[u] = __builtin_nontemporal_load(Wp + (size_t)c * 64);
      else w[u] = i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = c0 + wave + u * NW;
      if (c < C) {
        const i32x4 xv = *reinterpret_cast<const i32x4 *>(xq + (size_t)c * 16);
        acc = __builtin_amdgcn_sdot4(w[u].x, xv.x, acc, false);
        acc = __builtin_amdgcn_sdot4(w[u].y, xv.y, acc, false);
        acc = __builtin_amdgcn_sdot4(w[u].z, xv.z, acc, false);
        acc = __builtin_amdgcn_sdot4(w[u].w, xv.w, acc, false);
      }
    }
  }
  redi[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) s += redi[i * 64 + lane];
    const int row = panel * 64 + lane;
    Top2v t{-__builtin_inff(), -1, -__builtin_inff()};
    if (row < N) {
      const float f = (float)s * sx[0];
      const float v = f * ws[row];
      logits[row] = v;
      t = Top2v{v, row, -__builtin_inff()};
    }
    t = wave_top2(t);
    if (lane == 0) {
      pv[panel] = t.v1;
      pi[panel] = t.i1;
      pv2[panel] = t.v2;
    }
  }
  SYN_TL_EXIT(32);
}

syn_status_t launch_lmhead_top2(const void *W, const float *ws, int N, int C, const int8_t *xq,
                                const float *sx, float *logits, float *pv, int *pi, float *pv2,
                                hipStream_t s) {
  const int P = (int)cdiv((size_t)N, 64);
  SYN_LAUNCH((k_lmhead_top2<8, 8>), dim3(P), dim3(512), 0, s,
                     reinterpret_cast<const i32x4 *>(W), ws, N, C, xq, sx, logits, pv, pi, pv2);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

__global__ void __launch_bounds__(1024)
    k_argmax_advance(const float *__restrict__ pv, const int *__restrict__ pi,
                     const float *__restrict__ pv2, int np, StepState *st,
                     uint32_t *__restrict__ history, float *__restrict__ mhist) {
  __shared__ float s1[16], s2[16];
  __shared__ int si[16];
  SYN_TL_ENTER();
  Top2v t{-__builtin_inff(), -1, -__builtin_inff()};
  for (int i = threadIdx.x; i < np; i += 1024) t = top2v_merge(t, Top2v{pv[i], pi[i], pv2[i]});
  t = wave_top2(t);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s1[w] = t.v1;
    si[w] = t.i1;
    s2[w] = t.v2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Top2v r{s1[0], si[0], s2[0]};
    for (int i = 1; i < 16; i++) r = top2v_merge(r, Top2v{s1[i], si[i], s2[i]});
    const uint32_t tok = r.i1 < 0 ? 0u : (uint32_t)r.i1;
    const float margin = r.v1 - r.v2;
    const int step = st->step;
    st->token = tok;
    st->margin = margin;
    if (history) history[step] = tok;
    if (mhist) mhist[step] = margin;
    st->pos += 1;
    st->step = step + 1;
  }
  SYN_TL_EXIT(33);
}

syn_status_t launch_argmax_advance(const float *pv, const int *pi, const float *pv2, int np,
                                   StepState *st, uint32_t *history, float *mhist,
                                   hipStream_t s) {
  SYN_LAUNCH(k_argmax_advance, dim3(1), dim3(1024), 0, s, pv, pi, pv2, np, st, history,
                     mhist);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn

#ifdef SYN_PHASE_TIMING
// the step timeline: n entries of (kind, entry, exit); resets the ring
extern "C" syn_status_t syn_hip_debug_timeline(unsigned long long *host, int max_entries,
                                               int *n_out) {
  if (!host || !n_out || max_entries <= 0) return SYN_ERR_INVALID_ARG;
  SYN_HIP(hipDeviceSynchronize());
  unsigned n = 0;
  SYN_HIP(hipMemcpyFromSymbol(&n, HIP_SYMBOL(syn::syn_tl_n), 4, 0, hipMemcpyDeviceToHost));
  n = std::min<unsigned>(n, std::min<unsigned>(8192u, (unsigned)max_entries));
  if (n) SYN_HIP(hipMemcpyFromSymbol(host, HIP_SYMBOL(syn::syn_tl), (size_t)n * 24, 0,
                                     hipMemcpyDeviceToHost));
  const unsigned zero = 0;
  SYN_HIP(hipMemcpyToSymbol(HIP_SYMBOL(syn::syn_tl_n), &zero, 4, 0, hipMemcpyHostToDevice));
  *n_out = (int)n;
  return SYN_OK;
}

extern "C" syn_status_t syn_hip_debug_phase_ts(unsigned long long *host, int n) {
  if (!host || n <= 0 || n > 256) return SYN_ERR_INVALID_ARG;
  SYN_HIP(hipDeviceSynchronize());
  SYN_HIP(hipMemcpyFromSymbol(host, HIP_SYMBOL(syn::syn_phase_ts), (size_t)n * 8, 0,
                              hipMemcpyDeviceToHost));
  return SYN_OK;
}
#endif
