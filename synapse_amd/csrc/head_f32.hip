// Tied f32 lm_head of the fused decode steps (hybrid LFM2.5, Mamba): the
// final RMSNorm in the prologue, logits over the row-major f32 embedding and
// the per-panel top-2 in the epilogue (launch_argmax_advance merges them).
//
// 256 threads, 64 rows per workgroup (16 per wave).  Lane j holds the
// normalized activations of float4 columns j + 64 c of the row (H = 256 NC),
// so a weight row is NC coalesced 1 KiB loads per wave and a butterfly sum
// (the same value in every lane).  Every wave computes the row's sum of
// squares itself from registers; logits[row] = (E[row] . (x * gain)) * (1 /
// sqrt(sum(x^2) / H + eps)), the 1/rms applied to the finished dot product.
// Rows are loaded RB at a time with no prefetch: the other waves of the SIMD
// cover the latency, and at about 100 VGPRs the whole grid stays resident.
#include "decode_fused.hpp"
#include "head_f32.hpp"
#include "klm_fused.hpp"

namespace syn {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { HEAD_FX = 0, HEAD_ACC = 1, HEAD_F32 = 2 };

template <int NC, int KIND>
__global__ void __launch_bounds__(256)
    k_head_f32_top2(const f32x4 *__restrict__ E, int V, HeadIn in, float *__restrict__ logits,
                    float *__restrict__ pv, int *__restrict__ pi, float *__restrict__ pv2) {
  constexpr int H4 = 64 * NC, RB = NC <= 4 ? 4 : 2;
  __shared__ float sv1[4], sv2[4];
  __shared__ int si1[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 64 + wave * 16;
  float4 xg[NC];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int i = lane + 64 * c;
    float4 a;
    if constexpr (KIND == HEAD_FX) {
      const long long *rp = in.fx + 4 * (size_t)i;
      a = make_float4(kqf_unfix(rp[0]), kqf_unfix(rp[1]), kqf_unfix(rp[2]), kqf_unfix(rp[3]));
    } else {
      const float4 b = reinterpret_cast<const float4 *>(in.base)[i];
      constexpr bool ACC = KIND == HEAD_ACC;
      a = make_float4(row_value_t<ACC>(in.delta, 4 * i) + b.x,
                      row_value_t<ACC>(in.delta, 4 * i + 1) + b.y,
                      row_value_t<ACC>(in.delta, 4 * i + 2) + b.z,
                      row_value_t<ACC>(in.delta, 4 * i + 3) + b.w);
    }
    const float4 g = reinterpret_cast<const float4 *>(in.gain)[i];
    ss += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
    xg[c] = make_float4(a.x * g.x, a.y * g.y, a.z * g.z, a.w * g.w);
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float inv = 1.0f / sqrtf(ss / (float)(4 * H4) + in.eps);
  Top2v t{-__builtin_inff(), -1, -__builtin_inff()};
  f32x4 w[RB][NC];
#pragma unroll 1
  for (int b = 0; b < 16; b += RB) {
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
      const int row = min(row0 + b + rr, V - 1);
#pragma unroll
      for (int c = 0; c < NC; c++)
        w[rr][c] = __builtin_nontemporal_load(E + (size_t)row * H4 + lane + 64 * c);
    }
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        a = __builtin_fmaf(w[rr][c].x, xg[c].x, a);
        a = __builtin_fmaf(w[rr][c].y, xg[c].y, a);
        a = __builtin_fmaf(w[rr][c].z, xg[c].z, a);
        a = __builtin_fmaf(w[rr][c].w, xg[c].w, a);
      }
      for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
      const int row = row0 + b + rr;
      if (row < V) {
        const float v = a * inv;
        if (lane == 0) logits[row] = v;
        t = top2v_merge(t, Top2v{v, row, -__builtin_inff()});
      }
    }
  }
  if (lane == 0) {
    sv1[wave] = t.v1;
    si1[wave] = t.i1;
    sv2[wave] = t.v2;
  }
  __syncthreads();
  if (tid == 0) {
    Top2v m{sv1[0], si1[0], sv2[0]};
    for (int i = 1; i < 4; i++) m = top2v_merge(m, Top2v{sv1[i], si1[i], sv2[i]});
    pv[blockIdx.x] = m.v1;
    pi[blockIdx.x] = m.i1;
    pv2[blockIdx.x] = m.v2;
  }
}

template <int NC>
void launch_nc(dim3 grid, hipStream_t s, const float *E, int V, const HeadIn &in, float *logits,
               float *pv, int *pi, float *pv2) {
  const f32x4 *E4 = reinterpret_cast<const f32x4 *>(E);
  if (in.fx)
    hipLaunchKernelGGL((k_head_f32_top2<NC, HEAD_FX>), grid, dim3(256), 0, s, E4, V, in, logits,
                       pv, pi, pv2);
  else if (in.delta.acc)
    hipLaunchKernelGGL((k_head_f32_top2<NC, HEAD_ACC>), grid, dim3(256), 0, s, E4, V, in, logits,
                       pv, pi, pv2);
  else
    hipLaunchKernelGGL((k_head_f32_top2<NC, HEAD_F32>), grid, dim3(256), 0, s, E4, V, in, logits,
                       pv, pi, pv2);
}

}  // namespace

bool head_f32_fits(int H) {
  return H == 256 || H == 512 || H == 768 || H == 1024 || H == 1536 || H == 2048;
}

syn_status_t launch_head_f32_top2(const float *E, int V, int H, const HeadIn &in, float *logits,
                                  float *pv, int *pi, float *pv2, hipStream_t s) {
  if (!E || !in.gain || !logits || !pv || !pi || !pv2) return SYN_ERR_NULL_PTR;
  if (!in.fx && (!in.base || in.delta.empty())) {
    set_error("f32 lm_head: the residual row needs a fixed-point row or base + delta");
    return SYN_ERR_INVALID_ARG;
  }
  if (V <= 0 || !head_f32_fits(H)) {
    set_error("f32 lm_head: hidden must be 256, 512, 768, 1024, 1536 or 2048");
    return SYN_ERR_INVALID_ARG;
  }
  const dim3 grid((unsigned)cdiv((size_t)V, 64));
  switch (H / 256) {
    case 1: launch_nc<1>(grid, s, E, V, in, logits, pv, pi, pv2); break;
    case 2: launch_nc<2>(grid, s, E, V, in, logits, pv, pi, pv2); break;
    case 3: launch_nc<3>(grid, s, E, V, in, logits, pv, pi, pv2); break;
    case 4: launch_nc<4>(grid, s, E, V, in, logits, pv, pi, pv2); break;
    case 6: launch_nc<6>(grid, s, E, V, in, logits, pv, pi, pv2); break;
    default: launch_nc<8>(grid, s, E, V, in, logits, pv, pi, pv2); break;
  }
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn
