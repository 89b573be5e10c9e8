// Decoder-layer kernels around the quantized GEMVs.  They are small and
// latency-bound; what matters is that each reproduces the reference's float
// operation order exactly (compiled with -ffp-contract=off; explicit
// __builtin_fmaf only where the reference uses @mulAdd), so the token stream
// matches the cpu_simd path bit for bit.
#include "layer_ops.hpp"
#include "reduce_order.hpp"

namespace syn {

// ------------------------------------------------------------------ embed
__global__ void k_embed(const float *__restrict__ embed, const uint32_t *__restrict__ ids,
                        int hidden, int vocab, float *__restrict__ x) {
  const int r = blockIdx.x;
  const uint32_t id = ids[r];
  float *xr = x + (size_t)r * hidden;
  if (id < (uint32_t)vocab) {
    const float *src = embed + (size_t)id * hidden;
    for (int j = threadIdx.x; j < hidden; j += blockDim.x) xr[j] = src[j];
  } else {
    for (int j = threadIdx.x; j < hidden; j += blockDim.x) xr[j] = 0.0f;
  }
}

syn_status_t launch_embed(const float *embed, const uint32_t *ids, int rows, int hidden,
                          int vocab, float *x, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(rows), dim3(256), 0, s, embed, ids, hidden, vocab, x);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ residual
__global__ void k_add(float *__restrict__ x, const float *__restrict__ d, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] + d[i];
}

syn_status_t launch_add(float *x, const float *d, int n, hipStream_t s) {
  hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, s, x, d, n);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// Sum of squares in the order of syn_vmul + syn_vreduce_sum
// (exports.zig:366-375, 503-514): lane accumulators acc[i%4] over the
// 4-aligned prefix, reduced as ((a0+a1)+a2)+a3, then the tail.  v is in LDS;
// must be called by all threads of the block (uses red[0..3] and a barrier).
__device__ float sumsq_vec4_order(const float *v, int n, float *red) {
  const int n4 = n & ~3;
  if (threadIdx.x < 4) {
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n4; i += 4) {
      const float t = v[i] * v[i];
      acc = acc + t;
    }
    red[threadIdx.x] = acc;
  }
  __syncthreads();
  float s = ((red[0] + red[1]) + red[2]) + red[3];
  for (int i = n4; i < n; i++) {
    const float t = v[i] * v[i];
    s = s + t;
  }
  return s;
}

// block-wide max of non-negative values (exact in any order)
__device__ float block_max(float v, float *red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; i++) m = fmaxf(m, red[i]);
  return m;
}

// quantize a row held in LDS (quantize.zig:12-47); all threads participate
__device__ void quantize_row_lds(const float *v, int n, int8_t *q, float *scale_out, float *red) {
  float mx = 0.0f;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const float a = fabsf(v[j]);
    if (a > mx) mx = a;
  }
  mx = block_max(mx, red);
  if (mx == 0.0f) {
    for (int j = threadIdx.x; j < n; j += blockDim.x) q[j] = 0;
    if (threadIdx.x == 0) *scale_out = 1.0f;
    return;
  }
  const float inv = 127.0f / mx;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    float r = roundf(v[j] * inv);
    r = fminf(127.0f, fmaxf(-127.0f, r));
    q[j] = (int8_t)(int)r;
  }
  if (threadIdx.x == 0) *scale_out = mx / 127.0f;
}

// ------------------------------------------------------------------ RMSNorm + quantize
// ops/norm.rs:8-38: out = (x*w) * (1/sqrt(sumsq/n + eps)); then A1 on out.
// One workgroup of NT threads per row.  The squares are written in the
// sumsq_chains layout, so the four reference chains run from LDS with
// 16-byte loads.  dynamic LDS: v[H] | sq[H]
template <int NT>
__global__ void __launch_bounds__(NT)
    k_rmsnorm_quant(float *__restrict__ x, const float *__restrict__ delta,
                    const float *__restrict__ w, float eps, int H, int8_t *__restrict__ xq,
                    int ldq, float *__restrict__ sx, float *__restrict__ normed) {
  extern __shared__ __align__(16) float sm[];
  __shared__ float red[64];
  float *v = sm, *sq = sm + round_up4(H);
  const int row = blockIdx.x;
  float *xr = x + (size_t)row * H;
  for (int j = threadIdx.x; j < H; j += NT) {
    float a = xr[j];
    if (delta) {
      a = a + delta[(size_t)row * H + j];
      xr[j] = a;
    }
    v[j] = a;
    sq[sq_slot(j, H)] = a * a;
  }
  __syncthreads();
  const float ss = sumsq_chains<NT>(sq, H, red);
  const float scale = 1.0f / sqrtf(ss / (float)H + eps);
  for (int j = threadIdx.x; j < H; j += NT) {
    const float t = v[j] * w[j];
    const float nv = t * scale;
    v[j] = nv;
    if (normed) normed[(size_t)row * H + j] = nv;
  }
  if (!xq) return;  // f32 path: normed rows only
  __syncthreads();
  quantize_row_lds(v, H, xq + (size_t)row * ldq, sx + row, red);
}

syn_status_t launch_rmsnorm_quant(float *x, const float *delta, const float *w, float eps,
                                  int rows, int hidden, int8_t *xq, int ldq, float *sx,
                                  float *normed, hipStream_t s) {
  const size_t shm = 2 * round_up((size_t)hidden, 4) * sizeof(float);
  if (shm > 64 * 1024) {
    set_error("rmsnorm: hidden size too large for the LDS row");
    return SYN_ERR_INVALID_ARG;
  }
  if (hidden >= 2048)
    hipLaunchKernelGGL(k_rmsnorm_quant<1024>, dim3(rows), dim3(1024), shm, s, x, delta, w, eps,
                       hidden, xq, ldq, sx, normed);
  else
    hipLaunchKernelGGL(k_rmsnorm_quant<256>, dim3(rows), dim3(256), shm, s, x, delta, w, eps,
                       hidden, xq, ldq, sx, normed);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ q/k norm, RoPE, KV append
// ops/attention.rs:46-66: headwise RMSNorm (norm.rs:78-93), rotate-half RoPE
// (rope.rs:13-43) at the token's position, append RoPE'd K and raw V.
// Cache row = position + cache_off: a prefill into a non-empty cache
// (cached_attention_prefill, ops/attention.rs:177-198) rotates at positions
// 0.. of the new tokens but appends after the rows already held.
// grid (n_heads + 2*n_kv, rows), one wave per head.
__global__ void __launch_bounds__(64)
    k_qk_norm_rope_kv(const float *__restrict__ qkv, int ldqkv, int nh, int nkv, int hd,
                      const float *__restrict__ qn, const float *__restrict__ kn, float eps,
                      const float *__restrict__ cosT, const float *__restrict__ sinT,
                      const int *__restrict__ d_pos, int pos_static, int cache_off,
                      float *__restrict__ q_out, float *__restrict__ kc, float *__restrict__ vc,
                      int max_seq) {
  extern __shared__ float v[];  // hd
  __shared__ float red[8];
  __shared__ float s_scale;
  const int hh = blockIdx.x, r = blockIdx.y;
  const int pos = (d_pos ? d_pos[0] : pos_static) + r;
  const int crow = pos + cache_off;
  const int qd = nh * hd, kvd = nkv * hd, half = hd / 2;
  const float *row = qkv + (size_t)r * ldqkv;
  if (hh >= nh + nkv) {  // V head: raw copy into the cache
    const int vh = hh - nh - nkv;
    for (int d = threadIdx.x; d < hd; d += 64)
      vc[kv_v_index(crow, vh, d, hd, max_seq)] = row[qd + kvd + vh * hd + d];
    return;
  }
  const bool is_q = hh < nh;
  const float *src = is_q ? row + hh * hd : row + qd + (hh - nh) * hd;
  const float *wn = is_q ? qn : kn;
  for (int d = threadIdx.x; d < hd; d += 64) v[d] = src[d];
  __syncthreads();
  if (wn) {
    const float ss = sumsq_vec4_order(v, hd, red);
    if (threadIdx.x == 0) s_scale = 1.0f / sqrtf(ss / (float)hd + eps);
    __syncthreads();
    const float scale = s_scale;
    for (int d = threadIdx.x; d < hd; d += 64) {
      const float t = v[d] * wn[d];
      v[d] = t * scale;
    }
    __syncthreads();
  }
  const float *cr = cosT + (size_t)pos * half, *sr = sinT + (size_t)pos * half;
  const int kh = hh - nh;
  for (int i = threadIdx.x; i < half; i += 64) {
    const float c = cr[i], sn = sr[i];
    const float x1 = v[i], x2 = v[half + i];
    const float a = x1 * c, b = x2 * sn;
    const float e = x2 * c, f = x1 * sn;
    if (is_q) {
      float *dst = q_out + (size_t)r * qd + hh * hd;
      dst[i] = a - b;
      dst[half + i] = e + f;
    } else {
      kc[kv_k_index(crow, kh, i, hd, max_seq)] = a - b;
      kc[kv_k_index(crow, kh, half + i, hd, max_seq)] = e + f;
    }
  }
}

syn_status_t launch_qk_norm_rope_kv(const float *qkv, int ldqkv, int rows, int n_heads,
                                    int n_kv, int head_dim, const float *q_norm,
                                    const float *k_norm, float eps, const float *rope_cos,
                                    const float *rope_sin, const int *d_pos, int pos_static,
                                    float *q_out, float *kcache, float *vcache, int max_seq,
                                    hipStream_t s, int cache_off) {
  hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3(n_heads + 2 * n_kv, rows), dim3(64),
                     head_dim * sizeof(float), s, qkv, ldqkv, n_heads, n_kv, head_dim, q_norm,
                     k_norm, eps, rope_cos, rope_sin, d_pos, pos_static, cache_off, q_out, kcache,
                     vcache, max_seq);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ decode attention
// ops/attention.rs:24-147 without a window.  len >= 64 follows the
// gather + matmul_t / matmul_nn route, whose f32GemvRow (matmul.zig:223-347)
// uses @mulAdd chains for the 32/8-wide column blocks and plain a*b+c in the
// scalar tail; len < 64 follows the scalar loops (plain a*b+c).
__global__ void __launch_bounds__(256)
    k_attn_decode(const float *__restrict__ q, const float *__restrict__ kc,
                  const float *__restrict__ vc, const int *__restrict__ d_pos, int nh, int nkv,
                  int hd, float *__restrict__ scores, int max_seq, float *__restrict__ out) {
  extern __shared__ float qs[];  // hd
  __shared__ float red[64];
  __shared__ float s_sum;
  const int head = blockIdx.x;
  const int kvh = head / (nh / nkv);
  const int len = d_pos[0] + 1;
  const bool simd = len >= 64;
  float *e = scores + (size_t)head * max_seq;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = q[head * hd + d];
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)hd);
  const int n32 = len - len % 32;
  const int n8 = n32 + ((len - n32) / 8) * 8;
  float mx = -__builtin_inff();
  for (int sidx = threadIdx.x; sidx < len; sidx += blockDim.x) {
    float acc = 0.0f;
    if (simd && sidx < n8) {
      for (int d = 0; d < hd; d++)
        acc = __builtin_fmaf(qs[d], kc[kv_k_index(sidx, kvh, d, hd, max_seq)], acc);
    } else {
      for (int d = 0; d < hd; d++) {
        const float t = qs[d] * kc[kv_k_index(sidx, kvh, d, hd, max_seq)];
        acc = acc + t;
      }
    }
    const float sc = acc * scale;
    e[sidx] = sc;
    mx = fmaxf(mx, sc);
  }
  // softmax_slice (activation.rs:117-129)
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); i++) mx = fmaxf(mx, red[i]);
  for (int sidx = threadIdx.x; sidx < len; sidx += blockDim.x) e[sidx] = syn_expf(e[sidx] - mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.0f;
    for (int i = 0; i < len; i++) sum = sum + e[i];
    s_sum = sum;
  }
  __syncthreads();
  const float sum = s_sum;
  if (sum > 0.0f)
    for (int sidx = threadIdx.x; sidx < len; sidx += blockDim.x) e[sidx] = e[sidx] / sum;
  __syncthreads();
  const int d32 = hd - hd % 32;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.0f;
    if (simd && d < d32) {
      for (int i = 0; i < len; i++)
        acc = __builtin_fmaf(e[i], vc[kv_v_index(i, kvh, d, hd, max_seq)], acc);
    } else {
      for (int i = 0; i < len; i++) {
        const float t = e[i] * vc[kv_v_index(i, kvh, d, hd, max_seq)];
        acc = acc + t;
      }
    }
    out[head * hd + d] = acc;
  }
}

syn_status_t launch_attention_decode(const float *q, const float *kcache, const float *vcache,
                                     const int *d_pos, int n_heads, int n_kv, int head_dim,
                                     float *scores, int max_seq, float *out, hipStream_t s) {
  hipLaunchKernelGGL(k_attn_decode, dim3(n_heads), dim3(256), head_dim * sizeof(float), s, q,
                     kcache, vcache, d_pos, n_heads, n_kv, head_dim, scores, max_seq, out);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ prefill attention
// syn_fused_attention per head (exports.zig:1364-1478): Q tiles of 32 rows;
// S = Q K^T and O = P V through sgemmTiled, whose element order is a
// sequential chain over k — @mulAdd inside full 8x8 micro-tiles (or in the
// f32GemvRow 32/8-wide blocks when a tile has <= 16 rows), plain a*b+c
// elsewhere — then scale, causal mask, online max/sum, normalise.  The
// keys and values are the t rows appended by this prefill (cache rows
// cache_off ..): attention.rs:200-244 attends among the new tokens only.
// grid (n_heads, t): one workgroup per (head, query row).
__device__ __forceinline__ bool sgemm_fused(int tqs, int il, int ncols, int j, bool gemv_trans_b) {
  if (tqs <= 16) {  // f32GemvRow per row (matmul.zig:142-155)
    const int n32 = ncols - ncols % 32;
    if (gemv_trans_b) {
      const int n8 = n32 + ((ncols - n32) / 8) * 8;
      return j < n8;
    }
    return j < n32;
  }
  // GOTO path: MC=256 > 32 rows, NC=4096
  const bool row_full = (tqs - (il / 8) * 8) >= 8;
  const int jc = (j / 4096) * 4096;
  const int nc = min(4096, ncols - jc);
  const bool col_full = (nc - ((j - jc) / 8) * 8) >= 8;
  return row_full && col_full;
}

__global__ void __launch_bounds__(256)
    k_attn_prefill(const float *__restrict__ q, const float *__restrict__ kc,
                   const float *__restrict__ vc, int t, int nh, int nkv, int hd, int max_seq,
                   int cache_off, float *__restrict__ out) {
  extern __shared__ float sm[];  // qs[hd] | e[t] | c[t]
  float *qs = sm, *e = sm + hd, *cj = sm + hd + t;
  __shared__ float s_mx, s_inv;
  __shared__ float cmax[256];
  const int head = blockIdx.x, i = blockIdx.y;
  const int kvh = head / (nh / nkv);
  const int qd = nh * hd;
  const int tq = (i / 32) * 32, tqs = min(32, t - tq), il = i - tq;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = q[(size_t)i * qd + head * hd + d];
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)hd);
  for (int j = threadIdx.x; j < t; j += blockDim.x) {
    float acc = 0.0f;
    if (sgemm_fused(tqs, il, t, j, true)) {
      for (int d = 0; d < hd; d++)
        acc = __builtin_fmaf(qs[d], kc[kv_k_index(cache_off + j, kvh, d, hd, max_seq)], acc);
    } else {
      for (int d = 0; d < hd; d++) {
        const float p = qs[d] * kc[kv_k_index(cache_off + j, kvh, d, hd, max_seq)];
        acc = acc + p;
      }
    }
    float sc = acc * scale;
    if (j > i) sc = -__builtin_inff();
    e[j] = sc;
  }
  __syncthreads();
  // Online max / sum in the reference's order: at position j the running max
  // is the max of e[0..j-1], so every exponential is known up front.  Thread
  // i takes the contiguous chunk i of the positions: chunk maxima, their
  // exclusive prefix, then per position the exponential the reference takes
  // there (exp(mx - x) at a new maximum, stored negated; else exp(x - mx)).
  // Only the dependent chain se = se * c + 1 / se + c stays on one thread.
  const int per = (t + (int)blockDim.x - 1) / (int)blockDim.x;
  const int j0 = min((int)threadIdx.x * per, t), j1 = min(j0 + per, t);
  float lm = -__builtin_inff();
  for (int j = j0; j < j1; j++) lm = fmaxf(lm, e[j]);
  cmax[threadIdx.x] = lm;
  __syncthreads();
  float run = -__builtin_inff();
  for (int i = 0; i < (int)threadIdx.x; i++) run = fmaxf(run, cmax[i]);
  for (int j = j0; j < j1; j++) {
    const float x = e[j];
    cj[j] = x > run ? -syn_expf(run - x) : syn_expf(x - run);
    run = fmaxf(run, x);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float mx = -__builtin_inff(), se = 0.0f;
    for (int i = 0; i < (int)blockDim.x; i++) mx = fmaxf(mx, cmax[i]);
    int j = 0;
    for (; j + 8 <= t; j += 8) {
      float c[8];
#pragma unroll
      for (int u = 0; u < 8; u++) c[u] = cj[j + u];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const float cu = fabsf(c[u]);
        const float p = se * cu;
        se = __builtin_signbit(c[u]) ? p + 1.0f : se + cu;
      }
    }
    for (; j < t; j++) {
      const float cu = fabsf(cj[j]);
      const float p = se * cu;
      se = __builtin_signbit(cj[j]) ? p + 1.0f : se + cu;
    }
    s_mx = mx;
    s_inv = 1.0f / se;
  }
  __syncthreads();
  const float mx = s_mx, inv = s_inv;
  for (int j = threadIdx.x; j < t; j += blockDim.x) e[j] = syn_expf(e[j] - mx) * inv;
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.0f;
    if (sgemm_fused(tqs, il, hd, d, false)) {
      for (int p = 0; p < t; p++)
        acc = __builtin_fmaf(e[p], vc[kv_v_index(cache_off + p, kvh, d, hd, max_seq)], acc);
    } else {
      for (int p = 0; p < t; p++) {
        const float m = e[p] * vc[kv_v_index(cache_off + p, kvh, d, hd, max_seq)];
        acc = acc + m;
      }
    }
    out[(size_t)i * qd + head * hd + d] = acc;
  }
}

// Row-block form of k_attn_prefill: one workgroup per (head, 16 query rows),
// the head's K and V rows staged through LDS 64 positions at a time, so each
// row of the cache is read once per 16 queries instead of once per query.
// Every score, sum and product is the one k_attn_prefill forms, in the same
// order (the same chains per (row, position) and (row, column)).
constexpr int kPfRows = 16, kPfChunk = 64;

template <int HD>
__global__ void __launch_bounds__(256)
    k_attn_prefill_rows(const float *__restrict__ q, const float *__restrict__ kc,
                        const float *__restrict__ vc, int t, int nh, int nkv, int max_seq,
                        int cache_off, float *__restrict__ out) {
  constexpr int hd = HD;  // compile-time: LDS offsets become immediates
  extern __shared__ float sm[];
  // qs[16][hd] | kv[64][hd + 1] | e[16][t] | c[16][t]
  const int ldk = hd + 1;
  float *qs = sm, *kv = qs + kPfRows * hd, *e = kv + kPfChunk * ldk, *cj = e + kPfRows * t;
  __shared__ float s_mx[kPfRows], s_inv[kPfRows];
  // the exp table in LDS: a per-lane lookup in it does not wait on memory
  __shared__ uint64_t etab[32];
  if (threadIdx.x < 32) etab[threadIdx.x] = syn_exp2_tab[threadIdx.x];
  const int head = blockIdx.x, i0 = blockIdx.y * kPfRows;
  const int kvh = head / (nh / nkv);
  const int qd = nh * hd;
  const int nrow = min(kPfRows, t - i0);
  const int tid = threadIdx.x;
  for (int x = tid; x < kPfRows * hd; x += blockDim.x) {
    const int r = x / hd, d = x - r * hd;
    qs[x] = r < nrow ? q[(size_t)(i0 + r) * qd + head * hd + d] : 0.0f;
  }
  const float scale = 1.0f / sqrtf((float)hd);
  // ---- scores: 16 rows x 64 positions per chunk, 4 (row, position) pairs a thread
  for (int p0 = 0; p0 < t; p0 += kPfChunk) {
    const int np = min(kPfChunk, t - p0);
    __syncthreads();  // qs written / the previous chunk consumed
    // K rows: four consecutive columns are contiguous in the cache layout;
    // eight 16-byte loads in flight per thread before the LDS stores
    const int hd4 = hd / 4, nk = np * hd4;
    for (int x0 = tid; x0 < nk; x0 += 8 * (int)blockDim.x) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int x = min(x0 + u * (int)blockDim.x, nk - 1);
        const int pp = x / hd4, d4 = x - pp * hd4;
        v[u] = *reinterpret_cast<const float4 *>(
            kc + kv_k_index(cache_off + p0 + pp, kvh, 4 * d4, hd, max_seq));
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int x = x0 + u * (int)blockDim.x;
        if (x < nk) {
          const int pp = x / hd4, d4 = x - pp * hd4;
          float *dst = kv + pp * ldk + 4 * d4;
          dst[0] = v[u].x;
          dst[1] = v[u].y;
          dst[2] = v[u].z;
          dst[3] = v[u].w;
        }
      }
    }
    __syncthreads();
    // thread: position pp of the chunk for rows rb, rb+4, rb+8, rb+12 (one K
    // row read per step, four independent chains; the fused / plain choice
    // of each chain is a select, so all four keep their own order)
    const int pp = tid % kPfChunk, rb = tid / kPfChunk;
    if (pp < np) {
      const int j = p0 + pp;
      float acc[4];
      bool fz[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int i = i0 + rb + 4 * u;
        const int tq = (i / 32) * 32, tqs = min(32, t - tq), il = i - tq;
        fz[u] = sgemm_fused(tqs, il, t, j, true);
        acc[u] = 0.0f;
      }
      const float *kr = kv + pp * ldk;
      // the four chains usually agree on fused / plain: then one loop form
      const bool all_f = fz[0] && fz[1] && fz[2] && fz[3];
      const bool none_f = !fz[0] && !fz[1] && !fz[2] && !fz[3];
      if (all_f) {
#pragma unroll 8
        for (int d = 0; d < hd; d++) {
          const float kd = kr[d];
#pragma unroll
          for (int u = 0; u < 4; u++) acc[u] = __builtin_fmaf(qs[(rb + 4 * u) * hd + d], kd, acc[u]);
        }
      } else if (none_f) {
#pragma unroll 8
        for (int d = 0; d < hd; d++) {
          const float kd = kr[d];
#pragma unroll
          for (int u = 0; u < 4; u++) {
            const float pr = qs[(rb + 4 * u) * hd + d] * kd;
            acc[u] = acc[u] + pr;
          }
        }
      } else {
#pragma unroll 8
        for (int d = 0; d < hd; d++) {
          const float kd = kr[d];
#pragma unroll
          for (int u = 0; u < 4; u++) {
            const float qv = qs[(rb + 4 * u) * hd + d];
            const float f = __builtin_fmaf(qv, kd, acc[u]);
            const float pr = qv * kd;
            const float g = acc[u] + pr;
            acc[u] = fz[u] ? f : g;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = rb + 4 * u, i = i0 + r;
        if (r < nrow) {
          float sc = acc[u] * scale;
          if (j > i) sc = -__builtin_inff();
          e[r * t + j] = sc;
        }
      }
    }
  }
  __syncthreads();
  // ---- online max / sum per row (k_attn_prefill's order): 16 threads a row
  // precompute the exponentials over contiguous chunks, one thread a row
  // runs the dependent chain
  {
    const int r = tid / 16, part = tid % 16;
    const int per = (t + 15) / 16;
    const int j0 = min(part * per, t), j1 = min(j0 + per, t);
    float *er = e + r * t, *cr = cj + r * t;
    float lm = -__builtin_inff();
    if (r < nrow)
      for (int j = j0; j < j1; j++) lm = fmaxf(lm, er[j]);
    // exclusive prefix of the chunk maxima within the 16-lane group
    float run = -__builtin_inff(), all = -__builtin_inff();
    for (int o = 0; o < 16; o++) {
      const float v = __shfl(lm, (tid & ~15) + o);
      if (o < part) run = fmaxf(run, v);
      all = fmaxf(all, v);
    }
    if (r < nrow)
      for (int j = j0; j < j1; j++) {
        const float x = er[j];
        cr[j] = x > run ? -syn_expf_tab(run - x, etab) : syn_expf_tab(x - run, etab);
        run = fmaxf(run, x);
      }
    __syncthreads();
    if (part == 0 && r < nrow) {
      float se = 0.0f;
      int j = 0;
      for (; j + 8 <= t; j += 8) {
        float c[8];
#pragma unroll
        for (int u = 0; u < 8; u++) c[u] = cr[j + u];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const float cu = fabsf(c[u]);
          const float pr = se * cu;
          se = __builtin_signbit(c[u]) ? pr + 1.0f : se + cu;
        }
      }
      for (; j < t; j++) {
        const float cu = fabsf(cr[j]);
        const float pr = se * cu;
        se = __builtin_signbit(cr[j]) ? pr + 1.0f : se + cu;
      }
      s_mx[r] = all;
      s_inv[r] = 1.0f / se;
    }
    __syncthreads();
  }
  for (int x = tid; x < nrow * t; x += blockDim.x) {
    const int r = x / t;
    e[x] = syn_expf_tab(e[x] - s_mx[r], etab) * s_inv[r];
  }
  // ---- P V: 16 rows x hd columns, chains over the positions in order.
  // hd divides 256: thread = column d for rows r0, r0 + 256/hd, ... (one V
  // read per position, hd/16 independent chains)
  const int d = tid % hd, rstep = (int)blockDim.x / hd, r0 = tid / hd, nch = kPfRows / rstep;
  constexpr int kMaxPer = 8;
  float acc[kMaxPer];
  bool fz[kMaxPer];
#pragma unroll
  for (int u = 0; u < kMaxPer; u++) {
    const int i = i0 + r0 + u * rstep;
    const int tq = (i / 32) * 32, tqs = min(32, t - tq), il = i - tq;
    fz[u] = sgemm_fused(tqs, il, hd, d, false);
    acc[u] = 0.0f;
  }
  for (int p0 = 0; p0 < t; p0 += kPfChunk) {
    const int np = min(kPfChunk, t - p0);
    __syncthreads();
    const int nv = np * hd;  // eight loads in flight per thread
    for (int x0 = tid; x0 < nv; x0 += 8 * (int)blockDim.x) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int x = min(x0 + u * (int)blockDim.x, nv - 1);
        const int pp = x / hd, dd = x - pp * hd;
        v[u] = vc[kv_v_index(cache_off + p0 + pp, kvh, dd, hd, max_seq)];
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int x = x0 + u * (int)blockDim.x;
        if (x < nv) {
          const int pp = x / hd, dd = x - pp * hd;
          kv[pp * ldk + dd] = v[u];
        }
      }
    }
    __syncthreads();
    bool all_f = true, none_f = true;
#pragma unroll
    for (int u = 0; u < kMaxPer; u++)
      if (u < nch) {
        all_f = all_f && fz[u];
        none_f = none_f && !fz[u];
      }
    if (all_f) {
#pragma unroll 4
      for (int pp = 0; pp < np; pp++) {
        const float v = kv[pp * ldk + d];
#pragma unroll
        for (int u = 0; u < kMaxPer; u++)
          if (u < nch) acc[u] = __builtin_fmaf(e[(r0 + u * rstep) * t + p0 + pp], v, acc[u]);
      }
    } else if (none_f) {
#pragma unroll 4
      for (int pp = 0; pp < np; pp++) {
        const float v = kv[pp * ldk + d];
#pragma unroll
        for (int u = 0; u < kMaxPer; u++)
          if (u < nch) {
            const float m = e[(r0 + u * rstep) * t + p0 + pp] * v;
            acc[u] = acc[u] + m;
          }
      }
    } else {
#pragma unroll 4
      for (int pp = 0; pp < np; pp++) {
        const float v = kv[pp * ldk + d];
#pragma unroll
        for (int u = 0; u < kMaxPer; u++) {
          if (u < nch) {
            const float ev = e[(r0 + u * rstep) * t + p0 + pp];
            const float f = __builtin_fmaf(ev, v, acc[u]);
            const float m = ev * v;
            const float g = acc[u] + m;
            acc[u] = fz[u] ? f : g;
          }
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kMaxPer; u++) {
    const int r = r0 + u * rstep;
    if (u < nch && r < nrow) out[(size_t)(i0 + r) * qd + head * hd + d] = acc[u];
  }
}

// Prefill attention for the tolerance-graded decoders (K-quant): the same
// causal attention over the prompt block (row i sees positions 0 .. i of
// the t new ones at cache_off), without the reference's serial order.  One
// workgroup per (head, 32 query rows); K, then V, staged through LDS 64
// positions at a time in rows padded to HD + 4 floats (16-byte aligned,
// rows four banks apart).  Eight threads per query row: thread c8 of row r
// takes positions c8 + 8k of a chunk (eight independent FMA chains over
// d), the row's max and sum by shuffles over its 8 lanes, then the output
// columns c8 + 8k (HD / 8 chains over the positions; contiguous columns per
// thread with 16-byte reads of V measured slower, 86.6 against 76.4 us at
// LLaMA-3B, 256 tokens).  The scores of the
// block's rows stay in LDS (32 x t floats).
constexpr int kPtRows = 32, kPtChunk = 64;

template <int HD>
__global__ void __launch_bounds__(256)
    k_attn_prefill_tile(const float *__restrict__ q, const float *__restrict__ kc,
                        const float *__restrict__ vc, int t, int nh, int nkv, int max_seq,
                        int cache_off, float *__restrict__ out) {
  constexpr int LD = HD + 4, HD4 = HD / 4, NCOL = HD / 8;
  constexpr int KL = kPtChunk * HD4 / 256, VL = (17 * HD + 255) / 256;  // loads per thread
  extern __shared__ __align__(16) float smt[];
  const int tps = ((t + 3) & ~3) + 1;  // odd score-row stride
  float *qs = smt, *kv = qs + kPtRows * LD, *S = kv + kPtChunk * LD;
  __shared__ float s_inv[kPtRows];
  const int head = blockIdx.x, i0 = blockIdx.y * kPtRows;
  const int kvh = head / (nh / nkv), qd = nh * HD;
  const int nrow = min(kPtRows, t - i0), npos = i0 + nrow;
  const int tid = threadIdx.x, r = tid >> 3, c8 = tid & 7;
  for (int x = tid; x < kPtRows * HD; x += 256) {
    const int rr = x / HD, d = x - rr * HD;
    qs[rr * LD + d] = rr < nrow ? q[(size_t)(i0 + rr) * qd + head * HD + d] : 0.0f;
  }
  const float scale = 1.0f / sqrtf((float)HD);
  const f32x4 *q4 = reinterpret_cast<const f32x4 *>(qs + r * LD);
  // ---- scores
  for (int p0 = 0; p0 < npos; p0 += kPtChunk) {
    const int np = min(kPtChunk, npos - p0);
    // K rows: 16 bytes (four consecutive d) per load, all issued before
    // the barrier and the LDS stores; positions past np are stored as zeros
    f32x4 kr[KL];
#pragma unroll
    for (int i = 0; i < KL; i++) {
      const int x = tid + 256 * i, p = min(x & 63, np - 1), d4 = x >> 6;
      kr[i] = *reinterpret_cast<const f32x4 *>(
          kc + kv_k_index(cache_off + p0 + p, kvh, d4 * 4, HD, max_seq));
    }
    __syncthreads();  // qs written / the previous chunk consumed
#pragma unroll
    for (int i = 0; i < KL; i++) {
      const int x = tid + 256 * i, p = x & 63, d4 = x >> 6;
      *reinterpret_cast<f32x4 *>(kv + p * LD + d4 * 4) = p < np ? kr[i] : f32x4{0, 0, 0, 0};
    }
    __syncthreads();
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int d4 = 0; d4 < HD4; d4++) {
      const f32x4 a = q4[d4];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const f32x4 b = reinterpret_cast<const f32x4 *>(kv + (c8 + 8 * k) * LD)[d4];
        acc[k] = __builtin_fmaf(a.x, b.x, acc[k]);
        acc[k] = __builtin_fmaf(a.y, b.y, acc[k]);
        acc[k] = __builtin_fmaf(a.z, b.z, acc[k]);
        acc[k] = __builtin_fmaf(a.w, b.w, acc[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int p = p0 + c8 + 8 * k;
      if (p < npos) S[r * tps + p] = p <= i0 + r ? acc[k] * scale : -__builtin_inff();
    }
  }
  __syncthreads();
  // ---- softmax of row r (positions 0 .. npos-1; masked ones are -inf)
  float mx = -__builtin_inff();
  for (int p = c8; p < npos; p += 8) mx = fmaxf(mx, S[r * tps + p]);
  mx = fmaxf(mx, __shfl_xor(mx, 1));
  mx = fmaxf(mx, __shfl_xor(mx, 2));
  mx = fmaxf(mx, __shfl_xor(mx, 4));
  float sum = 0.0f;
  for (int p = c8; p < npos; p += 8) {
    const float e = syn_expf(S[r * tps + p] - mx);
    S[r * tps + p] = e;
    sum += e;
  }
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  if (c8 == 0) s_inv[r] = 1.0f / sum;
  // ---- P.V
  float o[NCOL];
#pragma unroll
  for (int k = 0; k < NCOL; k++) o[k] = 0.0f;
  for (int p0 = 0; p0 < npos; p0 += kPtChunk) {
    const int np = min(kPtChunk, npos - p0);
    // V: 16 bytes (four consecutive positions of one d) per load, from the
    // aligned group holding position cache_off + p0 on: ng <= 17 groups
    const int P0 = cache_off + p0, g0 = P0 >> 2, ng = ((P0 + np - 1) >> 2) - g0 + 1;
    f32x4 vr[VL];
#pragma unroll
    for (int i = 0; i < VL; i++) {
      const int x = tid + 256 * i, gi = min(x / HD, ng - 1), d = x % HD;
      vr[i] = *reinterpret_cast<const f32x4 *>(vc + kv_v_index(4 * (g0 + gi), kvh, d, HD, max_seq));
    }
    __syncthreads();  // scores and s_inv written / the previous chunk consumed
#pragma unroll
    for (int i = 0; i < VL; i++) {
      const int x = tid + 256 * i, gi = x / HD, d = x % HD;
      if (gi < ng) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int lp = 4 * (g0 + gi) + j - P0;
          if (lp >= 0 && lp < np) kv[lp * LD + d] = vr[i][j];
        }
      }
    }
    __syncthreads();
    const float *srow = S + r * tps + p0;
    for (int p = 0; p < np; p++) {
      const float e = srow[p];
      const float *vr = kv + p * LD + c8;
#pragma unroll
      for (int k = 0; k < NCOL; k++) o[k] = __builtin_fmaf(e, vr[8 * k], o[k]);
    }
  }
  if (r < nrow) {
    const float inv = s_inv[r];
#pragma unroll
    for (int k = 0; k < NCOL; k++) out[(size_t)(i0 + r) * qd + head * HD + c8 + 8 * k] = o[k] * inv;
  }
}

static size_t attn_prefill_tile_lds(int hd, int t) {
  return ((size_t)(kPtRows + kPtChunk) * (hd + 4) + (size_t)kPtRows * (((t + 3) & ~3) + 1)) *
         sizeof(float);
}

syn_status_t launch_attention_prefill_tol(const float *q, const float *kcache,
                                          const float *vcache, int t, int n_heads, int n_kv,
                                          int head_dim, int max_seq, float *out, hipStream_t s,
                                          int cache_off) {
  const size_t shm = attn_prefill_tile_lds(head_dim, t);
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128) ||
      shm > 144 * 1024)
    return launch_attention_prefill(q, kcache, vcache, t, n_heads, n_kv, head_dim, max_seq,
                                    nullptr, out, s, cache_off);
  static bool attr[4] = {false, false, false, false};
  auto run = [&](auto kern, int which) -> syn_status_t {
    if (!attr[which]) {  // more than the default 64 KiB of dynamic LDS
      SYN_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  144 * 1024));
      attr[which] = true;
    }
    SYN_LAUNCH(kern, dim3(n_heads, (t + kPtRows - 1) / kPtRows), dim3(256), shm, s, q, kcache,
               vcache, t, n_heads, n_kv, max_seq, cache_off, out);
    SYN_LAUNCH_CHECK();
    return SYN_OK;
  };
  switch (head_dim) {
    case 16: return run(k_attn_prefill_tile<16>, 0);
    case 32: return run(k_attn_prefill_tile<32>, 1);
    case 64: return run(k_attn_prefill_tile<64>, 2);
    default: return run(k_attn_prefill_tile<128>, 3);
  }
}

syn_status_t launch_attention_prefill(const float *q, const float *kcache, const float *vcache,
                                      int t, int n_heads, int n_kv, int head_dim, int max_seq,
                                      float *scores, float *out, hipStream_t s, int cache_off) {
  (void)scores;
  // row-block kernel when its LDS rows fit (hd <= 128: 8 outputs a thread)
  const size_t shm_rows = (size_t)(kPfRows * head_dim + kPfChunk * (head_dim + 1) +
                                   2 * kPfRows * t) * sizeof(float);
  if ((head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128) &&
      shm_rows <= 144 * 1024) {
    static bool attr_rows[4] = {false, false, false, false};
    auto run = [&](auto kern, int which) -> syn_status_t {
      if (!attr_rows[which]) {
        SYN_HIP(hipFuncSetAttribute((const void *)kern,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 144 * 1024));
        attr_rows[which] = true;
      }
      hipLaunchKernelGGL(kern, dim3(n_heads, (t + kPfRows - 1) / kPfRows), dim3(256), shm_rows,
                         s, q, kcache, vcache, t, n_heads, n_kv, max_seq, cache_off, out);
      SYN_LAUNCH_CHECK();
      return SYN_OK;
    };
    switch (head_dim) {
      case 16: return run(k_attn_prefill_rows<16>, 0);
      case 32: return run(k_attn_prefill_rows<32>, 1);
      case 64: return run(k_attn_prefill_rows<64>, 2);
      default: return run(k_attn_prefill_rows<128>, 3);
    }
  }
  const size_t shm = (size_t)(head_dim + 2 * t) * sizeof(float);
  if (shm > 144 * 1024) {
    set_error("prefill attention: prompt too long for one workgroup's LDS rows");
    return SYN_ERR_INVALID_ARG;
  }
  static bool attr = false;
  if (!attr) {  // more than the default 64 KiB of dynamic LDS
    SYN_HIP(hipFuncSetAttribute((const void *)k_attn_prefill,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 144 * 1024));
    attr = true;
  }
  hipLaunchKernelGGL(k_attn_prefill, dim3(n_heads, t), dim3(256), shm, s, q, kcache, vcache, t,
                     n_heads, n_kv, head_dim, max_seq, cache_off, out);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ SwiGLU + quantize
__global__ void __launch_bounds__(256)
    k_swiglu_quant(const float *__restrict__ gu, int ldgu, int inter, int8_t *__restrict__ hq,
                   int ldq, float *__restrict__ sh) {
  extern __shared__ float sm[];  // inter
  __shared__ float red[64];
  const int row = blockIdx.x;
  const float *g = gu + (size_t)row * ldgu, *u = g + inter;
  for (int j = threadIdx.x; j < inter; j += blockDim.x) {
    const float a = syn_silu(g[j]);
    sm[j] = a * u[j];
  }
  __syncthreads();
  quantize_row_lds(sm, inter, hq + (size_t)row * ldq, sh + row, red);
}

syn_status_t launch_swiglu_quant(const float *gu, int ldgu, int rows, int inter, int8_t *hq,
                                 int ldq, float *sh, hipStream_t s) {
  hipLaunchKernelGGL(k_swiglu_quant, dim3(rows), dim3(256), inter * sizeof(float), s, gu, ldgu,
                     inter, hq, ldq, sh);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ SwiGLU (f32 path)
// zig/src/ops/silu.zig:85-114 (syn_swiglu, used by the f32 decoder
// decoder_layer.rs:690-700): on the 4-aligned prefix sig = 1/(1+exp(-g)),
// h = (g*sig)*u; on the tail h = (g/(1+exp(-g)))*u.
__global__ void k_swiglu_f32(const float *__restrict__ gu, int ldgu, int inter,
                             float *__restrict__ h, int ldh) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= inter) return;
  const float g = gu[(size_t)row * ldgu + i], u = gu[(size_t)row * ldgu + inter + i];
  const int n4 = inter - inter % 4;
  float t;
  if (i < n4) {
    const float sig = 1.0f / (1.0f + syn_expf(-g));
    t = g * sig;
  } else {
    t = g / (1.0f + syn_expf(-g));
  }
  h[(size_t)row * ldh + i] = t * u;
}

syn_status_t launch_swiglu_f32(const float *gu, int ldgu, int rows, int inter, float *h, int ldh,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_swiglu_f32, dim3((inter + 255) / 256, rows), dim3(256), 0, s, gu, ldgu,
                     inter, h, ldh);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ------------------------------------------------------------------ argmax
struct Top2 {
  float v1;
  int i1;
  float v2;
};

__device__ __forceinline__ Top2 top2_merge(Top2 a, Top2 b) {
  // winner: larger value; on equal values the larger index (last max)
  const bool bw = (b.v1 > a.v1) || (b.v1 == a.v1 && b.i1 > a.i1);
  const Top2 w = bw ? b : a, l = bw ? a : b;
  Top2 r;
  r.v1 = w.v1;
  r.i1 = w.i1;
  r.v2 = fmaxf(w.v2, l.v1);
  return r;
}

__device__ Top2 block_top2(Top2 t, float *sv1, int *si1, float *sv2) {
  for (int o = 32; o > 0; o >>= 1) {
    Top2 u;
    u.v1 = __shfl_xor(t.v1, o);
    u.i1 = __shfl_xor(t.i1, o);
    u.v2 = __shfl_xor(t.v2, o);
    t = top2_merge(t, u);
  }
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv1[w] = t.v1;
    si1[w] = t.i1;
    sv2[w] = t.v2;
  }
  __syncthreads();
  Top2 r{sv1[0], si1[0], sv2[0]};
  for (int i = 1; i < nw; i++) r = top2_merge(r, Top2{sv1[i], si1[i], sv2[i]});
  return r;
}

__global__ void __launch_bounds__(256)
    k_argmax_stage1(const float *__restrict__ x, int n, float *pv, int *pi, float *pv2) {
  __shared__ float sv1[4], sv2[4];
  __shared__ int si1[4];
  Top2 t{-__builtin_inff(), -1, -__builtin_inff()};
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    t = top2_merge(t, Top2{x[i], i, -__builtin_inff()});
  t = block_top2(t, sv1, si1, sv2);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = t.v1;
    pi[blockIdx.x] = t.i1;
    pv2[blockIdx.x] = t.v2;
  }
}

__global__ void __launch_bounds__(256)
    k_argmax_stage2(const float *pv, const int *pi, const float *pv2, int np, StepState *st,
                    uint32_t *history, float *mhist) {
  __shared__ float sv1[4], sv2[4];
  __shared__ int si1[4];
  Top2 t{-__builtin_inff(), -1, -__builtin_inff()};
  for (int i = threadIdx.x; i < np; i += 256) t = top2_merge(t, Top2{pv[i], pi[i], pv2[i]});
  t = block_top2(t, sv1, si1, sv2);
  if (threadIdx.x == 0) {
    const uint32_t tok = t.i1 < 0 ? 0u : (uint32_t)t.i1;
    st->token = tok;
    st->margin = t.v1 - t.v2;
    if (history) history[st->step] = tok;
    if (mhist) mhist[st->step] = t.v1 - t.v2;
  }
}

syn_status_t launch_argmax(const float *logits, int n, float *part_v, int *part_i,
                           float *part_v2, StepState *state, uint32_t *history,
                           float *margin_hist, hipStream_t s) {
  const int blocks = 256;
  hipLaunchKernelGGL(k_argmax_stage1, dim3(blocks), dim3(256), 0, s, logits, n, part_v, part_i,
                     part_v2);
  SYN_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_argmax_stage2, dim3(1), dim3(256), 0, s, part_v, part_i, part_v2, blocks,
                     state, history, margin_hist);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

__global__ void k_step_advance(StepState *st, int add_pos) {
  if (threadIdx.x == 0) {
    st->pos += add_pos;
    st->step += 1;
  }
}

syn_status_t launch_step_advance(StepState *state, int add_pos, hipStream_t s) {
  hipLaunchKernelGGL(k_step_advance, dim3(1), dim3(64), 0, s, state, add_pos);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// zero K and V rows at position st->pos of `layers` consecutive layer caches
// (the draft forward's padding, causal_lm.rs:306-315); grid (layers)
__global__ void k_kv_zero_rows(float *__restrict__ kc, float *__restrict__ vc, size_t k_stride,
                               size_t v_stride, int nkv, int hd, int max_seq,
                               const StepState *__restrict__ st) {
  const int pos = st->pos;
  float *kl = kc + (size_t)blockIdx.x * k_stride, *vl = vc + (size_t)blockIdx.x * v_stride;
  for (int i = threadIdx.x; i < nkv * hd; i += blockDim.x) {
    const int g = i / hd, d = i - g * hd;
    kl[kv_k_index(pos, g, d, hd, max_seq)] = 0.0f;
    vl[kv_v_index(pos, g, d, hd, max_seq)] = 0.0f;
  }
}

syn_status_t launch_kv_zero_rows(float *kc, float *vc, size_t k_stride, size_t v_stride,
                                 int layers, int nkv, int hd, int max_seq, const StepState *st,
                                 hipStream_t s) {
  if (layers <= 0) return SYN_OK;
  hipLaunchKernelGGL(k_kv_zero_rows, dim3(layers), dim3(256), 0, s, kc, vc, k_stride, v_stride,
                     nkv, hd, max_seq, st);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

__global__ void k_state_set(StepState *st, int pos, int nhist) {
  if (threadIdx.x == 0) {
    if (pos >= 0) st->pos = pos;
    st->nhist = nhist;
  }
}

syn_status_t launch_state_set(StepState *state, int pos, int nhist, hipStream_t s) {
  hipLaunchKernelGGL(k_state_set, dim3(1), dim3(64), 0, s, state, pos, nhist);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

}  // namespace syn

__global__ void k_eval_expf(const float *__restrict__ x, float *__restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = syn_expf(x[i]);
}

extern "C" syn_status_t syn_hip_eval_expf(const float *d_x, float *d_y, size_t n, void *stream) {
  if (n == 0) return SYN_OK;
  if (!d_x || !d_y) return SYN_ERR_NULL_PTR;
  SYN_TRY(syn::ensure_init());
  hipLaunchKernelGGL(k_eval_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     syn::pick_stream(stream), d_x, d_y, n);
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}
