// CombinedSampler on the device (generation/sampler.rs:152-259):
// repetition penalty -> temperature -> top-k -> top-p -> softmax + draw.
//
// One workgroup of 1024 threads per call; the logits are copied into a
// scratch vector and every float operation is the reference's, in its order:
// the sums of softmax_inplace and top_p_filter and the categorical draw are
// sequential in index (or sorted-probability) order, so they run on one
// thread over the list of candidates (the finite logits after top-k, in
// index order; the other logits contribute exact zeros).
//
// top-k: the k-th largest value is found among the values >= L, where L is
// the k-th largest of the threads' maxima (at least k values are >= L, so
// the top k are all among them); those candidates are sorted in LDS.  When
// more than kSortMax values are >= L, a 32-step binary search over the order
// of the value keys finds the threshold instead.  top-p sorts the candidates
// by probability (descending, index ascending among equal probabilities):
// up to kSortMax of them with a bitonic sort in LDS, more (top-p without
// top-k over a large vocabulary) with a stable radix sort in global memory,
// one bit per pass over the candidates' list.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "sampler.hpp"

namespace syn {

constexpr int kSampNT = 1024;
constexpr int kSortMax = 4096;

// float -> unsigned key with the same order (-0 below +0)
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// block-wide sum / max of one value per thread (every thread gets it)
__device__ int block_sum_i(int v, int *red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  int s = 0;
  for (int i = 0; i < kSampNT / 64; i++) s += red[i];
  return s;
}

// argmax with sampler.rs:217-224's tie rule (the last maximum wins): the
// largest value, the largest index among equal values
__device__ uint32_t block_argmax(const float *w, int V, float *redf, int *redi) {
  float bv = -__builtin_inff();
  int bi = -1;
  for (int i = threadIdx.x; i < V; i += kSampNT) {
    const float x = w[i];
    if (bi < 0 || !(x < bv)) {
      bv = x;
      bi = i;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
      bv = ov;
      bi = oi;
    }
  }
  const int w_ = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    redf[w_] = bv;
    redi[w_] = bi;
  }
  __syncthreads();
  float rv = redf[0];
  int ri = redi[0];
  for (int i = 1; i < kSampNT / 64; i++) {
    const float ov = redf[i];
    const int oi = redi[i];
    if (oi >= 0 && (ri < 0 || ov > rv || (ov == rv && oi > ri))) {
      rv = ov;
      ri = oi;
    }
  }
  return ri < 0 ? 0u : (uint32_t)ri;
}

// ascending bitonic sort of n (a power of two <= kSortMax) keys in LDS
__device__ void bitonic_sort(unsigned long long *buf, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += kSampNT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long a = buf[i], b = buf[ixj];
          const bool asc = (i & k) == 0;
          if ((a > b) == asc) {
            buf[i] = b;
            buf[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Write the entries of w[0..V) that satisfy keep(value), in index order, to
// cidx/cval; returns their count (every thread).  Thread t owns the
// contiguous range [t*chunk, (t+1)*chunk).
template <class Keep>
__device__ int compact(const float *w, int V, Keep keep, uint32_t *cidx, float *cval,
                       int *scan, int *red) {
  const int chunk = (V + kSampNT - 1) / kSampNT;
  const int b = min(V, threadIdx.x * chunk), e = min(V, b + chunk);
  int c = 0;
  for (int i = b; i < e; i++) c += keep(w[i]) ? 1 : 0;
  scan[threadIdx.x] = c;
  __syncthreads();
  // exclusive scan of 1024 counts (Hillis-Steele in LDS)
  for (int o = 1; o < kSampNT; o <<= 1) {
    const int v = threadIdx.x >= o ? scan[threadIdx.x - o] : 0;
    __syncthreads();
    scan[threadIdx.x] += v;
    __syncthreads();
  }
  const int total = scan[kSampNT - 1];
  int off = scan[threadIdx.x] - c;
  for (int i = b; i < e; i++) {
    const float x = w[i];
    if (keep(x)) {
      cidx[off] = (uint32_t)i;
      cval[off] = x;
      off++;
    }
  }
  (void)red;
  __syncthreads();
  return total;
}

// exclusive prefix sum of one int per thread over the block; *total gets the
// sum (every thread)
__device__ int block_excl_scan(int v, int *scan, int *total) {
  scan[threadIdx.x] = v;
  __syncthreads();
  for (int o = 1; o < kSampNT; o <<= 1) {
    const int t = threadIdx.x >= o ? scan[threadIdx.x - o] : 0;
    __syncthreads();
    scan[threadIdx.x] += t;
    __syncthreads();
  }
  *total = scan[kSampNT - 1];
  const int r = scan[threadIdx.x] - v;
  __syncthreads();
  return r;
}

// Stable ascending sort of the n (key, index) pairs in (ka, va) by the key
// bits below `bits`: one stable partition per bit (zeros before ones, each
// in their order), ping-ponging with (kb, vb).  Thread t owns a contiguous
// range, so a block scan of the zero counts places every element.  Returns
// the buffer pair that holds the result (0: ka/va, 1: kb/vb).
__device__ int radix_sort_global(uint32_t *ka, uint32_t *va, uint32_t *kb, uint32_t *vb, int n,
                                 int bits, int *scan) {
  const int chunk = (n + kSampNT - 1) / kSampNT;
  const int b = min(n, (int)threadIdx.x * chunk), e = min(n, b + chunk);
  int cur = 0;
  for (int bit = 0; bit < bits; bit++) {
    const uint32_t *ks = cur ? kb : ka, *vs = cur ? vb : va;
    uint32_t *kd = cur ? ka : kb, *vd = cur ? va : vb;
    int z = 0;
    for (int i = b; i < e; i++) z += ((ks[i] >> bit) & 1u) ? 0 : 1;
    int zeros;
    int zo = block_excl_scan(z, scan, &zeros);
    int oo = zeros + (b - zo);  // ones before this range: elements before it minus zeros
    for (int i = b; i < e; i++) {
      const uint32_t k = ks[i], v = vs[i];
      const int d = ((k >> bit) & 1u) ? oo++ : zo++;
      kd[d] = k;
      vd[d] = v;
    }
    __syncthreads();
    cur ^= 1;
  }
  return cur;
}

// softmax's exponentials exp(v - mx) in place (all threads), then their
// sequential sum in list order (thread 0, loads 16 ahead of the adds);
// every thread gets the sum
__device__ float exp_then_seq_sum(float *v, int n, float mx, float *slot) {
  for (int i = threadIdx.x; i < n; i += kSampNT) v[i] = syn_expf(v[i] - mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
      float e[16];
#pragma unroll
      for (int k = 0; k < 16; k++) e[k] = v[i + k];
#pragma unroll
      for (int k = 0; k < 16; k++) s = s + e[k];
    }
    for (; i < n; i++) s = s + v[i];
    slot[0] = s;
  }
  __syncthreads();
  return slot[0];
}

__global__ void __launch_bounds__(kSampNT)
    k_sample(const float *__restrict__ logits, int V, const uint32_t *__restrict__ hist, int nh_arg,
             SampleArgs a, const float *__restrict__ u_src, StepState *st, int add_pos,
             uint32_t *__restrict__ history, float *__restrict__ mhist, float *__restrict__ w,
             uint32_t *__restrict__ cidx, float *__restrict__ cval, int *__restrict__ status,
             uint32_t *__restrict__ token_out, uint32_t *__restrict__ ka,
             uint32_t *__restrict__ kb, uint32_t *__restrict__ va, uint32_t *__restrict__ vb) {
  __shared__ unsigned long long sbuf[kSortMax];
  __shared__ int scan[kSampNT];
  __shared__ float redf[32];
  __shared__ int redi[32];
  __shared__ float bcast_f[4];
  __shared__ int bcast_i[4];
  __shared__ int s_err;  // block-uniform error flag
  const int tid = threadIdx.x;
  const int step = st ? st->step : 0;
  const int nh = st ? (st->nhist >= 0 ? st->nhist : step) : nh_arg;
  const float u = u_src[st ? step : 0];
  if (tid == 0) s_err = 0;

  // the working copy; repetition penalty (sampler.rs:132-149, every
  // occurrence in history order, one thread)
  for (int i = tid; i < V; i += kSampNT) w[i] = logits[i];
  __syncthreads();
  if (a.apply_rep) {
    if (tid == 0) {
      for (int j = 0; j < nh; j++) {
        const uint32_t idx = hist[j];
        if (idx < (uint32_t)V) {
          const float x = w[idx];
          w[idx] = x > 0.0f ? x / a.rep : x * a.rep;
        }
      }
    }
    __syncthreads();
  }

  uint32_t tok = 0;
  float chosen_p = 0.0f;
  bool done = false;
  if (a.temperature <= 0.0f) {  // sampler.rs:172-174
    tok = block_argmax(w, V, redf, redi);
    done = true;
  } else {
    for (int i = tid; i < V; i += kSampNT) w[i] = w[i] * a.inv_t;
    __syncthreads();
    if (a.top_k > 0 && a.top_k < V && a.top_k == 1) {
      tok = block_argmax(w, V, redf, redi);
      done = true;
    }
  }

  int nc = 0;  // candidates (cidx/cval, index order)
  if (!done) {
    const bool topk = a.top_k > 1 && a.top_k < V;
    if (topk) {
      // L = the k-th largest of the threads' maxima (k <= 1024), or -inf
      float tmax = -__builtin_inff();
      for (int i = tid; i < V; i += kSampNT) tmax = fmaxf(tmax, w[i]);
      float L = -__builtin_inff();
      if (a.top_k <= kSampNT) {
        sbuf[tid] = ((unsigned long long)(~fkey(tmax)) << 32) | (unsigned)tid;
        __syncthreads();
        bitonic_sort(sbuf, kSampNT);
        L = fkey_inv(~(uint32_t)(sbuf[a.top_k - 1] >> 32));
        __syncthreads();
      }
      nc = compact(w, V, [L](float x) { return x >= L; }, cidx, cval, scan, redi);
      float thr;
      if (nc <= kSortMax) {
        // the k-th largest value among the candidates (top_k_filter's threshold)
        int n2 = 1;
        while (n2 < nc) n2 <<= 1;
        for (int i = tid; i < n2; i += kSampNT)
          sbuf[i] = i < nc ? ((unsigned long long)(~fkey(cval[i])) << 32) | (unsigned)i : ~0ull;
        __syncthreads();
        bitonic_sort(sbuf, n2);
        thr = fkey_inv(~(uint32_t)(sbuf[a.top_k - 1] >> 32));
        __syncthreads();
      } else {
        // the largest key T with at least k values >= T, bit by bit
        uint32_t T = 0;
        for (int bit = 31; bit >= 0; bit--) {
          const uint32_t cand = T | (1u << bit);
          int c = 0;
          for (int i = tid; i < V; i += kSampNT) c += fkey(w[i]) >= cand ? 1 : 0;
          if (block_sum_i(c, redi) >= a.top_k) T = cand;
        }
        thr = fkey_inv(T);
      }
      // top_k_filter keeps the values that are not below the threshold
      nc = compact(w, V, [thr](float x) { return !(x < thr); }, cidx, cval, scan, redi);
    } else {
      nc = compact(w, V, [](float x) { return x > -__builtin_inff(); }, cidx, cval, scan, redi);
    }

    if (a.top_p > 0.0f && a.top_p < 1.0f) {  // top_p_filter (sampler.rs:279-319)
      // softmax over the candidates: max, exp, sequential sum, division
      float mx = -__builtin_inff();
      for (int i = tid; i < nc; i += kSampNT) mx = fmaxf(mx, cval[i]);
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      __syncthreads();
      if ((tid & 63) == 0) redf[tid >> 6] = mx;
      __syncthreads();
      mx = redf[0];
      for (int i = 1; i < kSampNT / 64; i++) mx = fmaxf(mx, redf[i]);
      float *pr = w;  // the probabilities, in the free working vector
      for (int i = tid; i < nc; i += kSampNT) pr[i] = cval[i];
      __syncthreads();
      const float sum = exp_then_seq_sum(pr, nc, mx, bcast_f);
      if (sum > 0.0f)
        for (int i = tid; i < nc; i += kSampNT) pr[i] = pr[i] / sum;
      __syncthreads();
      // the candidates sorted by probability descending, index ascending
      // among equal ones: rank r holds token sidx[r] with probability sp[r]
      const uint32_t *sidx;
      const uint32_t *skey;
      if (nc <= kSortMax) {
        int n2 = 1;
        while (n2 < nc) n2 <<= 1;
        for (int i = tid; i < n2; i += kSampNT)
          sbuf[i] = i < nc ? ((unsigned long long)(~fkey(pr[i])) << 32) | cidx[i] : ~0ull;
        __syncthreads();
        bitonic_sort(sbuf, n2);
        for (int i = tid; i < nc; i += kSampNT) {
          ka[i] = ~(uint32_t)(sbuf[i] >> 32);  // fkey of the probability
          va[i] = (uint32_t)(sbuf[i] & 0xffffffffu);
        }
        __syncthreads();
        sidx = va;
        skey = ka;
      } else {
        // probabilities are >= +0, so ~bits orders them descending; the
        // sign bit is set in every key and needs no pass
        for (int i = tid; i < nc; i += kSampNT) {
          ka[i] = ~__float_as_uint(pr[i]);
          va[i] = cidx[i];
        }
        __syncthreads();
        const int in_b = radix_sort_global(ka, va, kb, vb, nc, 31, scan);
        for (int i = tid; i < nc; i += kSampNT) {  // as fkey, like the LDS route
          const uint32_t k = in_b ? kb[i] : ka[i];
          (in_b ? kb : ka)[i] = ~k | 0x80000000u;
        }
        __syncthreads();
        sidx = in_b ? vb : va;
        skey = in_b ? kb : ka;
      }
      // cumulative probability in sorted order until it reaches p
      if (tid == 0) {
        float cum = 0.0f;
        int j = 0;
        for (; j < nc; j++) {
          const float p = fkey_inv(skey[j]);
          cum += p;
          if (cum >= a.top_p) {
            j++;
            break;
          }
        }
        bcast_i[0] = j;
      }
      __syncthreads();
      const int keep_n = bcast_i[0];
      // drop the candidates outside the nucleus: mark through w
      for (int i = tid; i < nc; i += kSampNT) w[i] = 0.0f;
      __syncthreads();
      for (int r = tid; r < keep_n; r += kSampNT) {
        // rank r holds token idx; find its candidate slot by binary search
        const uint32_t idx = sidx[r];
        int lo = 0, hi = nc - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (cidx[mid] < idx) lo = mid + 1;
          else hi = mid;
        }
        w[lo] = 1.0f;
      }
      __syncthreads();
      for (int i = tid; i < nc; i += kSampNT)
        if (w[i] == 0.0f) cval[i] = -__builtin_inff();
      __syncthreads();
    }

    // softmax_sample (sampler.rs:227-259) over the candidates in index order
    if (s_err == 0) {
      float mx = -__builtin_inff();
      for (int i = tid; i < nc; i += kSampNT) mx = fmaxf(mx, cval[i]);
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      __syncthreads();
      if ((tid & 63) == 0) redf[tid >> 6] = mx;
      __syncthreads();
      mx = redf[0];
      for (int i = 1; i < kSampNT / 64; i++) mx = fmaxf(mx, redf[i]);
      __syncthreads();
      const float sum = exp_then_seq_sum(cval, nc, mx, bcast_f);
      if (sum > 0.0f)
        for (int i = tid; i < nc; i += kSampNT) cval[i] = cval[i] / sum;
      __syncthreads();
      if (tid == 0) {
        float cum = 0.0f;
        uint32_t t = (uint32_t)(V - 1);  // the reference's fallback: the last token
        float pt = 0.0f;
        for (int i = 0; i < nc; i++) {
          cum += cval[i];
          if (u < cum) {
            t = cidx[i];
            pt = cval[i];
            break;
          }
        }
        bcast_i[1] = (int)t;
        bcast_f[1] = pt;
      }
      __syncthreads();
      tok = (uint32_t)bcast_i[1];
      chosen_p = bcast_f[1];
    }
  }

  if (tid == 0) {
    status[0] = s_err;
    if (token_out) token_out[0] = tok;
    if (st) {
      st->token = tok;
      st->margin = chosen_p;
      if (history) history[step] = tok;
      if (mhist) mhist[step] = chosen_p;
      st->pos += add_pos;
      st->step = step + 1;
    }
  }
}

SampleArgs make_sample_args(const syn_hip_sampler &p) {
  SampleArgs a;
  a.temperature = p.temperature;
  a.inv_t = p.temperature > 0.0f ? 1.0f / p.temperature : 1.0f;
  a.top_k = (int)std::min<uint32_t>(p.top_k, 0x7fffffffu);
  a.top_p = p.top_p;
  a.rep = p.repetition_penalty;
  a.apply_rep = std::fabs(p.repetition_penalty - 1.0f) > 1.1920929e-07f ? 1 : 0;
  return a;
}

syn_status_t SampleScratch::ensure(size_t v) {
  if (vocab >= v && w.p) return SYN_OK;
  SYN_HIP(hipDeviceSynchronize());
  SYN_TRY(w.alloc(v * 4));
  SYN_TRY(cidx.alloc(v * 4));
  SYN_TRY(cval.alloc(v * 4));
  SYN_TRY(status.alloc(64));
  SYN_TRY(ka.alloc(v * 4));
  SYN_TRY(kb.alloc(v * 4));
  SYN_TRY(va.alloc(v * 4));
  SYN_TRY(vb.alloc(v * 4));
  vocab = v;
  return SYN_OK;
}

syn_status_t launch_sample(const float *logits, int V, const uint32_t *hist, int nh,
                           const SampleArgs &a, const float *u, StepState *st, int add_pos,
                           uint32_t *history, float *mhist, SampleScratch &scr,
                           uint32_t *token_out, hipStream_t s) {
  if (V <= 0) return SYN_ERR_INVALID_ARG;
  if (scr.vocab < (size_t)V || !scr.w.p) {
    set_error("sampler scratch not prepared for this vocabulary");
    return SYN_ERR_INTERNAL;
  }
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(kSampNT), 0, s, logits, V, hist, nh, a, u, st,
                     add_pos, history, mhist, scr.w.as<float>(), scr.cidx.as<uint32_t>(),
                     scr.cval.as<float>(), scr.status.as<int>(), token_out,
                     scr.ka.as<uint32_t>(), scr.kb.as<uint32_t>(), scr.va.as<uint32_t>(),
                     scr.vb.as<uint32_t>());
  SYN_LAUNCH_CHECK();
  return SYN_OK;
}

// ---------------------------------------------------------------- host RNG
static uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

// one ChaCha block (64-bit block counter in words 12-13, stream 0)
static void chacha_block(const uint32_t key[8], uint64_t counter, int rounds, uint32_t out[16]) {
  const uint32_t init[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                             key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                             (uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u};
  uint32_t x[16];
  std::memcpy(x, init, sizeof(x));
  auto qr = [&](int a, int b, int c, int d) {
    x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 16);
    x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 12);
    x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 8);
    x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 7);
  };
  for (int r = 0; r < rounds; r += 2) {
    qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
    qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
  }
  for (int i = 0; i < 16; i++) out[i] = x[i] + init[i];
}

void host_stdrng_f32(uint64_t seed, size_t n, float *out) {
  // rand_core seed_from_u64: PCG32 steps (state advanced first, XSH-RR
  // output) give the eight little-endian key words
  uint32_t key[8];
  uint64_t state = seed;
  for (int i = 0; i < 8; i++) {
    state = state * 6364136223846793005ull + 11634580027462260723ull;
    const uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
  }
  // ChaCha12Rng: next_u32 walks a buffer of four consecutive blocks;
  // gen::<f32>() = (u32 >> 8) * 2^-24
  uint32_t buf[64];
  uint64_t ctr = 0;
  size_t idx = 64;
  for (size_t i = 0; i < n; i++) {
    if (idx >= 64) {
      for (int b = 0; b < 4; b++) chacha_block(key, ctr + (uint64_t)b, 12, buf + 16 * b);
      ctr += 4;
      idx = 0;
    }
    out[i] = (float)(buf[idx++] >> 8) * (1.0f / 16777216.0f);
  }
}

}  // namespace syn

using namespace syn;

namespace {
struct StandaloneSampler {
  SampleScratch scr;
  DevBuf u;
};
StandaloneSampler &standalone() {
  static StandaloneSampler s;
  return s;
}
}  // namespace

extern "C" syn_status_t syn_hip_sample(const float *d_logits, size_t vocab,
                                       const uint32_t *d_history, size_t n_history,
                                       const syn_hip_sampler *params, float u, uint32_t *d_token,
                                       int *d_status, void *stream) {
  if (vocab == 0) return SYN_OK;
  if (!d_logits || !params || !d_token || (n_history && !d_history)) return SYN_ERR_NULL_PTR;
  if (vocab > 0x7fffffffu || n_history > 0x7fffffffu) return SYN_ERR_INVALID_ARG;
  SYN_TRY(ensure_init());
  StandaloneSampler &S = standalone();
  SYN_TRY(S.scr.ensure(vocab));
  if (!S.u.p) SYN_TRY(S.u.alloc(256));
  hipStream_t s = pick_stream(stream);
  // the draw as a kernel argument would do; a 4-byte upload keeps one kernel
  SYN_HIP(hipMemcpyAsync(S.u.p, &u, 4, hipMemcpyHostToDevice, s));
  const SampleArgs a = make_sample_args(*params);
  SYN_TRY(launch_sample(d_logits, (int)vocab, d_history, (int)n_history, a, S.u.as<float>(),
                        nullptr, 0, nullptr, nullptr, S.scr, d_token, s));
  if (d_status)
    SYN_HIP(hipMemcpyAsync(d_status, S.scr.status.p, 4, hipMemcpyDeviceToDevice, s));
  return SYN_OK;
}

extern "C" syn_status_t syn_hip_stdrng_f32(uint64_t seed, size_t n, float *out) {
  if (n == 0) return SYN_OK;
  if (!out) return SYN_ERR_NULL_PTR;
  host_stdrng_f32(seed, n, out);
  return SYN_OK;
}
