// Token sampling on the device (generation/sampler.rs) and the host random
// stream that feeds it.
#pragma once

#include "common.hpp"
#include "layer_ops.hpp"

namespace syn {

// CombinedSampler (sampler.rs:152-157) as the kernels take it
struct SampleArgs {
  float temperature = 0.0f;
  float inv_t = 1.0f;       // 1 / temperature (f32 division on the host)
  float top_p = 1.0f;
  float rep = 1.0f;         // repetition penalty
  int top_k = 0;
  int apply_rep = 0;        // |rep - 1| > f32::EPSILON (sampler.rs:168)
};

SampleArgs make_sample_args(const syn_hip_sampler &p);

// Scratch of one sampler: a working copy of the logits, the candidate list
// and the key / index buffers of the large top-p sort, sized for `vocab`.
struct SampleScratch {
  DevBuf w, cidx, cval, status, ka, kb, va, vb;
  size_t vocab = 0;
  syn_status_t ensure(size_t v);
};

// Sample one token from logits[0..V) on `s`.  The history is hist[0..nh)
// or, with st set, the first st->step entries of hist; the draw is u[0] or,
// with st set, u[st->step].  With st set the kernel also records the token
// (st->token, history[st->step], margin history = the chosen token's
// probability, or 0 on the greedy route) and advances st->step (and st->pos
// when add_pos).
syn_status_t launch_sample(const float *logits, int V, const uint32_t *hist, int nh,
                           const SampleArgs &a, const float *u, StepState *st, int add_pos,
                           uint32_t *history, float *mhist, SampleScratch &scr,
                           uint32_t *token_out, hipStream_t s);

// The first n draws of StdRng::seed_from_u64(seed).gen::<f32>() (rand 0.8.5:
// rand_chacha 0.3.1 ChaCha12 seeded by rand_core 0.6.4's PCG32 expansion).
void host_stdrng_f32(uint64_t seed, size_t n, float *out);

}  // namespace syn
