// One channel of the LFM2 LIV conv step (double-gated short conv, decode):
// conv1d_step_single (models/ssm/hybrid/layer.rs:25-42) inside LivConv's
// forward_one (layer.rs:609-627).  The channel's state row holds its last ck
// conv inputs B*x, oldest first; the step shifts the row, appends B*x and
// returns C * (sum_j row[j] w[j] (+ bias)), the sum folded from -0.0 in tap
// order.  The state is double-buffered by position parity: the step at
// position p reads half p & 1 and writes half (p + 1) & 1 (snew may be null
// for a reader that does not write), so kernels whose workgroups recompute
// the same channel never read a half that another is writing.
#pragma once

#include "common.hpp"

namespace syn {

constexpr int kLivMaxUnrolled = 8;  // kernels up to this many taps load them all at once

__device__ __forceinline__ float liv_conv_channel(float b_gate, float c_gate, float x_sig, int ck,
                                                  const float *__restrict__ sold,
                                                  float *__restrict__ snew,
                                                  const float *__restrict__ w,
                                                  const float *__restrict__ bias) {
  const float bx = b_gate * x_sig;
  float sum = -0.0f;
  if (ck <= kLivMaxUnrolled) {
    float sv[kLivMaxUnrolled], wv[kLivMaxUnrolled];
#pragma unroll
    for (int j = 0; j < kLivMaxUnrolled; j++)
      if (j < ck) {
        sv[j] = j + 1 < ck ? sold[j + 1] : bx;
        wv[j] = w[j];
      }
    const float bb = bias ? *bias : 0.0f;
#pragma unroll
    for (int j = 0; j < kLivMaxUnrolled; j++)
      if (j < ck) {
        if (snew) snew[j] = sv[j];
        const float t = sv[j] * wv[j];
        sum = sum + t;
      }
    const float cv = bias ? sum + bb : sum;
    return c_gate * cv;
  }
  for (int j = 0; j < ck; j++) {
    const float v = j + 1 < ck ? sold[j + 1] : bx;
    if (snew) snew[j] = v;
    const float t = v * w[j];
    sum = sum + t;
  }
  const float cv = bias ? sum + *bias : sum;
  return c_gate * cv;
}

}  // namespace syn
