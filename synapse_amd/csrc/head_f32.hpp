// Tied f32 lm_head of a fused decode step (head_f32.hip): RMSNorm of the
// residual row in the prologue, logits = (E[row] . (x * gain)) / rms(x) over
// the row-major f32 embedding, and the per-panel top-2 for
// launch_argmax_advance.  The sums run in tree order (the decoders that use
// it are graded by tolerance).
#pragma once

#include "decode_fused.hpp"

namespace syn {

// The residual row x: a fixed-point row (value * 2^32 in an int64), or
// base + delta with delta a RowSrc (an INT8 GEMV's int32 accumulator with its
// scales, or f32 values; x = delta + base, the residual add of the caller)
struct HeadIn {
  const long long *fx = nullptr;
  const float *base = nullptr;
  RowSrc delta;
  const float *gain = nullptr;
  float eps = 0.0f;
};

// whether the kernel takes a row of H elements (256 * {1, 2, 3, 4, 6, 8})
bool head_f32_fits(int H);
// grid cdiv(V, 64) panels: pv / pi / pv2 hold cdiv(V, 64) entries
syn_status_t launch_head_f32_top2(const float *E, int V, int H, const HeadIn &in, float *logits,
                                  float *pv, int *pi, float *pv2, hipStream_t s);

}  // namespace syn
