// Exact-order f32 kernels shared by the f32-weight decoders (mamba.hip).
#pragma once

#include <vector>

#include "common.hpp"

namespace syn {

// [n][k] row-major f32 weights -> the [panel][K/4][64][4] layout of the
// exact-order GEMV (zero padded)
std::vector<float> to_panels(const float *w_nk, size_t n, size_t k);
// rows of the 32- and 8-wide column blocks of f32GemvRow (matmul.zig:223-305)
int n8_of(int n);
// floats the activation buffer of a K-long exact f32 GEMV must hold
size_t f32_exact_x_elems(size_t K);
// y[N] = W x in f32GemvRow order (one sequential chain over k per row,
// @mulAdd for rows < n8): W in to_panels layout, x padded to
// f32_exact_x_elems(K) floats
syn_status_t launch_gemv_f32_exact(const float *Wp, const float *x, size_t x_elems, int N, int K,
                                   int n8, float *y, hipStream_t s);

}  // namespace syn
