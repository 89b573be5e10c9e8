// Weight files as tensor views (weights.hip): GGUF and safetensors tensors
// looked up by name, with the reference's conversions to f32 (gguf.rs:
// 208-233, 255-487; safetensors.rs:228-292; converter.rs:12-46).  The model
// loaders read their tensors through WeightSource so one name table serves
// both containers.
#pragma once

#include <initializer_list>
#include <memory>
#include <string>

#include "common.hpp"

namespace syn {

// safetensors dtypes the reference converts (safetensors.rs:228-292)
enum StDtype : uint32_t { ST_F32 = 0, ST_F16, ST_BF16, ST_I64, ST_I32, ST_U8 };

struct TensorView {
  std::string name;
  bool gguf = false;
  uint32_t type = 0;  // GGML type (gguf) or StDtype (safetensors)
  int n_dims = 0;
  uint64_t shape[8] = {};  // slowest axis first: a weight of N rows over K is {N, K}
  const uint8_t *data = nullptr;
  uint64_t nbytes = 0;
  uint64_t numel() const {
    uint64_t n = 1;
    for (int d = 0; d < n_dims; d++) n *= shape[d];
    return n;
  }
  bool is_matrix(uint64_t rows, uint64_t cols) const {
    return n_dims == 2 && shape[0] == rows && shape[1] == cols;
  }
  bool is_vector(uint64_t n) const { return numel() == n && (n_dims == 1 || shape[0] == 1); }
};

class WeightSource {
 public:
  virtual ~WeightSource() = default;
  virtual bool find(const std::string &name, TensorView *t) const = 0;
  // first of `names` present
  bool find_any(std::initializer_list<std::string> names, TensorView *t) const {
    for (const std::string &n : names)
      if (find(n, t)) return true;
    return false;
  }
};

std::unique_ptr<WeightSource> gguf_source(const syn_hip_gguf_t *g);
std::unique_ptr<WeightSource> safetensors_source(const syn_hip_safetensors_t *st);

// numel() f32 values of a tensor, converted as the reference's loaders do
// (GGUF: F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K and BF16; safetensors: F32,
// F16, BF16, I64, I32, U8)
syn_status_t tensor_to_f32(const TensorView &t, float *out);

}  // namespace syn
