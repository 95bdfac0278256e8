#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "common.hpp"
#include "safetensors.hpp"

namespace s1 {

enum class TensorKind { Weight, NormWeight, Bias };

struct TensorSpec {
  std::string name;
  std::vector<int64_t> shape;
  TensorKind kind;
};

// Every tensor of a decision-model checkpoint, in file order.
std::vector<TensorSpec> checkpoint_layout(const ModelConfig& c, int scorer_width, int n_act);

// The checkpoint as safetensors bytes (bf16 tensors).
std::vector<uint8_t> synth_checkpoint(const ModelConfig& c, uint64_t seed, int scorer_width, int n_act, bool jitter);

// One standard-normal draw of the generator, exposed so tests can recompute single values.
double synth_normal(uint64_t key, uint64_t e);
uint64_t synth_key(uint64_t seed, const std::string& name);

}  // namespace s1
