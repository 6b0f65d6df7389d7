// C++ spelling of the weight layout (reference: kernels/model_weights.cuh:7-34).
// ModelWeights IS an ie_model_weights (same fields, bf16 pointers) with the
// reference's static constructor and free(); pass &weights to the C-ABI.
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../infengine.h"

using bf16 = ie_bf16;
using TransformerBlockWeights = ie_transformer_block_weights;
using FFNBlockWeights = ie_ffn_block_weights;
using RoPEWeights = ie_rope_weights;
using Layer = ie_layer;

struct ModelWeights : ie_model_weights {
  ModelWeights() : ie_model_weights{} {}

  // model_weights.cu:142-154: load BF16 safetensors shards (kept BF16), build RoPE tables.
  static ModelWeights from_safetensors(std::vector<std::string> safetensors_paths) {
    std::vector<const char*> p;
    for (auto& s : safetensors_paths) p.push_back(s.c_str());
    ModelWeights m;
    if (ie_model_weights_from_safetensors(&m, p.data(), (int)p.size()) < 0)
      throw std::runtime_error(ie_last_error());
    return m;
  }

  // Synthetic Llama-3.1-8B: matrices ~N(0, std), norms ~1+N(0, 0.02) (benchmarks, tests).
  static ModelWeights random_init(uint64_t seed, float std = 0.02f) {
    ModelWeights m;
    if (ie_model_weights_random_init(&m, seed, std) < 0) throw std::runtime_error(ie_last_error());
    return m;
  }

  void free() {
    if (ie_model_weights_free(this) < 0) throw std::runtime_error(ie_last_error());
  }
};
