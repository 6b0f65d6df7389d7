// Request driver over the engine API (reference: manager.h:6-17, manager.cpp:31-110),
// without the tokenizer: prompt and output are token ids.  Differences from the
// reference loop: it stops at max_new_tokens or an EOS id, keeps the decode
// step on the context's stream (hipGraph replay inside ie_decode_step), and
// reports prefill and per-token decode time separately (manager.cpp:95 divides
// the whole run by 100).  Needs the HIP runtime API for buffer allocation.
#pragma once
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <stdexcept>
#include <string>
#include <vector>

#include "engine.h"

class Manager {
 public:
  struct Timing {
    double prefill_ms = 0.0;
    double decode_ms = 0.0;
    int decode_tokens = 0;
    double ms_per_token() const { return decode_tokens ? decode_ms / decode_tokens : 0.0; }
  };

  // Manager::Manager (manager.cpp:17-25) loads safetensors shards.
  explicit Manager(const std::vector<std::string>& model_files, int device = 0)
      : model_weights(ModelWeights::from_safetensors(model_files)) {
    init(device);
  }
  // Synthetic weights (benchmarks and tests).
  Manager(uint64_t random_seed, float std, int device = 0)
      : model_weights(ModelWeights::random_init(random_seed, std)) {
    init(device);
  }
  ~Manager() {
    release();
    model_weights.free();
    ie_destroy_handle(handle);
  }
  Manager(const Manager&) = delete;
  Manager& operator=(const Manager&) = delete;

  // manager.cpp:31-110: prefill the prompt, then greedy decode_step until
  // max_new_tokens or eos_token.  Returns prompt + generated ids.
  std::vector<int> handle_request(const std::vector<int>& prompt, int max_new_tokens,
                                  int eos_token = -1) {
    using clock = std::chrono::steady_clock;
    if (prompt.empty()) throw std::invalid_argument("handle_request: empty prompt");
    if ((int)prompt.size() + max_new_tokens > InfEngineConfig::MAX_CONTEXT_LENGTH)
      throw std::invalid_argument("handle_request: request exceeds the 8192-position KV cache");
    ensure_buffers((int)prompt.size());
    std::vector<int> tokens = prompt;
    check(hipMemcpy(tokenid_buff, tokens.data(), tokens.size() * sizeof(int),
                    hipMemcpyHostToDevice));
    timing = Timing{};
    auto t0 = clock::now();
    int tok = prefill(handle, model_weights, (int)tokens.size(), tokenid_buff, data_buffer,
                      aux_buffer, attn_buffer, output_distr, output_token, workspace, kv_cache);
    timing.prefill_ms = std::chrono::duration<double, std::milli>(clock::now() - t0).count();
    tokens.push_back(tok);
    auto t1 = clock::now();
    for (int n = 1; n < max_new_tokens && tok != eos_token; ++n) {
      // the new token goes into tokenid_buff[seq_len - 1] (manager.cpp:84)
      check(hipMemcpy(tokenid_buff + tokens.size() - 1, output_token, sizeof(int),
                      hipMemcpyDeviceToDevice));
      tok = decode_step(handle, model_weights, (int)tokens.size(), tokenid_buff, data_buffer,
                        aux_buffer, attn_buffer, output_distr, output_token, workspace, kv_cache);
      tokens.push_back(tok);
      ++timing.decode_tokens;
    }
    timing.decode_ms = std::chrono::duration<double, std::milli>(clock::now() - t1).count();
    return tokens;
  }

  const Timing& last_timing() const { return timing; }
  const ModelWeights& weights() const { return model_weights; }

 private:
  static void check(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
  }

  void init(int device) {
    check(hipSetDevice(device));
    handle = ie_create_handle(device, nullptr);
  }

  // manager.cpp:38-67: token buffer, data/aux/attn [8192, 4096], logits, token,
  // workspace sized for the prompt, 1 GiB KV cache.
  void ensure_buffers(int prompt_len) {
    const size_t ws = std::max(attn_workspace_size(prompt_len), ffn_workspace_size(prompt_len));
    if (workspace && ws <= workspace_bytes) return;
    release();
    const size_t act = (size_t)InfEngineConfig::MAX_CONTEXT_LENGTH *
                       InfEngineConfig::HIDDEN_SIZE * sizeof(bf16);
    check(hipMalloc(&tokenid_buff, InfEngineConfig::MAX_CONTEXT_LENGTH * sizeof(int)));
    check(hipMalloc(&data_buffer, act));
    check(hipMalloc(&aux_buffer, act));
    check(hipMalloc(&attn_buffer, act));
    check(hipMalloc(&output_distr, InfEngineConfig::VOCAB_SIZE * sizeof(float)));
    check(hipMalloc(&output_token, sizeof(int)));
    check(hipMalloc(&workspace, ws));
    check(hipMalloc(&kv_cache, kv_cache_size()));
    workspace_bytes = ws;
  }

  void release() {
    for (void* p : {(void*)tokenid_buff, (void*)data_buffer, (void*)aux_buffer,
                    (void*)attn_buffer, (void*)output_distr, (void*)output_token, workspace,
                    kv_cache})
      if (p) (void)hipFree(p);
    tokenid_buff = nullptr;
    data_buffer = aux_buffer = attn_buffer = nullptr;
    output_distr = nullptr;
    output_token = nullptr;
    workspace = kv_cache = nullptr;
    workspace_bytes = 0;
  }

  ModelWeights model_weights;
  IEHandle handle = nullptr;
  int* tokenid_buff = nullptr;
  bf16 *data_buffer = nullptr, *aux_buffer = nullptr, *attn_buffer = nullptr;
  float* output_distr = nullptr;
  int* output_token = nullptr;
  void* workspace = nullptr;
  void* kv_cache = nullptr;
  size_t workspace_bytes = 0;
  Timing timing;
};
