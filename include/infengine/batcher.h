// Continuous batching over the paged KV cache: requests join and leave between decode steps.
// The reference serves one request at a time (manager.cpp:31-110) and keeps a per-request
// RequestContext it never uses (manager.h:19-24); this driver is the continuous form of that
// loop.  Each admitted request is prefilled alone, straight into its pages
// (ie_prefill_paged_chunk, 8192 prompt tokens per call), then decoded together with every other
// running request, up to 16 per ie_decode_step_batched_paged call; a request may span up to
// IE_MAX_LONG_CONTEXT positions.  Pages (64
// positions of all layers, 8 MiB) come from a fixed pool; a request reserves the pages its
// whole lifetime needs when it is admitted, so a running request never waits for memory, and
// returns them when it finishes (max_new_tokens or eos_token).  Every row of the batched step
// is computed independently of the others, so a request's tokens do not depend on which
// requests share its steps (up to 2048 positions of context in the batch).
// Uses the HIP runtime API for buffers; synchronous on the device.
#pragma once
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <deque>
#include <stdexcept>
#include <vector>

#include "engine.h"

class ContinuousBatcher {
 public:
  static constexpr int kMaxBatch = 16;
  static constexpr int kPagePos = 64;
  // a request may span the paged path's whole context; prompts are prefilled in chunks of the
  // reference context length, so the prefill buffers stay that size
  static constexpr int kMaxPositions = IE_MAX_LONG_CONTEXT;
  static constexpr int kTableStride = kMaxPositions / kPagePos;
  static constexpr int kPrefillChunk = InfEngineConfig::MAX_CONTEXT_LENGTH;

  // n_pages: size of the page pool (ie_kv_page_size() bytes each).
  ContinuousBatcher(IEHandle handle, const ModelWeights& weights, int n_pages)
      : handle_(handle), weights_(weights), n_pages_(n_pages) {
    if (n_pages < 1) throw std::invalid_argument("ContinuousBatcher: n_pages < 1");
    check(hipMalloc(&pool_, (size_t)n_pages * ie_kv_page_size()));
    check(hipMalloc(&d_table_, sizeof(int) * kMaxBatch * kTableStride));
    check(hipMalloc(&d_tokens_, sizeof(int) * kMaxBatch * kMaxPositions));
    check(hipMalloc(&d_data_, sizeof(bf16) * kMaxBatch * InfEngineConfig::HIDDEN_SIZE));
    check(hipMalloc(&d_attn_, sizeof(bf16) * kMaxBatch * InfEngineConfig::HIDDEN_SIZE));
    check(hipMalloc(&d_logits_, sizeof(float) * kMaxBatch * InfEngineConfig::VOCAB_SIZE));
    check(hipMalloc(&d_out_, sizeof(int) * kMaxBatch));
    check(hipMalloc(&d_ws_, ie_batch_workspace_size(kMaxBatch)));
    for (int p = n_pages - 1; p >= 0; --p) free_pages_.push_back(p);
  }
  ~ContinuousBatcher() {
    for (void* p : {pool_, (void*)d_table_, (void*)d_tokens_, (void*)d_data_, (void*)d_attn_,
                    (void*)d_logits_, (void*)d_out_, d_ws_, (void*)p_tokens_, (void*)p_data_,
                    (void*)p_aux_, (void*)p_attn_, (void*)p_logits_, (void*)p_out_, p_ws_})
      if (p) (void)hipFree(p);
  }
  ContinuousBatcher(const ContinuousBatcher&) = delete;
  ContinuousBatcher& operator=(const ContinuousBatcher&) = delete;

  // Queues a request; returns its id.
  int submit(const std::vector<int>& prompt, int max_new_tokens, int eos_token = -1) {
    if (prompt.empty() || max_new_tokens < 1)
      throw std::invalid_argument("submit: empty prompt or max_new_tokens < 1");
    if ((int)prompt.size() + max_new_tokens > kMaxPositions)
      throw std::invalid_argument("submit: request exceeds the paged KV cache's positions");
    if (pages_for(prompt, max_new_tokens) > n_pages_)
      throw std::invalid_argument("submit: request needs more pages than the pool holds");
    reqs_.push_back(Req{prompt, (int)prompt.size(), max_new_tokens, eos_token, {}, false});
    waiting_.push_back((int)reqs_.size() - 1);
    return (int)reqs_.size() - 1;
  }

  // Admits waiting requests (in order) while rows and pages allow, then runs one batched decode
  // step over the running requests.  Returns false once nothing is waiting or running.
  bool step() {
    while (!waiting_.empty() && (int)running_.size() < kMaxBatch) {
      Req& r = reqs_[waiting_.front()];
      if (pages_for(r.tokens, r.max_new) > (int)free_pages_.size()) break;
      const int id = waiting_.front();
      waiting_.pop_front();
      admit(id);
    }
    if (running_.empty()) return !waiting_.empty();
    const int B = (int)running_.size();
    std::vector<int> seq(B), table((size_t)B * kTableStride, -1);
    for (int b = 0; b < B; ++b) {
      const Req& r = reqs_[running_[b]];
      seq[b] = (int)r.tokens.size();  // the newest token sits at position seq - 1
      std::copy(r.pages.begin(), r.pages.end(), table.begin() + (size_t)b * kTableStride);
      check(hipMemcpy(d_tokens_ + (size_t)b * kMaxPositions + seq[b] - 1,
                      &r.tokens.back(), sizeof(int), hipMemcpyHostToDevice));
    }
    check(hipMemcpy(d_table_, table.data(), table.size() * sizeof(int), hipMemcpyHostToDevice));
    std::vector<int> out(B);
    infengine_detail::checked(ie_decode_step_batched_paged(
        handle_, &weights_, B, seq.data(), d_tokens_, kMaxPositions, d_data_, d_attn_, d_logits_,
        d_out_,
        out.data(), d_ws_, pool_, n_pages_, d_table_, kTableStride));
    std::vector<int> still;
    for (int b = 0; b < B; ++b) {
      Req& r = reqs_[running_[b]];
      r.tokens.push_back(out[b]);
      if (finished_now(r)) retire(r);
      else still.push_back(running_[b]);
    }
    running_ = still;
    return true;
  }

  void run() {
    while (step()) {
    }
  }

  bool finished(int id) const { return reqs_.at(id).done; }
  // prompt + generated ids
  const std::vector<int>& tokens(int id) const { return reqs_.at(id).tokens; }
  int free_pages() const { return (int)free_pages_.size(); }

 private:
  struct Req {
    std::vector<int> tokens;
    int prompt_len, max_new, eos;
    std::vector<int> pages;
    bool done;
  };

  static void check(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
  }
  // pages covering positions 0 .. prompt + max_new - 2 (the last token is never written)
  static int pages_for(const std::vector<int>& prompt, int max_new) {
    return ((int)prompt.size() + max_new - 1 + kPagePos - 1) / kPagePos;
  }
  bool finished_now(const Req& r) const {
    return (int)r.tokens.size() - r.prompt_len >= r.max_new || r.tokens.back() == r.eos;
  }
  void retire(Req& r) {
    r.done = true;
    for (int p : r.pages) free_pages_.push_back(p);
    r.pages.clear();
  }

  // Prefill alone, writing the prompt's K/V rows into the request's pages, kPrefillChunk tokens
  // per call.  If it throws, the request is back at the head of the queue with no pages and the
  // exception propagates.
  void admit(int id) {
    Req& r = reqs_[id];
    const int S = r.prompt_len;
    const int need = pages_for(r.tokens, r.max_new);
    for (int i = 0; i < need; ++i) {
      r.pages.push_back(free_pages_.back());
      free_pages_.pop_back();
    }
    int tok = -1;
    try {
      ensure_prefill_buffers(std::min(S, kPrefillChunk));
      check(hipMemcpy(p_tokens_, r.tokens.data(), S * sizeof(int), hipMemcpyHostToDevice));
      check(hipMemcpy(d_table_, r.pages.data(), r.pages.size() * sizeof(int),
                      hipMemcpyHostToDevice));
      for (int start = 0; start < S; start += kPrefillChunk)
        tok = infengine_detail::checked(ie_prefill_paged_chunk(
            handle_, &weights_, start, std::min(kPrefillChunk, S - start), p_tokens_, p_data_,
            p_aux_, p_attn_, p_logits_, p_out_, p_ws_, pool_, n_pages_, d_table_));
    } catch (...) {
      // the request goes back to the head of the queue and its pages back to the pool
      for (auto it = r.pages.rbegin(); it != r.pages.rend(); ++it) free_pages_.push_back(*it);
      r.pages.clear();
      waiting_.push_front(id);
      throw;
    }
    r.tokens.push_back(tok);
    if (finished_now(r)) retire(r);
    else running_.push_back(id);
  }

  // buffers for prefill calls of up to `rows` tokens
  void ensure_prefill_buffers(int rows) {
    const size_t ws = std::max(attn_workspace_size(rows), ffn_workspace_size(rows));
    if (p_ws_ && ws <= p_ws_bytes_) return;
    if (!p_tokens_) {
      const size_t act = (size_t)kPrefillChunk * InfEngineConfig::HIDDEN_SIZE * sizeof(bf16);
      check(hipMalloc(&p_tokens_, kMaxPositions * sizeof(int)));
      check(hipMalloc(&p_data_, act));
      check(hipMalloc(&p_aux_, act));
      check(hipMalloc(&p_attn_, act));
      check(hipMalloc(&p_logits_, InfEngineConfig::VOCAB_SIZE * sizeof(float)));
      check(hipMalloc(&p_out_, sizeof(int)));
    }
    if (p_ws_) check(hipFree(p_ws_));
    check(hipMalloc(&p_ws_, ws));
    p_ws_bytes_ = ws;
  }

  IEHandle handle_;
  const ModelWeights& weights_;
  int n_pages_;
  std::vector<Req> reqs_;
  std::deque<int> waiting_;
  std::vector<int> running_;
  std::vector<int> free_pages_;
  // batched step
  void* pool_ = nullptr;
  int* d_table_ = nullptr;
  int* d_tokens_ = nullptr;
  bf16 *d_data_ = nullptr, *d_attn_ = nullptr;
  float* d_logits_ = nullptr;
  int* d_out_ = nullptr;
  void* d_ws_ = nullptr;
  // prefill (one request at a time)
  int* p_tokens_ = nullptr;
  bf16 *p_data_ = nullptr, *p_aux_ = nullptr, *p_attn_ = nullptr;
  float* p_logits_ = nullptr;
  int* p_out_ = nullptr;
  void* p_ws_ = nullptr;
  size_t p_ws_bytes_ = 0;
};
