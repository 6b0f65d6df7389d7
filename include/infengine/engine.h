// C++ spelling of the engine entry points and op launchers (reference:
// prefill.cuh:6-9, decode.cuh:6-9 and the kernels/<op>.cuh launchers), over the
// C-ABI of infengine.h.  cublasHandle_t becomes IEHandle (an ie_context*),
// half becomes bf16, logits are fp32.  Errors throw std::runtime_error with
// ie_last_error(); the reference's launchers reported none.
#pragma once
#include <stdexcept>

#include "../infengine.h"
#include "config.h"
#include "model_weights.h"

using IEHandle = ie_context*;

namespace infengine_detail {
inline int checked(int rc) {
  if (rc < 0) throw std::runtime_error(ie_last_error());
  return rc;
}
}  // namespace infengine_detail

// cublasCreate / cublasDestroy (manager.cpp:58-59,107).  stream = nullptr runs
// on the legacy default stream, like the reference.
inline IEHandle ie_create_handle(int device = 0, void* stream = nullptr) {
  IEHandle h = nullptr;
  infengine_detail::checked(ie_context_create(&h, device, stream));
  return h;
}
inline void ie_destroy_handle(IEHandle h) { ie_context_destroy(h); }

// ---- engine (prefill.cuh:6-9, decode.cuh:6-9) ----
inline int prefill(IEHandle handle, const ModelWeights& weights, int seq_len, int* tokenid_buff,
                   bf16* data_buffer, bf16* aux_buffer, bf16* attn_buffer, float* output_distr,
                   int* output_token, void* workspace, void* kv_cache) {
  return infengine_detail::checked(ie_prefill(handle, &weights, seq_len, tokenid_buff, data_buffer,
                                              aux_buffer, attn_buffer, output_distr, output_token,
                                              workspace, kv_cache));
}

inline int decode_step(IEHandle handle, const ModelWeights& weights, int seq_len,
                       int* tokenid_buff, bf16* data_buffer, bf16* aux_buffer, bf16* attn_buffer,
                       float* output_distr, int* output_token, void* workspace, void* kv_cache) {
  return infengine_detail::checked(ie_decode_step(handle, &weights, seq_len, tokenid_buff,
                                                  data_buffer, aux_buffer, attn_buffer,
                                                  output_distr, output_token, workspace,
                                                  kv_cache));
}

// ---- sizing (attn.cu:295-307, ffn.cu:35-37) ----
inline size_t attn_workspace_size(int max_seq_len) { return ie_attn_workspace_size(max_seq_len); }
inline size_t ffn_workspace_size(int max_seq_len) { return ie_ffn_workspace_size(max_seq_len); }
inline size_t kv_cache_size() { return ie_kv_cache_size(); }

// ---- op launchers (legacy default stream, as in the reference) ----
inline void emblookup(int seq_len, int* d_input, bf16* d_weights, bf16* d_output) {
  infengine_detail::checked(ie_emblookup(seq_len, d_input, d_weights, d_output, nullptr));
}
inline void rmsnorm(int seq_len, bf16* d_input, bf16* d_weight, bf16* d_output) {
  infengine_detail::checked(ie_rmsnorm(seq_len, d_input, d_weight, d_output, nullptr));
}
inline void residual_add(int rows, int cols, bf16* d_x, bf16* d_delta) {
  infengine_detail::checked(ie_residual_add(rows, cols, d_x, d_delta, nullptr));
}
inline void swiglu(int seq_len, bf16* d_gate, bf16* d_up, bf16* d_output) {
  infengine_detail::checked(ie_swiglu(seq_len, d_gate, d_up, d_output, nullptr));
}
inline void apply_rope(int start_pos, int num_heads, int seq_len, const float* d_rope_cos,
                       const float* d_rope_sin, bf16* d_input, bf16* d_output, bool is_kv_cache) {
  infengine_detail::checked(ie_apply_rope(start_pos, num_heads, seq_len, d_rope_cos, d_rope_sin,
                                          d_input, d_output, is_kv_cache ? 1 : 0, nullptr));
}
inline void scale_causal_softmax(int seq_len, bf16* d_input, bf16* d_output, bool is_row) {
  infengine_detail::checked(ie_scale_causal_softmax(seq_len, d_input, d_output, is_row ? 1 : 0,
                                                    nullptr));
}
inline void init_rope_buffer(float** cu_rope_cos, float** cu_rope_sin) {
  infengine_detail::checked(ie_init_rope_buffer(cu_rope_cos, cu_rope_sin));
}
inline void cleanup_rope_buffer(float* cu_rope_cos, float* cu_rope_sin) {
  infengine_detail::checked(ie_cleanup_rope_buffer(cu_rope_cos, cu_rope_sin));
}
inline void multiply_by_weight(IEHandle handle, int m, int k, int n, const bf16* d_in,
                               const bf16* d_w, bf16* d_out) {
  infengine_detail::checked(ie_multiply_by_weight(handle, m, k, n, d_in, d_w, d_out));
}
inline void ffn(IEHandle handle, int seq_len, bf16* d_in, bf16* d_out, bf16* d_wup,
                bf16* d_wdown, bf16* d_wgate, void* workspace) {
  infengine_detail::checked(ie_ffn(handle, seq_len, d_in, d_out, d_wup, d_wdown, d_wgate,
                                   workspace));
}
inline void attn(IEHandle handle, const float* d_rope_cos, const float* d_rope_sin, int seq_len,
                 bf16* d_input, bf16* d_qproj, bf16* d_kproj, bf16* d_vproj, bf16* d_oproj,
                 bf16* d_output, void* workspace, void* kv_cache, int layer_idx) {
  infengine_detail::checked(ie_attn(handle, d_rope_cos, d_rope_sin, seq_len, d_input, d_qproj,
                                    d_kproj, d_vproj, d_oproj, d_output, workspace, kv_cache,
                                    layer_idx));
}
inline void decode_attn(IEHandle handle, const float* d_rope_cos, const float* d_rope_sin,
                        int seq_len, bf16* d_input, bf16* d_qproj, bf16* d_kproj, bf16* d_vproj,
                        bf16* d_oproj, bf16* d_output, void* workspace, void* kv_cache,
                        int layer_idx) {
  infengine_detail::checked(ie_decode_attn(handle, d_rope_cos, d_rope_sin, seq_len, d_input,
                                           d_qproj, d_kproj, d_vproj, d_oproj, d_output,
                                           workspace, kv_cache, layer_idx));
}
inline void lm_head(IEHandle handle, int seq_len, bf16* d_input, bf16* d_weight,
                    float* d_output) {
  infengine_detail::checked(ie_lm_head(handle, seq_len, d_input, d_weight, d_output));
}
inline void sample_token_amax(IEHandle handle, const float* d_logits, int* d_output) {
  infengine_detail::checked(ie_sample_token_amax(handle, d_logits, d_output));
}

namespace infengine_detail {
// The context behind the handle-free launchers: one per host thread, on the device current at
// its first use and on the legacy default stream (where the reference's launchers run),
// destroyed when the thread ends.
inline IEHandle thread_default_handle() {
  struct Holder {
    IEHandle h = nullptr;
    ~Holder() {
      if (h) ie_context_destroy(h);
    }
  };
  thread_local Holder holder;
  if (!holder.h) checked(ie_context_create(&holder.h, IE_CURRENT_DEVICE, nullptr));
  return holder.h;
}
}  // namespace infengine_detail

// sampling.cuh:4, the reference's own spelling: no handle (the argmax's reduction state lives in
// the calling thread's default context).  Asynchronous on the legacy default stream, like the
// reference's launcher; the caller's copy of *d_output orders after it.
inline void sample_token_amax(const float* d_logits, int* d_output) {
  infengine_detail::checked(
      ie_sample_token_amax(infengine_detail::thread_default_handle(), d_logits, d_output));
}
