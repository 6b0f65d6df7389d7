// Engine: context, workspace layout, the prefill / decode_step entry points and
// the extern "C" op launchers.
//
// Reference flow being replaced: decode_step (decode.cu:11-49) and prefill
// (prefill.cu:11-48), which launch ~19 kernels per layer on the legacy stream.
// decode_step here is 5 kernels per layer:
//   1. QKV GEMV  (RMSNorm prologue; RoPE + KV-cache write epilogue)
//   2. GQA decode attention (split context, last-block merge)
//   3. O GEMV    (residual-add epilogue into data_buffer)
//   4. gate/up GEMV (RMSNorm prologue; SwiGLU epilogue)
//   5. down GEMV (residual-add epilogue)
// then final-norm + lm_head GEMV (fp32 logits) and argmax.  The per-step scalar
// (seq_len) lives in device memory, so the whole step is captured once into a
// hipGraph and replayed.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <chrono>
#include <cstring>
#include <mutex>
#include <numbers>
#include <vector>

#include "ie_kernels.h"

struct ie_context : public ie::Context {};

namespace ie {

namespace {
thread_local char g_err[1024] = "";

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// ---- decode workspace: [q | h | attn1 | partials | xn | ss]
struct DecodeWs {
  uint16_t* q;      // [batch][4096]   rotated q
  uint16_t* h;      // [batch][14336]  SwiGLU output
  uint16_t* attn1;  // [batch][4096]   attention output (op-level decode_attn only)
  float* part_o;
  float* part_ml;
  uint16_t* xn;     // [batch][4096]   final-RMSNorm rows for the lm_head (batched path)
  float* ss;        // [256][16]       partial sums of squares of those rows (batched path)
  float* sk_part;   // the skinny GEMM's K-half partials (batched path)
};


size_t decode_ws_bytes(int batch) {
  return align256((size_t)batch * kHidden * 2) + align256((size_t)batch * kFFN * 2) +
         align256((size_t)batch * kHidden * 2) + align256(attn_decode_partials_bytes(batch)) +
         align256((size_t)batch * kHidden * 2) + align256((size_t)kNormParts * 16 * sizeof(float)) +
         align256(kSkPartBytes);
}

DecodeWs decode_ws(void* ws, int batch) {
  char* p = static_cast<char*>(ws);
  DecodeWs d;
  d.q = reinterpret_cast<uint16_t*>(p);
  p += align256((size_t)batch * kHidden * 2);
  d.h = reinterpret_cast<uint16_t*>(p);
  p += align256((size_t)batch * kFFN * 2);
  d.attn1 = reinterpret_cast<uint16_t*>(p);
  p += align256((size_t)batch * kHidden * 2);
  const size_t slots = (size_t)batch * kKVHeads * kAttnSplits * kGQA;
  d.part_o = reinterpret_cast<float*>(p);
  d.part_ml = d.part_o + slots * kHeadDim;
  p += align256(attn_decode_partials_bytes(batch));
  d.xn = reinterpret_cast<uint16_t*>(p);
  p += align256((size_t)batch * kHidden * 2);
  d.ss = reinterpret_cast<float*>(p);
  p += align256((size_t)kNormParts * 16 * sizeof(float));
  d.sk_part = reinterpret_cast<float*>(p);
  return d;
}

// ---- prefill workspace: [qkv / attention scratch | rotated q] (attention phase)
//                         [h]                                   (FFN phase)
size_t prefill_attn_bytes(int S) {
  return align256((size_t)S * kQKVDim * 2) + align256((size_t)S * kHidden * 2);
}
// [h (S x 14336 bf16) | split-K partials of the 4096-column projections (S <= kSplitMaxRows)];
// the O projection's partials reuse the start (q/k/v and rotated q are dead by then).
size_t prefill_split_bytes(int S) { return align256(gemm_split_bytes(std::min(S, kSplitMaxRows), kHidden)); }
size_t prefill_ffn_bytes(int S) { return align256((size_t)S * kFFN * 2) + prefill_split_bytes(S); }

uint16_t* kv_layer(void* kv, int layer) {
  return static_cast<uint16_t*>(kv) + (size_t)layer * kKVLayer;
}

// ---- decode building blocks -------------------------------------------------
int qkv_rope_gemv(const ie_layer& L, const ie_rope_weights& rope, const uint16_t* x,
                  const uint16_t* norm_w, uint16_t* q_out, uint16_t* kvl, const int* d_seq_len,
                  int pos, hipStream_t st) {
  GemvParams p{};
  p.x = x;
  p.norm_w = norm_w;
  p.w0 = L.transformer.w_q;
  p.w1 = L.transformer.w_k;
  p.w2 = L.transformer.w_v;
  p.out = q_out;
  p.k_cache = kvl;
  p.v_cache = kvl + (size_t)kKVHeads * kKVPlane;
  p.rope_cos = rope.cos;
  p.rope_sin = rope.sin;
  p.d_seq_len = d_seq_len;
  p.pos = pos;
  p.n_pairs = (kQHeads + 2 * kKVHeads) * 64;
  return launch_gemv(kHidden, kEpiQkvRope, norm_w != nullptr, p, 1, st);
}

// merge: also write the bf16 attention output to `out` (merge kernel); otherwise only the
// partials are written, for an O projection that merges them.  max_len: host-known bound on
// the context lengths; beyond kAttnFusedMaxCtx the splits go up to kAttnSplits (merge only).
// Paged KV (block_table set): kvl is the layer's base inside page 0, n_pages the pool size.
int attn_decode(const uint16_t* q, uint16_t* kvl, uint16_t* out, const DecodeWs& w,
                const int* d_seq_len, int seq_len, int max_len, int batch, long long cache_stride,
                bool merge, hipStream_t st, const int* block_table = nullptr, int table_stride = 0,
                int n_pages = 0, bool batched = false) {
  AttnDecodeParams a{};
  a.q = q;
  a.k_cache = kvl;
  a.v_cache = kvl + (size_t)kKVHeads * (block_table ? kPageHead : kKVPlane);
  a.cache_batch_stride = cache_stride;
  a.block_table = block_table;
  a.table_stride = table_stride;
  a.n_pages = n_pages;
  a.out = out;
  a.part_o = w.part_o;
  a.part_ml = w.part_ml;
  a.d_seq_len = d_seq_len;
  a.seq_len = seq_len;
  // batched step: 16 x 8 (sequence, kv head) workgroups already fill the chip, so up to
  // kAttnDirectMaxCtx one split per pair writes the output (no merge launch).  At every batch
  // size, so that a sequence's results do not depend on how many others share its step.
  a.max_splits = (batched && merge && max_len <= kAttnDirectMaxCtx) ? 1
                 : max_len <= kAttnFusedMaxCtx                        ? attn_fused_splits(max_len)
                                                                     : kAttnSplits;
  IE_REQUIRE(merge || a.max_splits <= kAttnFusedSplitsLong,
             "attn_decode: contexts past %d need the merge kernel", kAttnFusedMaxCtx);
  return launch_attn_decode(a, batch, merge, st);
}

int gemv_plain(int K, int epi, const uint16_t* x, const uint16_t* norm_w, const uint16_t* w0,
               const uint16_t* w1, int n_pairs, uint16_t* out, float* out_f32, int rows,
               long long out_stride, hipStream_t st) {
  GemvParams p{};
  p.x = x;
  p.norm_w = norm_w;
  p.w0 = w0;
  p.w1 = w1;
  p.out = out;
  p.out_f32 = out_f32;
  p.n_pairs = n_pairs;
  p.x_stride = K;
  p.out_stride = out_stride;
  return launch_gemv(K, epi, norm_w != nullptr, p, rows, st);
}

// True when the decode step merges the attention partials inside the O projection (no
// merge launch); the host-known context bound decides (graph capture keys on it).
bool attn_fused(int seq_len) { return seq_len <= kAttnFusedMaxCtx; }

// seq_len: the context length; with d_seq_len set the kernels read it from there and seq_len
// only bounds it on the host (it picks the attention path).
// The decode layer from its attention on (decode.cu:22-39): the row whose rotated q is at q
// attends over positions 0 .. seq_len-1 of the layer's cache kvl (paged: the layer's base in
// page 0, block_table the sequence's pages), then the O projection + residual into x and the
// FFN block.  w.q is not read (q is).
int decode_layer_tail(hipStream_t st, const ie_layer& L, const uint16_t* q, uint16_t* x,
                      uint16_t* attn_out, const DecodeWs& w, uint16_t* kvl, const int* d_seq_len,
                      int seq_len, const int* block_table = nullptr, int n_pages = 0) {
  const bool fused = attn_fused(seq_len);
  IE_TRY(attn_decode(q, kvl, attn_out, w, d_seq_len, seq_len, seq_len, 1, 0, !fused, st,
                     block_table, 0, n_pages));
  if (fused) {
    // O projection + residual, its input merged from the split partials in its prologue
    GemvParams p{};
    p.w0 = L.transformer.w_o;
    p.out = x;
    p.n_pairs = kHidden / 2;
    p.x_stride = kHidden;
    p.d_seq_len = d_seq_len;
    p.pos = seq_len;
    p.attn_part_o = w.part_o;
    p.attn_part_ml = w.part_ml;
    p.attn_max_splits = attn_fused_splits(seq_len);
    IE_TRY(launch_gemv(kHidden, kEpiResid, false, p, 1, st));
  } else {
    IE_TRY(gemv_plain(kHidden, kEpiResid, attn_out, nullptr, L.transformer.w_o, nullptr,
                      kHidden / 2, x, nullptr, 1, 0, st));
  }
  IE_TRY(gemv_plain(kHidden, kEpiSwiglu, x, L.post_attention_layernorm, L.ffn_block.w_gate,
                    L.ffn_block.w_up, kFFN, w.h, nullptr, 1, 0, st));
  IE_TRY(gemv_plain(kFFN, kEpiResid, w.h, nullptr, L.ffn_block.w_down, nullptr, kHidden / 2, x,
                    nullptr, 1, 0, st));
  return IE_OK;
}

int decoder_layer_decode(Context* c, hipStream_t st, const ie_model_weights& W, int layer,
                         uint16_t* x, uint16_t* attn_out, const DecodeWs& w, void* kv,
                         const int* d_seq_len, int seq_len) {
  (void)c;
  const ie_layer& L = W.layers[layer];
  uint16_t* kvl = kv_layer(kv, layer);
  IE_TRY(qkv_rope_gemv(L, W.rope, x, L.input_layernorm, w.q, kvl, d_seq_len, seq_len - 1, st));
  return decode_layer_tail(st, L, w.q, x, attn_out, w, kvl, d_seq_len, seq_len);
}

// wb_buf: when set, the argmax also stores the token at wb_buf[seq_len] (the Manager loop's
// write-back, manager.cpp:84).  The argmax always advances d_params[0] and hands the token to
// the host through mapped memory.
int enqueue_decode(Context* c, hipStream_t st, const ie_model_weights& W, int seq_len,
                   int* tokenid_buff, uint16_t* data, uint16_t* attn, float* logits, int* out_tok,
                   void* ws, void* kv, int* wb_buf) {
  const int* d_sl = c->d_params;
  const DecodeWs w = decode_ws(ws, 1);
  IE_TRY(launch_emblookup(1, tokenid_buff, W.emb_lookup, data, d_sl, 0, st));
  for (int l = 0; l < kLayers; ++l)
    IE_TRY(decoder_layer_decode(c, st, W, l, data, attn, w, kv, d_sl, seq_len));
  IE_TRY(gemv_plain(kHidden, kEpiF32, data, W.final_norm, W.lm_head, nullptr, kVocab / 2,
                    nullptr, logits, 1, kVocab, st));
  ArgmaxTail tail;
  tail.host_tok = c->h_token_dev;
  tail.tok_buf = wb_buf;
  tail.seq = c->d_params;
  IE_TRY(launch_argmax_rows(1, kVocab, logits, out_tok, c->d_slots, c->d_counters + kCntArgmax,
                            st, tail));
  return IE_OK;
}

// Rows of the weights' RoPE tables (0: the reference's 8192).
int rope_rows(const ie_model_weights& W) { return W.rope_rows > 0 ? W.rope_rows : kMaxCtx; }

bool weights_complete(const ie_model_weights& W) {
  if (!W.emb_lookup || !W.final_norm || !W.lm_head || !W.rope.cos || !W.rope.sin) return false;
  for (int l = 0; l < kLayers; ++l) {
    const ie_layer& L = W.layers[l];
    if (!L.input_layernorm || !L.post_attention_layernorm || !L.transformer.w_q ||
        !L.transformer.w_k || !L.transformer.w_v || !L.transformer.w_o || !L.ffn_block.w_up ||
        !L.ffn_block.w_gate || !L.ffn_block.w_down)
      return false;
  }
  return true;
}

// FNV-1a over the bytes of the weight table (graph cache key).
uint64_t hash_bytes(const void* p, size_t n, uint64_t h = 1469598103934665603ull) {
  const unsigned char* b = static_cast<const unsigned char*>(p);
  for (size_t i = 0; i < n; ++i) h = (h ^ b[i]) * 1099511628211ull;
  return h;
}

int set_device(Context* c) {
  IE_CHECK_HIP(hipSetDevice(c->device));
  return IE_OK;
}

// ---- RoPE tables: rope.cu:68-96 (Llama-3 frequency scaling, theta 500000)
void rope_tables_host(std::vector<float>& cos_t, std::vector<float>& sin_t) {
  const float theta = 500000.0f;
  const int factor = 8, low_ff = 1, high_ff = 4, orig = 8192;
  const int low_wl = orig / low_ff, high_wl = orig / high_ff;
  float freqs[kHeadDim / 2];
  for (int i = 0; i < kHeadDim / 2; ++i) {
    const float freq = 1 / std::pow(theta, 2.0 * i / kHeadDim);
    const float wavelength = 2 * std::numbers::pi / freq;
    if (wavelength > low_wl) {
      freqs[i] = freq / factor;
    } else if (wavelength < high_wl) {
      freqs[i] = freq;
    } else {
      const float smooth = (orig / wavelength - low_ff) / (high_ff - low_ff);
      freqs[i] = (1 - smooth) * (freq / factor) + smooth * freq;
    }
  }
  // rows 0..8191 are the reference's table; the same formula continues to kMaxLongCtx
  cos_t.resize((size_t)kMaxLongCtx * 64);
  sin_t.resize((size_t)kMaxLongCtx * 64);
  for (int pos = 0; pos < kMaxLongCtx; ++pos)
    for (int i = 0; i < 64; ++i) {
      const float angle = pos * freqs[i];
      cos_t[(size_t)pos * 64 + i] = std::cos(angle);
      sin_t[(size_t)pos * 64 + i] = std::sin(angle);
    }
}

}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}
const char* get_error() { return g_err; }

}  // namespace ie

using namespace ie;

#define CTX_OK(ctx)                                                   \
  do {                                                                \
    IE_REQUIRE((ctx) != nullptr, "%s: null context", __func__);       \
    IE_TRY(set_device(ctx));                                          \
  } while (0)

extern "C" {

const char* ie_last_error(void) { return get_error(); }

int ie_context_create(ie_context** out, int device, void* stream) {
  IE_REQUIRE(out != nullptr, "ie_context_create: out is null");
  *out = nullptr;
  int n = 0;
  IE_CHECK_HIP(hipGetDeviceCount(&n));
  if (device == IE_CURRENT_DEVICE) IE_CHECK_HIP(hipGetDevice(&device));
  IE_REQUIRE(device >= 0 && device < n, "ie_context_create: device %d of %d", device, n);
  IE_CHECK_HIP(hipSetDevice(device));
  ie_context* c = new ie_context;
  c->device = device;
  int rc = IE_OK;
  do {
    c->stream = stream_of(stream);
    if (hipStreamCreateWithFlags(&c->capture, hipStreamNonBlocking) != hipSuccess) {
      rc = IE_ERR_HIP;
      break;
    }
    if (hipMalloc(&c->d_counters, kNumCounters * sizeof(unsigned int)) != hipSuccess ||
        hipMalloc(&c->d_slots, kNumSlots * kSlotStride * sizeof(unsigned long long)) != hipSuccess ||
        hipMalloc(&c->d_params, 64 * sizeof(int)) != hipSuccess ||
        hipMalloc(&c->d_sk_part, kSkPartBytes) != hipSuccess ||
        hipHostMalloc(&c->h_params, 64 * sizeof(int), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(&c->h_token, 64 * sizeof(int), hipHostMallocMapped) != hipSuccess) {
      rc = IE_ERR_OOM;
      break;
    }
    if (hipHostGetDevicePointer(reinterpret_cast<void**>(&c->h_token_dev), c->h_token, 0) !=
        hipSuccess) {
      rc = IE_ERR_HIP;
      break;
    }
    // the no-allocation top-p sampler's scratch: resolve this device's address once
    if (top_p_scratch_init(device) != IE_OK) {
      rc = IE_ERR_HIP;
      break;
    }
    if (hipMemset(c->d_counters, 0, kNumCounters * sizeof(unsigned int)) != hipSuccess ||
        hipMemset(c->d_slots, 0, kNumSlots * kSlotStride * sizeof(unsigned long long)) != hipSuccess ||
        hipMemset(c->d_params, 0, 64 * sizeof(int)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
      rc = IE_ERR_HIP;
      break;
    }
  } while (0);
  if (rc != IE_OK) {
    set_error("ie_context_create: HIP allocation/initialisation failed");
    ie_context_destroy(c);
    return rc;
  }
  *out = c;
  return IE_OK;
}

int ie_context_destroy(ie_context* c) {
  if (!c) return IE_OK;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
  for (auto& bg : c->bgraph)
    if (bg.exec) (void)hipGraphExecDestroy(bg.exec);
  (void)hipFree(c->d_counters);
  (void)hipFree(c->d_slots);
  (void)hipFree(c->d_params);
  (void)hipFree(c->d_sk_part);
  if (c->h_params) (void)hipHostFree(c->h_params);
  if (c->h_token) (void)hipHostFree(c->h_token);
  if (c->capture) (void)hipStreamDestroy(c->capture);
  if (c->gemm_ws) (void)hipFree(c->gemm_ws);
  delete c;
  return IE_OK;
}

void* ie_context_stream(ie_context* c) { return c ? (void*)c->stream : nullptr; }

int ie_context_set_graph(ie_context* c, int enable) {
  IE_REQUIRE(c != nullptr, "ie_context_set_graph: null context");
  c->use_graph = enable != 0;
  return IE_OK;
}

size_t ie_attn_workspace_size(int max_seq_len) {
  const int S = max_seq_len < 1 ? 1 : max_seq_len;
  // q/k/v, rotated q, then split-K partials of the q/k/v projection (prompts of up to 512)
  const size_t a = decode_ws_bytes(1),
               b = prefill_attn_bytes(S) + align256(gemm_split_bytes(std::min(S, kSplitMaxRows), kQKVDim));
  return a > b ? a : b;
}

size_t ie_ffn_workspace_size(int max_seq_len) {
  const int S = max_seq_len < 1 ? 1 : max_seq_len;
  const size_t a = decode_ws_bytes(1), b = prefill_ffn_bytes(S);
  return a > b ? a : b;
}

size_t ie_kv_cache_size(void) { return (size_t)kLayers * kKVLayer * sizeof(uint16_t); }

size_t ie_batch_workspace_size(int batch) {
  return decode_ws_bytes(batch < 1 ? 1 : batch);
}

// ---------------------------------------------------------------- decode_step
}  // extern "C"

namespace ie {
namespace {

// One decode step (decode.cuh:6-9).  d_params[0] (the position the kernels read) is copied
// from the host only when it differs from what the previous step's argmax advanced it to; the
// token reaches the host through mapped memory written by the argmax, so a step costs one
// graph launch and one stream synchronisation.  wb = true also writes the token back to
// tokenid_buff[seq_len] on the device (manager.cpp:84).
int decode_step_impl(Context* c, const ie_model_weights* weights, int seq_len, int* tokenid_buff,
                     ie_bf16* data_buffer, ie_bf16* attn_buffer, float* output_distr,
                     int* output_token, void* workspace, void* kv_cache, bool wb,
                     bool poll = false) {
  IE_REQUIRE(weights && weights_complete(*weights), "decode_step: incomplete weights");
  IE_REQUIRE(seq_len >= 1 && seq_len <= kMaxCtx, "decode_step: seq_len %d out of [1, %d]",
             seq_len, kMaxCtx);
  IE_REQUIRE(!wb || seq_len < kMaxCtx, "decode_step: no slot after position %d", seq_len - 1);
  IE_REQUIRE(tokenid_buff && data_buffer && attn_buffer && output_distr && output_token &&
                 workspace && kv_cache,
             "decode_step: null buffer");
  hipStream_t st = c->stream;
  const bool copy = seq_len != c->next_seq;
  c->next_seq = -1;  // unknown until this step is enqueued
  if (copy) {
    c->h_params[0] = seq_len;
    IE_CHECK_HIP(hipMemcpyAsync(c->d_params, c->h_params, sizeof(int), hipMemcpyHostToDevice, st));
  }
  int* wb_buf = wb ? tokenid_buff : nullptr;
  volatile int* htok = static_cast<volatile int*>(c->h_token);
  *htok = -1;  // token ids are >= 0: -1 = not yet written by this step's argmax

  if (c->use_graph) {
    const void* key[12] = {(const void*)weights, tokenid_buff, data_buffer, attn_buffer,
                           output_distr, output_token, workspace, kv_cache,
                           (const void*)(uintptr_t)hash_bytes(weights, sizeof(*weights)),
                           // the captured attention path and split cap depend on the context
                           // length
                           (const void*)(uintptr_t)(attn_fused(seq_len)
                                                        ? (seq_len <= kAttnFusedShortCtx ? 1 : 3)
                                                        : 2),
                           wb_buf,
                           nullptr};
    if (!c->graph_exec || std::memcmp(key, c->graph_key, sizeof key) != 0) {
      if (c->graph_exec) {
        IE_CHECK_HIP(hipGraphExecDestroy(c->graph_exec));
        c->graph_exec = nullptr;
      }
      // captured on the private stream (capture is not allowed on the legacy
      // default stream), replayed on the context's stream
      hipGraph_t g = nullptr;
      IE_CHECK_HIP(hipStreamBeginCapture(c->capture, hipStreamCaptureModeThreadLocal));
      const int rc = enqueue_decode(c, c->capture, *weights, seq_len, tokenid_buff, data_buffer,
                                    attn_buffer, output_distr, output_token, workspace, kv_cache,
                                    wb_buf);
      const hipError_t ec = hipStreamEndCapture(c->capture, &g);
      if (rc != IE_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
      }
      IE_CHECK_HIP(ec);
      const hipError_t ei = hipGraphInstantiate(&c->graph_exec, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      IE_CHECK_HIP(ei);
      std::memcpy(c->graph_key, key, sizeof key);
    }
    IE_CHECK_HIP(hipGraphLaunch(c->graph_exec, st));
  } else {
    IE_TRY(enqueue_decode(c, st, *weights, seq_len, tokenid_buff, data_buffer, attn_buffer,
                          output_distr, output_token, workspace, kv_cache, wb_buf));
  }
  if (poll) {
    // The argmax stores the token to mapped host memory as the step's last action; the next
    // step is ordered after this one on the stream, so the caller of this loop only needs the
    // token.  Bounded: past ~2 s fall back to a stream synchronisation.
    const auto t0 = std::chrono::steady_clock::now();
    while (*htok < 0) {
      if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2)) {
        IE_CHECK_HIP(hipStreamSynchronize(st));
        break;
      }
    }
  } else {
    IE_CHECK_HIP(hipStreamSynchronize(st));
  }
  c->next_seq = seq_len + 1;
  return *htok;
}

}  // namespace
}  // namespace ie

extern "C" {

int ie_decode_step(ie_context* c, const ie_model_weights* weights, int seq_len,
                   int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                   ie_bf16* attn_buffer, float* output_distr, int* output_token,
                   void* workspace, void* kv_cache) {
  (void)aux_buffer;  // normalised activations never leave the GEMV prologues
  CTX_OK(c);
  return decode_step_impl(c, weights, seq_len, tokenid_buff, data_buffer, attn_buffer,
                          output_distr, output_token, workspace, kv_cache, false);
}

// Manager::handle_request's generation loop (manager.cpp:60-86) without the tokenizer: the
// prompt ids go to the device, one prefill, then decode steps, each token written back to
// tokenid_buff on the device before the next step reads it.  out_tokens[0] is the prefill's
// token, out_tokens[i] the i-th decode step's.  The loop ends after max_new_tokens tokens or
// right after a token equal to eos_token (>= 0; negative: no EOS), which is kept in out_tokens.
// timed_ms (optional) receives the host wall time of decode steps timed_from .. the last one
// (after a stream synchronisation; 0 when none ran).  Returns the number of tokens produced.
int ie_generate(ie_context* c, const ie_model_weights* weights, const int* prompt, int prompt_len,
                int max_new_tokens, int eos_token, int timed_from, int* out_tokens,
                int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                ie_bf16* attn_buffer, float* output_distr, int* output_token, void* workspace,
                void* kv_cache, double* timed_ms) {
  CTX_OK(c);
  IE_REQUIRE(prompt && out_tokens, "generate: null prompt / output");
  IE_REQUIRE(prompt_len >= 1 && max_new_tokens >= 1 && prompt_len + max_new_tokens <= kMaxCtx,
             "generate: prompt %d + %d new tokens exceed the context %d", prompt_len,
             max_new_tokens, kMaxCtx);
  if (timed_ms) *timed_ms = 0.0;
  IE_CHECK_HIP(hipMemcpyAsync(tokenid_buff, prompt, prompt_len * sizeof(int),
                              hipMemcpyHostToDevice, c->stream));
  const int first = ie_prefill(c, weights, prompt_len, tokenid_buff, data_buffer, aux_buffer,
                               attn_buffer, output_distr, output_token, workspace, kv_cache);
  if (first < 0) return first;
  out_tokens[0] = first;
  if (first == eos_token) return 1;
  IE_CHECK_HIP(hipMemcpyAsync(tokenid_buff + prompt_len, output_token, sizeof(int),
                              hipMemcpyDeviceToDevice, c->stream));
  auto t0 = std::chrono::steady_clock::now();
  bool timing = false;
  int n = 1;
  while (n < max_new_tokens) {
    if (n == timed_from) {
      IE_CHECK_HIP(hipStreamSynchronize(c->stream));
      t0 = std::chrono::steady_clock::now();
      timing = true;
    }
    const int tok = decode_step_impl(c, weights, prompt_len + n, tokenid_buff, data_buffer,
                                     attn_buffer, output_distr, output_token, workspace, kv_cache,
                                     true, true);
    if (tok < 0) return tok;
    out_tokens[n++] = tok;
    if (tok == eos_token) break;
  }
  IE_CHECK_HIP(hipStreamSynchronize(c->stream));
  if (timed_ms && timing)
    *timed_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                    .count();
  return n;
}

// ---------------------------------------------------------------- prefill
namespace {
// One decoder layer of the prefill (prefill.cu:17-38's loop body) over the S rows of
// data_buffer at positions start_pos.., in place: RMSNorm, the Q/K/V product, RoPE and the K/V
// write-out, causal attention, the O product + residual, RMSNorm, gate/up + SwiGLU, down +
// residual.  The workspace holds q/k/v and the rotated q, then h.
// K halves of a skinny (M <= 16) product's tiles (gemm_skinny_split): partials in `part`
// (kSkPartBytes), the context's arrival counters.
void skinny_split(Context* c, int epi, GemmParams& g, float* part) {
  if (g.M > 16) return;
  g.sk_tail = gemm_skinny_split(epi, g.N, g.K);
  g.sk_part = part;
  g.sk_cnt = c->d_counters + kCntSkinny;
}

// aux_ready: aux_buffer already holds this layer's input RMSNorm of data_buffer (written by
// the previous layer's down-projection reduction).  next_norm_w: the next layer's input norm
// weight, or nullptr; *aux_next is set when this layer left that norm in aux_buffer (the down
// projection ran with K split and its reduction applied the norm).
// last_row: the layer's K/V rows for all S positions, its output for the last row only (the
// rows before it keep the layer's input).  The final norm and lm_head of prefill.cu:41-43 read
// the last row alone and the later positions' attention reads only the K/V cache, so the last
// layer's attention, O projection and FFN over the other rows feed nothing: the last row runs
// them as a decode step does.
int prefill_layer(Context* c, hipStream_t st, const ie_model_weights& W, int l, int start_pos,
                  int S, ie_bf16* data_buffer, ie_bf16* aux_buffer, ie_bf16* attn_buffer,
                  void* workspace, void* kv_cache, const int* block_table, int n_pages,
                  bool aux_ready, const uint16_t* next_norm_w, bool* aux_next,
                  bool last_row = false) {
  if (aux_next) *aux_next = false;
  char* wsb = static_cast<char*>(workspace);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(wsb);
  uint16_t* qrot = reinterpret_cast<uint16_t*>(wsb + align256((size_t)S * kQKVDim * 2));
  uint16_t* h = reinterpret_cast<uint16_t*>(wsb);
  const ie_layer& L = W.layers[l];
  uint16_t* kvl = block_table ? static_cast<uint16_t*>(kv_cache) + (size_t)l * kPageLayer
                              : kv_layer(kv_cache, l);
  uint16_t* vpl = kvl + (size_t)kKVHeads * (block_table ? kPageHead : kKVPlane);
  if (!aux_ready) IE_TRY(launch_rmsnorm(S, data_buffer, L.input_layernorm, aux_buffer, st));
  GemmParams g{};
  g.x = aux_buffer;
  g.w0 = L.transformer.w_q;
  g.w1 = L.transformer.w_k;
  g.w2 = L.transformer.w_v;
  g.n0 = kHidden;
  g.n1 = kKVDim;
  g.y = qkv;
  g.M = S;
  g.N = kQKVDim;
  g.K = kHidden;
  g.ldy = kQKVDim;
  // split K's partials after q/k/v and the rotated q (the rest of the workspace)
  g.split_ws = reinterpret_cast<float*>(wsb + prefill_attn_bytes(S));
  g.split_ws_bytes = (long long)(ie_attn_workspace_size(S) - prefill_attn_bytes(S));
  // RoPE and the K/V scatter in the product's epilogue where the product runs on the 192 x 256
  // ping-pong tiles (long prompts), else the product to [S][6144] and the scatter kernel
  GemmParams f = g;
  f.y = qrot;
  f.ldy = kHidden;
  f.rope_cos = W.rope.cos;
  f.rope_sin = W.rope.sin;
  f.k_cache = kvl;
  f.v_cache = vpl;
  f.block_table = block_table;
  f.n_pages = n_pages;
  f.start_pos = start_pos;
  const int fused = launch_qkv_rope_prefill(f, st);
  if (fused < 0) return fused;
  if (fused != IE_OK) {
    skinny_split(c, kGemmBf16, g, c->d_sk_part);
    IE_TRY(launch_gemm(kGemmBf16, g, st));
    IE_TRY(launch_qkv_rope_scatter(S, start_pos, qkv, W.rope.cos, W.rope.sin, qrot, kvl, vpl,
                                   nullptr, 0, st, block_table, n_pages));
  }
  if (last_row) {
    // the decode workspace after q/k/v and the rotated q (the split-K partials' room)
    const size_t room = std::max(ie_attn_workspace_size(S), ie_ffn_workspace_size(S)) -
                        prefill_attn_bytes(S);
    IE_REQUIRE(decode_ws_bytes(1) <= room, "prefill: workspace too small for the last row");
    const DecodeWs dw = decode_ws(wsb + prefill_attn_bytes(S), 1);
    return decode_layer_tail(st, L, qrot + (size_t)(S - 1) * kHidden,
                             data_buffer + (size_t)(S - 1) * kHidden, dw.attn1, dw, kvl, nullptr,
                             start_pos + S, block_table, n_pages);
  }
  AttnPrefillParams a{qrot, kvl, vpl, attn_buffer, S, start_pos, block_table, n_pages};
  IE_TRY(launch_attn_prefill(a, st));
  GemmParams o{};
  o.x = attn_buffer;
  o.w0 = L.transformer.w_o;
  o.n0 = kHidden;
  o.y = data_buffer;
  o.M = S;
  o.N = kHidden;
  o.K = kHidden;
  o.ldy = kHidden;
  o.split_ws = reinterpret_cast<float*>(wsb);  // q/k/v and rotated q are dead
  o.split_ws_bytes = (long long)std::max(ie_attn_workspace_size(S), ie_ffn_workspace_size(S));
  skinny_split(c, kGemmResid, o, c->d_sk_part);
  // with K split the reduction applies the post-attention RMSNorm too
  int normed = 0;
  o.rn_w = L.post_attention_layernorm;
  o.rn_out = aux_buffer;
  o.rn_done = &normed;
  IE_TRY(launch_gemm(kGemmResid, o, st));
  if (!normed) IE_TRY(launch_rmsnorm(S, data_buffer, L.post_attention_layernorm, aux_buffer, st));
  GemmParams gu{};
  gu.x = aux_buffer;
  gu.w0 = L.ffn_block.w_gate;
  gu.w1 = L.ffn_block.w_up;
  gu.y = h;
  gu.M = S;
  gu.N = kFFN;
  gu.K = kHidden;
  gu.ldy = kFFN;
  gu.split_ws = reinterpret_cast<float*>(wsb + align256((size_t)S * kFFN * 2));  // after h
  gu.split_ws_bytes = (long long)(std::max(ie_attn_workspace_size(S), ie_ffn_workspace_size(S)) -
                                  align256((size_t)S * kFFN * 2));
  skinny_split(c, kGemmSwiglu, gu, c->d_sk_part);
  IE_TRY(launch_gemm(kGemmSwiglu, gu, st));
  GemmParams dn{};
  dn.x = h;
  dn.w0 = L.ffn_block.w_down;
  dn.n0 = kHidden;
  dn.y = data_buffer;
  dn.M = S;
  dn.N = kHidden;
  dn.K = kFFN;
  dn.ldy = kHidden;
  dn.split_ws = reinterpret_cast<float*>(wsb + align256((size_t)S * kFFN * 2));  // after h
  dn.split_ws_bytes = (long long)(std::max(ie_attn_workspace_size(S), ie_ffn_workspace_size(S)) -
                                  align256((size_t)S * kFFN * 2));
  skinny_split(c, kGemmResid, dn, c->d_sk_part);
  int next_normed = 0;
  if (next_norm_w) {
    dn.rn_w = next_norm_w;
    dn.rn_out = aux_buffer;
    dn.rn_done = &next_normed;
  }
  IE_TRY(launch_gemm(kGemmResid, dn, st));
  if (aux_next) *aux_next = next_normed != 0;
  return IE_OK;
}

// The prefill body over a reference-layout cache (block_table null) or over a page pool
// (kv_cache = n_pages pages, block_table the sequence's page per 64-position block).  The
// seq_len tokens sit at positions start_pos .. (tokenid_buff indexed by position); with pages,
// the K/V of positions before start_pos are already there (chunked prefill).
int prefill_impl(ie_context* c, const ie_model_weights* weights, int start_pos, int seq_len,
                 int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                 ie_bf16* attn_buffer, float* output_distr, int* output_token, void* workspace,
                 void* kv_cache, const int* block_table, int n_pages) {
  IE_REQUIRE(weights && weights_complete(*weights), "prefill: incomplete weights");
  const int cap = block_table ? kMaxLongCtx : kMaxCtx;
  IE_REQUIRE(start_pos >= 0 && (start_pos == 0 || block_table),
             "prefill: start_pos %d needs the paged cache", start_pos);
  IE_REQUIRE(seq_len >= 1 && start_pos + seq_len <= cap,
             "prefill: positions [%d, %d) out of [0, %d]", start_pos, start_pos + seq_len, cap);
  IE_REQUIRE(start_pos + seq_len <= rope_rows(*weights),
             "prefill: position %d past the weights' %d RoPE table rows (rope_rows)",
             start_pos + seq_len - 1, rope_rows(*weights));
  IE_REQUIRE(tokenid_buff && data_buffer && aux_buffer && attn_buffer && output_distr &&
                 output_token && workspace && kv_cache,
             "prefill: null buffer");
  const ie_model_weights& W = *weights;
  hipStream_t st = c->stream;
  const int S = seq_len;

  IE_TRY(launch_emblookup(S, tokenid_buff + start_pos, W.emb_lookup, data_buffer, nullptr, 0, st));
  bool aux_ready = false;
  for (int l = 0; l < kLayers; ++l)
    IE_TRY(prefill_layer(c, st, W, l, start_pos, S, data_buffer, aux_buffer, attn_buffer,
                         workspace, kv_cache, block_table, n_pages, aux_ready,
                         l + 1 < kLayers ? W.layers[l + 1].input_layernorm : nullptr, &aux_ready,
                         l == kLayers - 1));
  // prefill.cu:41-43: final norm, lm_head on the last row only, argmax
  IE_TRY(gemv_plain(kHidden, kEpiF32, data_buffer + (size_t)(S - 1) * kHidden, W.final_norm,
                    W.lm_head, nullptr, kVocab / 2, nullptr, output_distr, 1, kVocab, st));
  IE_TRY(launch_argmax_rows(1, kVocab, output_distr, output_token, c->d_slots,
                            c->d_counters + kCntArgmax, st));
  IE_CHECK_HIP(hipMemcpyAsync(c->h_token, output_token, sizeof(int), hipMemcpyDeviceToHost, st));
  IE_CHECK_HIP(hipStreamSynchronize(st));
  return c->h_token[0];
}
}  // namespace

int ie_prefill(ie_context* c, const ie_model_weights* weights, int seq_len, int* tokenid_buff,
               ie_bf16* data_buffer, ie_bf16* aux_buffer, ie_bf16* attn_buffer,
               float* output_distr, int* output_token, void* workspace, void* kv_cache) {
  CTX_OK(c);
  return prefill_impl(c, weights, 0, seq_len, tokenid_buff, data_buffer, aux_buffer, attn_buffer,
                      output_distr, output_token, workspace, kv_cache, nullptr, 0);
}

int ie_prefill_paged(ie_context* c, const ie_model_weights* weights, int seq_len,
                     int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                     ie_bf16* attn_buffer, float* output_distr, int* output_token,
                     void* workspace, void* kv_pages, int n_pages, const int* block_table) {
  CTX_OK(c);
  IE_REQUIRE(kv_pages && block_table && n_pages >= 1, "prefill_paged: needs a page pool and a block table");
  return prefill_impl(c, weights, 0, seq_len, tokenid_buff, data_buffer, aux_buffer, attn_buffer,
                      output_distr, output_token, workspace, kv_pages, block_table, n_pages);
}

int ie_prefill_paged_chunk(ie_context* c, const ie_model_weights* weights, int start_pos,
                           int n_tokens, int* tokenid_buff, ie_bf16* data_buffer,
                           ie_bf16* aux_buffer, ie_bf16* attn_buffer, float* output_distr,
                           int* output_token, void* workspace, void* kv_pages, int n_pages,
                           const int* block_table) {
  CTX_OK(c);
  IE_REQUIRE(kv_pages && block_table && n_pages >= 1,
             "prefill_paged_chunk: needs a page pool and a block table");
  return prefill_impl(c, weights, start_pos, n_tokens, tokenid_buff, data_buffer, aux_buffer,
                      attn_buffer, output_distr, output_token, workspace, kv_pages, block_table,
                      n_pages);
}

int ie_decoder_layer_prefill(ie_context* c, const ie_model_weights* weights, int layer_idx,
                             int seq_len, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                             ie_bf16* attn_buffer, void* workspace, void* kv_cache) {
  CTX_OK(c);
  IE_REQUIRE(weights && weights_complete(*weights), "decoder_layer_prefill: incomplete weights");
  IE_REQUIRE(layer_idx >= 0 && layer_idx < kLayers, "decoder_layer_prefill: layer %d", layer_idx);
  IE_REQUIRE(seq_len >= 1 && seq_len <= kMaxCtx, "decoder_layer_prefill: seq_len %d out of [1, %d]",
             seq_len, kMaxCtx);
  IE_REQUIRE(data_buffer && aux_buffer && attn_buffer && workspace && kv_cache,
             "decoder_layer_prefill: null buffer");
  return prefill_layer(c, c->stream, *weights, layer_idx, 0, seq_len, data_buffer, aux_buffer,
                       attn_buffer, workspace, kv_cache, nullptr, 0, false, nullptr, nullptr);
}

int ie_decoder_layer_prefill_last_row(ie_context* c, const ie_model_weights* weights,
                                      int layer_idx, int seq_len, ie_bf16* data_buffer,
                                      ie_bf16* aux_buffer, ie_bf16* attn_buffer, void* workspace,
                                      void* kv_cache) {
  CTX_OK(c);
  IE_REQUIRE(weights && weights_complete(*weights),
             "decoder_layer_prefill_last_row: incomplete weights");
  IE_REQUIRE(layer_idx >= 0 && layer_idx < kLayers, "decoder_layer_prefill_last_row: layer %d",
             layer_idx);
  IE_REQUIRE(seq_len >= 1 && seq_len <= kMaxCtx,
             "decoder_layer_prefill_last_row: seq_len %d out of [1, %d]", seq_len, kMaxCtx);
  IE_REQUIRE(data_buffer && aux_buffer && attn_buffer && workspace && kv_cache,
             "decoder_layer_prefill_last_row: null buffer");
  return prefill_layer(c, c->stream, *weights, layer_idx, 0, seq_len, data_buffer, aux_buffer,
                       attn_buffer, workspace, kv_cache, nullptr, 0, false, nullptr, nullptr,
                       true);
}

// ---------------------------------------------------------------- batched decode
namespace {
// One decoder layer of the batched step over the batch rows of data_buffer (in place), the
// rows' partial sums of squares already in w.ss (from the previous layer's down projection or
// the prep kernel); with ss_next the down projection leaves those of its output rows there.
int batched_layer(Context* c, hipStream_t st, const ie_model_weights& W, int l, int batch,
                  int len_class, ie_bf16* data_buffer, ie_bf16* attn_buffer, const DecodeWs& w,
                  void* kv_caches, const int* block_table, int table_stride, int n_pages,
                  bool ss_next) {
  const int* d_sl = c->d_params + 1;
  const long long cstride = (long long)kLayers * kKVLayer;
  const ie_layer& L = W.layers[l];
  uint16_t* kvl = block_table ? static_cast<uint16_t*>(kv_caches) + (size_t)l * kPageLayer
                              : kv_layer(kv_caches, l);
  GemmParams g{};
  g.x = data_buffer;
  g.w0 = L.transformer.w_q;
  g.w1 = L.transformer.w_k;
  g.w2 = L.transformer.w_v;
  g.n0 = kHidden;
  g.n1 = kKVDim;
  g.y = w.q;  // q rotated; k rotated and v into each sequence's cache row
  g.M = batch;
  g.N = kQKVDim;
  g.K = kHidden;
  g.ldy = kQKVDim;
  g.rope_cos = W.rope.cos;
  g.rope_sin = W.rope.sin;
  g.k_cache = kvl;
  g.v_cache = kvl + (size_t)kKVHeads * (block_table ? kPageHead : kKVPlane);
  g.cache_stride = cstride;
  g.block_table = block_table;
  g.table_stride = table_stride;
  g.n_pages = n_pages;
  g.d_seq_len = d_sl;
  g.ss_in = w.ss;
  g.ss_parts = kNormParts;
  g.x_norm_w = L.input_layernorm;
  skinny_split(c, kGemmQkvRope, g, w.sk_part);
  IE_TRY(launch_gemm(kGemmQkvRope, g, st));
  IE_TRY(attn_decode(w.q, kvl, attn_buffer, w, d_sl, 0, len_class, batch, cstride, true, st,
                     block_table, table_stride, n_pages, true));
  GemmParams o{};
  o.x = attn_buffer;
  o.w0 = L.transformer.w_o;
  o.n0 = kHidden;
  o.y = data_buffer;
  o.M = batch;
  o.N = kHidden;
  o.K = kHidden;
  o.ldy = kHidden;
  o.ss_out = w.ss;
  skinny_split(c, kGemmResid, o, w.sk_part);
  IE_TRY(launch_gemm(kGemmResid, o, st));
  GemmParams gu{};
  gu.x = data_buffer;
  gu.w0 = L.ffn_block.w_gate;
  gu.w1 = L.ffn_block.w_up;
  gu.y = w.h;
  gu.M = batch;
  gu.N = kFFN;
  gu.K = kHidden;
  gu.ldy = kFFN;
  gu.ss_in = w.ss;
  gu.ss_parts = kNormParts;
  gu.x_norm_w = L.post_attention_layernorm;
  skinny_split(c, kGemmSwiglu, gu, w.sk_part);
  IE_TRY(launch_gemm(kGemmSwiglu, gu, st));
  GemmParams dn{};
  dn.x = w.h;
  dn.w0 = L.ffn_block.w_down;
  dn.n0 = kHidden;
  dn.y = data_buffer;
  dn.M = batch;
  dn.N = kHidden;
  dn.K = kFFN;
  dn.ldy = kHidden;
  if (ss_next) dn.ss_out = w.ss;
  skinny_split(c, kGemmResid, dn, w.sk_part);
  IE_TRY(launch_gemm(kGemmResid, dn, st));
  return IE_OK;
}

// The kernels of one batched step on stream st, the sequences' lengths already in
// d_params[1 .. batch].  len_class bounds the longest context and picks the attention path:
// kAttnDirectMaxCtx (one split per sequence and kv head, no merge launch), kAttnFusedMaxCtx or
// beyond (split contexts + the merge kernel).
int enqueue_batched(Context* c, hipStream_t st, const ie_model_weights& W, int batch,
                    int len_class, int* tokenid_buffs, int tokens_stride, ie_bf16* data_buffer,
                    ie_bf16* attn_buffer, float* output_distr, int* output_tokens,
                    void* workspace, void* kv_caches, const int* block_table, int table_stride,
                    int n_pages) {
  const int* d_sl = c->d_params + 1;
  const DecodeWs w = decode_ws(workspace, batch);
  IE_TRY(launch_emblookup(batch, tokenid_buffs, W.emb_lookup, data_buffer, d_sl, tokens_stride,
                          st));
  // RMSNorm inside the projections: the QKV and gate/up projections read the residual rows
  // with kNormParts partial sums of squares per row (layer 0: from this prep kernel; later:
  // from the residual epilogue of the O / down projection, the same partials bit for bit) and
  // normalise the rows on their way in, with rmsnorm.cu:61's two roundings
  IE_TRY(launch_rmsnorm_prep(batch, data_buffer, w.ss, st));
  for (int l = 0; l < kLayers; ++l)
    IE_TRY(batched_layer(c, st, W, l, batch, len_class, data_buffer, attn_buffer, w, kv_caches,
                         block_table, table_stride, n_pages, l + 1 < kLayers));
  // prefill.cu:41-43 / decode.cu:41: final RMSNorm of the rows, then the lm_head product
  IE_TRY(launch_rmsnorm(batch, data_buffer, W.final_norm, w.xn, st));
  GemmParams lm{};
  lm.x = w.xn;
  lm.w0 = W.lm_head;
  lm.n0 = kVocab;
  lm.yf = output_distr;
  lm.M = batch;
  lm.N = kVocab;
  lm.K = kHidden;
  lm.ldy = kVocab;
  skinny_split(c, kGemmF32, lm, w.sk_part);
  IE_TRY(launch_gemm(kGemmF32, lm, st));
  IE_TRY(launch_argmax_rows(batch, kVocab, output_distr, output_tokens, c->d_slots,
                            c->d_counters + kCntArgmax, st));
  return IE_OK;
}

// One batched step over per-sequence caches (block_table null: kv = batch caches in the
// reference layout, kv_cache_size() apart) or over a page pool (kv = n_pages pages,
// block_table [batch][table_stride] page ids).  With graphs on (the default) the kernels are
// replayed from a graph captured on first use of the same arguments.
int batched_step(ie_context* c, const ie_model_weights* weights, int batch, const int* seq_lens,
                 int* tokenid_buffs, int tokens_stride, ie_bf16* data_buffer,
                 ie_bf16* attn_buffer, float* output_distr, int* output_tokens, int* tokens_out,
                 void* workspace, void* kv_caches, const int* block_table, int table_stride,
                 int n_pages) {
  IE_REQUIRE(weights && weights_complete(*weights), "decode_step_batched: incomplete weights");
  IE_REQUIRE(batch >= 1 && batch <= 16, "decode_step_batched: batch %d out of [1, 16]", batch);
  IE_REQUIRE(seq_lens && tokenid_buffs && data_buffer && attn_buffer && output_distr &&
                 output_tokens && workspace && kv_caches,
             "decode_step_batched: null buffer");
  const int cap = block_table ? kMaxLongCtx : kMaxCtx;
  for (int b = 0; b < batch; ++b) {
    IE_REQUIRE(seq_lens[b] >= 1 && seq_lens[b] <= cap && seq_lens[b] <= tokens_stride,
               "decode_step_batched: seq_lens[%d]=%d out of [1, %d] (token rows of %d)", b,
               seq_lens[b], cap, tokens_stride);
    IE_REQUIRE(seq_lens[b] <= rope_rows(*weights),
               "decode_step_batched: seq_lens[%d]=%d past the weights' %d RoPE table rows "
               "(rope_rows)", b, seq_lens[b], rope_rows(*weights));
  }
  hipStream_t st = c->stream;
  int max_len = 1;
  for (int b = 0; b < batch; ++b) {
    c->h_params[1 + b] = seq_lens[b];
    max_len = std::max(max_len, seq_lens[b]);
  }
  IE_CHECK_HIP(hipMemcpyAsync(c->d_params + 1, c->h_params + 1, batch * sizeof(int),
                              hipMemcpyHostToDevice, st));
  const int len_class = max_len <= kAttnDirectMaxCtx  ? kAttnDirectMaxCtx
                        : max_len <= kAttnFusedMaxCtx ? kAttnFusedMaxCtx
                                                      : cap;
  if (c->use_graph) {
    // replayed from a graph captured with the same buffers, batch and attention path (the
    // lengths are read from d_params on the device)
    const void* key[16] = {(const void*)weights,
                           (const void*)(uintptr_t)hash_bytes(weights, sizeof(*weights)),
                           tokenid_buffs, (const void*)(intptr_t)tokens_stride, data_buffer,
                           attn_buffer, output_distr, output_tokens, workspace, kv_caches,
                           block_table, (const void*)(intptr_t)table_stride,
                           (const void*)(intptr_t)n_pages, (const void*)(intptr_t)batch,
                           (const void*)(intptr_t)len_class, nullptr};
    Context::BatchGraph* slot = nullptr;
    for (auto& bg : c->bgraph)
      if (bg.exec && std::memcmp(bg.key, key, sizeof key) == 0) slot = &bg;
    if (!slot) {
      slot = &c->bgraph[0];
      for (auto& bg : c->bgraph)
        if (!bg.exec || bg.used < slot->used) slot = &bg;
      if (slot->exec) {
        IE_CHECK_HIP(hipGraphExecDestroy(slot->exec));
        slot->exec = nullptr;
      }
      hipGraph_t g = nullptr;
      IE_CHECK_HIP(hipStreamBeginCapture(c->capture, hipStreamCaptureModeThreadLocal));
      const int rc = enqueue_batched(c, c->capture, *weights, batch, len_class, tokenid_buffs,
                                     tokens_stride, data_buffer, attn_buffer, output_distr,
                                     output_tokens, workspace, kv_caches, block_table,
                                     table_stride, n_pages);
      const hipError_t ec = hipStreamEndCapture(c->capture, &g);
      if (rc != IE_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
      }
      IE_CHECK_HIP(ec);
      const hipError_t ei = hipGraphInstantiate(&slot->exec, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      IE_CHECK_HIP(ei);
      std::memcpy(slot->key, key, sizeof key);
    }
    slot->used = ++c->bgraph_tick;
    IE_CHECK_HIP(hipGraphLaunch(slot->exec, st));
  } else {
    IE_TRY(enqueue_batched(c, st, *weights, batch, len_class, tokenid_buffs, tokens_stride,
                           data_buffer, attn_buffer, output_distr, output_tokens, workspace,
                           kv_caches, block_table, table_stride, n_pages));
  }
  if (tokens_out) {
    IE_CHECK_HIP(hipMemcpyAsync(c->h_token, output_tokens, batch * sizeof(int),
                                hipMemcpyDeviceToHost, st));
    IE_CHECK_HIP(hipStreamSynchronize(st));
    std::memcpy(tokens_out, c->h_token, batch * sizeof(int));
  } else {
    IE_CHECK_HIP(hipStreamSynchronize(st));
  }
  return IE_OK;
}
}  // namespace

int ie_decode_step_batched(ie_context* c, const ie_model_weights* weights, int batch,
                           const int* seq_lens, int* tokenid_buffs, ie_bf16* data_buffer,
                           ie_bf16* attn_buffer, float* output_distr, int* output_tokens,
                           int* tokens_out, void* workspace, void* kv_caches) {
  CTX_OK(c);
  return batched_step(c, weights, batch, seq_lens, tokenid_buffs, kMaxCtx, data_buffer,
                      attn_buffer, output_distr, output_tokens, tokens_out, workspace, kv_caches,
                      nullptr, 0, 0);
}

int ie_decoder_layer_batched(ie_context* c, const ie_model_weights* weights, int layer_idx,
                             int batch, const int* seq_lens, ie_bf16* data_buffer,
                             ie_bf16* attn_buffer, void* workspace, void* kv_caches) {
  CTX_OK(c);
  IE_REQUIRE(weights && weights_complete(*weights), "decoder_layer_batched: incomplete weights");
  IE_REQUIRE(layer_idx >= 0 && layer_idx < kLayers, "decoder_layer_batched: layer %d", layer_idx);
  IE_REQUIRE(batch >= 1 && batch <= 16, "decoder_layer_batched: batch %d out of [1, 16]", batch);
  IE_REQUIRE(seq_lens && data_buffer && attn_buffer && workspace && kv_caches,
             "decoder_layer_batched: null buffer");
  int max_len = 1;
  for (int b = 0; b < batch; ++b) {
    IE_REQUIRE(seq_lens[b] >= 1 && seq_lens[b] <= kMaxCtx,
               "decoder_layer_batched: seq_lens[%d]=%d out of [1, %d]", b, seq_lens[b], kMaxCtx);
    c->h_params[1 + b] = seq_lens[b];
    max_len = std::max(max_len, seq_lens[b]);
  }
  hipStream_t st = c->stream;
  IE_CHECK_HIP(hipMemcpyAsync(c->d_params + 1, c->h_params + 1, batch * sizeof(int),
                              hipMemcpyHostToDevice, st));
  // the attention path ie_decode_step_batched takes for these lengths
  const int len_class = max_len <= kAttnDirectMaxCtx  ? kAttnDirectMaxCtx
                        : max_len <= kAttnFusedMaxCtx ? kAttnFusedMaxCtx
                                                      : kMaxCtx;
  const DecodeWs w = decode_ws(workspace, batch);
  IE_TRY(launch_rmsnorm_prep(batch, data_buffer, w.ss, st));
  IE_TRY(batched_layer(c, st, *weights, layer_idx, batch, len_class, data_buffer, attn_buffer, w,
                       kv_caches, nullptr, 0, 0, false));
  // the lengths' pinned staging is reused by the next call
  IE_CHECK_HIP(hipStreamSynchronize(st));
  return IE_OK;
}

size_t ie_kv_page_size(void) { return kPageElems * sizeof(uint16_t); }

int ie_kv_cache_to_pages(ie_context* c, const void* kv_cache, int first_pos, int n_pos,
                         void* kv_pages, int n_pages, const int* block_table) {
  CTX_OK(c);
  IE_TRY(launch_kv_to_pages(static_cast<const uint16_t*>(kv_cache), first_pos, n_pos,
                            static_cast<uint16_t*>(kv_pages), n_pages, block_table, c->stream));
  return IE_OK;
}

int ie_decode_step_batched_paged(ie_context* c, const ie_model_weights* weights, int batch,
                                 const int* seq_lens, int* tokenid_buffs, int tokens_stride,
                                 ie_bf16* data_buffer, ie_bf16* attn_buffer, float* output_distr,
                                 int* output_tokens, int* tokens_out, void* workspace,
                                 void* kv_pages, int n_pages, const int* block_tables,
                                 int table_stride) {
  CTX_OK(c);
  IE_REQUIRE(kv_pages && block_tables && n_pages >= 1,
             "decode_step_batched_paged: needs a page pool and block tables");
  IE_REQUIRE(table_stride >= 1 && table_stride <= kMaxLongCtx / kPagePos,
             "decode_step_batched_paged: table_stride %d out of [1, %d]", table_stride,
             kMaxLongCtx / kPagePos);
  IE_REQUIRE(tokens_stride >= 1, "decode_step_batched_paged: tokens_stride %d", tokens_stride);
  for (int b = 0; seq_lens && b < batch && b < 16; ++b)
    IE_REQUIRE(seq_lens[b] <= table_stride * kPagePos,
               "decode_step_batched_paged: seq_lens[%d]=%d needs more than %d table entries", b,
               seq_lens[b], table_stride);
  return batched_step(c, weights, batch, seq_lens, tokenid_buffs, tokens_stride, data_buffer,
                      attn_buffer, output_distr, output_tokens, tokens_out, workspace, kv_pages,
                      block_tables, table_stride, n_pages);
}

// ---------------------------------------------------------------- weights
int ie_init_rope_buffer(float** cu_rope_cos, float** cu_rope_sin) {
  IE_REQUIRE(cu_rope_cos && cu_rope_sin, "init_rope_buffer: null output");
  std::vector<float> ct, stb;
  rope_tables_host(ct, stb);
  const size_t bytes = ct.size() * sizeof(float);
  IE_CHECK_HIP(hipMalloc(reinterpret_cast<void**>(cu_rope_cos), bytes));
  IE_CHECK_HIP(hipMalloc(reinterpret_cast<void**>(cu_rope_sin), bytes));
  IE_CHECK_HIP(hipMemcpy(*cu_rope_cos, ct.data(), bytes, hipMemcpyHostToDevice));
  IE_CHECK_HIP(hipMemcpy(*cu_rope_sin, stb.data(), bytes, hipMemcpyHostToDevice));
  return IE_OK;
}

int ie_cleanup_rope_buffer(float* cu_rope_cos, float* cu_rope_sin) {
  IE_CHECK_HIP(hipFree(cu_rope_cos));
  IE_CHECK_HIP(hipFree(cu_rope_sin));
  return IE_OK;
}

int ie_fill_synthetic_bf16(ie_bf16* out, size_t n, uint64_t seed, uint64_t tensor_id,
                           float mean, float std, void* stream) {
  IE_REQUIRE(out != nullptr || n == 0, "fill_synthetic: null output");
  return launch_fill_synthetic(out, n, seed, tensor_id, mean, std, stream_of(stream));
}

}  // extern "C"

namespace ie {
// Tensor ids of the synthetic model (shared with the CPU oracle).
uint64_t tensor_id_of(int layer, int field) { return 16 + (uint64_t)layer * 16 + field; }

// Layer field f in the order of the synthetic tensor ids: input_layernorm, w_q, w_k, w_v, w_o,
// post_attention_layernorm, w_gate, w_up, w_down.
ie_bf16** layer_field(ie_layer& L, int f) {
  ie_bf16** slots[kLayerFields] = {&L.input_layernorm, &L.transformer.w_q, &L.transformer.w_k,
                                   &L.transformer.w_v, &L.transformer.w_o,
                                   &L.post_attention_layernorm, &L.ffn_block.w_gate,
                                   &L.ffn_block.w_up, &L.ffn_block.w_down};
  return slots[f];
}

size_t layer_field_elems(int f) {
  const size_t mat = (size_t)kHidden * kHidden, kvm = (size_t)kKVDim * kHidden,
               ffm = (size_t)kFFN * kHidden;
  const size_t e[kLayerFields] = {(size_t)kHidden, mat, kvm, kvm, mat, (size_t)kHidden, ffm, ffm, ffm};
  return e[f];
}

// One arena per model: emb | 32 x 9 layer fields | final_norm | lm_head | rope cos | rope sin,
// every tensor 256-byte aligned.
size_t weights_arena_bytes() {
  const size_t emb = (size_t)kVocab * kHidden;
  size_t total = align256(emb * 2);
  for (int l = 0; l < kLayers; ++l)
    for (int f = 0; f < kLayerFields; ++f) total += align256(layer_field_elems(f) * 2);
  return total + align256(kHidden * 2) + align256(emb * 2) +
         2 * align256((size_t)kMaxLongCtx * 64 * 4);
}

void weights_arena_assign(ie_model_weights* w, void* arena) {
  char* p = static_cast<char*>(arena);
  auto take = [&](size_t bytes) {
    void* r = p;
    p += align256(bytes);
    return r;
  };
  const size_t emb = (size_t)kVocab * kHidden;
  w->storage = arena;
  w->emb_lookup = static_cast<ie_bf16*>(take(emb * 2));
  for (int l = 0; l < kLayers; ++l)
    for (int f = 0; f < kLayerFields; ++f)
      *layer_field(w->layers[l], f) = static_cast<ie_bf16*>(take(layer_field_elems(f) * 2));
  w->final_norm = static_cast<ie_bf16*>(take(kHidden * 2));
  w->lm_head = static_cast<ie_bf16*>(take(emb * 2));
  w->rope.cos = static_cast<float*>(take((size_t)kMaxLongCtx * 64 * 4));
  w->rope.sin = static_cast<float*>(take((size_t)kMaxLongCtx * 64 * 4));
  w->rope_rows = kMaxLongCtx;
}

int weights_upload_rope(ie_model_weights* w) {
  std::vector<float> ct, stb;
  rope_tables_host(ct, stb);
  IE_CHECK_HIP(hipMemcpy(w->rope.cos, ct.data(), ct.size() * 4, hipMemcpyHostToDevice));
  IE_CHECK_HIP(hipMemcpy(w->rope.sin, stb.data(), stb.size() * 4, hipMemcpyHostToDevice));
  return IE_OK;
}
}  // namespace ie

extern "C" {

int ie_model_weights_random_init(ie_model_weights* out, uint64_t seed, float std) {
  IE_REQUIRE(out != nullptr, "random_init: null output");
  std::memset(out, 0, sizeof *out);
  void* arena = nullptr;
  IE_CHECK_HIP(hipMalloc(&arena, ie::weights_arena_bytes()));
  ie::weights_arena_assign(out, arena);
  const size_t emb = (size_t)kVocab * kHidden;
  int rc = launch_fill_synthetic(out->emb_lookup, emb, seed, 1, 0.f, std, nullptr);
  for (int l = 0; l < kLayers && rc == IE_OK; ++l) {
    for (int f = 0; f < ie::kLayerFields && rc == IE_OK; ++f) {
      const bool norm = (f == 0 || f == 5);
      rc = launch_fill_synthetic(*ie::layer_field(out->layers[l], f), ie::layer_field_elems(f),
                                 seed, tensor_id_of(l, f), norm ? 1.f : 0.f, norm ? 0.02f : std,
                                 nullptr);
    }
  }
  if (rc == IE_OK) rc = launch_fill_synthetic(out->final_norm, kHidden, seed, 2, 1.f, 0.02f, nullptr);
  if (rc == IE_OK) rc = launch_fill_synthetic(out->lm_head, emb, seed, 3, 0.f, std, nullptr);
  if (rc == IE_OK) rc = ie::weights_upload_rope(out);
  if (rc == IE_OK && hipDeviceSynchronize() != hipSuccess) {
    set_error("random_init: fill failed");
    rc = IE_ERR_HIP;
  }
  if (rc != IE_OK) {
    (void)hipFree(arena);
    std::memset(out, 0, sizeof *out);
  }
  return rc;
}

int ie_model_weights_free(ie_model_weights* w) {
  IE_REQUIRE(w != nullptr, "model_weights_free: null");
  if (w->storage) IE_CHECK_HIP(hipFree(w->storage));
  std::memset(w, 0, sizeof *w);
  return IE_OK;
}

// ---------------------------------------------------------------- ops
int ie_emblookup(int seq_len, const int* d_input, const ie_bf16* d_weights, ie_bf16* d_output,
                 void* stream) {
  IE_REQUIRE(d_input && d_weights && d_output, "emblookup: null pointer");
  return launch_emblookup(seq_len, d_input, d_weights, d_output, nullptr, 0, stream_of(stream));
}

int ie_rmsnorm(int seq_len, const ie_bf16* d_input, const ie_bf16* d_weight, ie_bf16* d_output,
               void* stream) {
  IE_REQUIRE(d_input && d_weight && d_output, "rmsnorm: null pointer");
  return launch_rmsnorm(seq_len, d_input, d_weight, d_output, stream_of(stream));
}

int ie_residual_add(int rows, int cols, ie_bf16* d_x, const ie_bf16* d_delta, void* stream) {
  IE_REQUIRE(d_x && d_delta, "residual_add: null pointer");
  IE_REQUIRE(rows >= 0 && cols >= 0, "residual_add: negative shape");
  return launch_residual_add((size_t)rows * cols, d_x, d_delta, stream_of(stream));
}

int ie_swiglu(int seq_len, const ie_bf16* d_gate, const ie_bf16* d_up, ie_bf16* d_output,
              void* stream) {
  IE_REQUIRE(d_gate && d_up && d_output, "swiglu: null pointer");
  IE_REQUIRE(seq_len >= 0, "swiglu: negative seq_len");
  return launch_swiglu((size_t)seq_len * kFFN, d_gate, d_up, d_output, stream_of(stream));
}

int ie_apply_rope(int start_pos, int num_heads, int seq_len, const float* d_rope_cos,
                  const float* d_rope_sin, const ie_bf16* d_input, ie_bf16* d_output,
                  int is_kv_cache, void* stream) {
  IE_REQUIRE(d_rope_cos && d_rope_sin && d_input && d_output, "apply_rope: null pointer");
  return launch_rope(start_pos, num_heads, seq_len, d_rope_cos, d_rope_sin, d_input, d_output,
                     is_kv_cache, stream_of(stream));
}

int ie_scale_causal_softmax(int seq_len, const ie_bf16* d_input, ie_bf16* d_output, int is_row,
                            void* stream) {
  IE_REQUIRE(d_input && d_output, "scale_causal_softmax: null pointer");
  return launch_softmax(seq_len, d_input, d_output, is_row, stream_of(stream));
}

int ie_multiply_by_weight(ie_context* c, int m, int k, int n, const ie_bf16* d_in,
                          const ie_bf16* d_w, ie_bf16* d_out) {
  CTX_OK(c);
  IE_REQUIRE(d_in && d_w && d_out, "multiply_by_weight: null pointer");
  IE_REQUIRE(m >= 1 && k >= 1 && n >= 1, "multiply_by_weight: bad shape m=%d k=%d n=%d", m, k, n);
  if (m == 1 && (k == kHidden || k == kFFN) && n % 2 == 0)
    return gemv_plain(k, kEpiBf16, d_in, nullptr, d_w, nullptr, n / 2, d_out, nullptr, 1, n,
                      c->stream);
  GemmParams g{};
  g.x = d_in;
  g.w0 = d_w;
  g.n0 = n;
  g.y = d_out;
  g.M = m;
  g.N = n;
  g.K = k;
  g.ldy = n;
  skinny_split(c, kGemmBf16, g, c->d_sk_part);
  return launch_gemm(kGemmBf16, g, c->stream);
}

int ie_gemm_bf16(ie_context* c, int m, int k, int n, const ie_bf16* d_x, const ie_bf16* d_w,
                 ie_bf16* d_y) {
  CTX_OK(c);
  IE_REQUIRE(d_x && d_w && d_y, "gemm_bf16: null pointer");
  GemmParams g{};
  g.x = d_x;
  g.w0 = d_w;
  g.n0 = n;
  g.y = d_y;
  g.M = m;
  g.N = n;
  g.K = k;
  g.ldy = n;
  skinny_split(c, kGemmBf16, g, c->d_sk_part);
  return launch_gemm(kGemmBf16, g, c->stream);
}

int ie_attn_prefill_core(ie_context* c, int seq_len, int start_pos, const ie_bf16* d_q,
                         const ie_bf16* d_k, const ie_bf16* d_v, ie_bf16* d_out) {
  CTX_OK(c);
  IE_REQUIRE(d_q && d_k && d_v && d_out, "attn_prefill_core: null pointer");
  AttnPrefillParams a{d_q, d_k, d_v, d_out, seq_len, start_pos};
  return launch_attn_prefill(a, c->stream);
}

int ie_attn_prefill_core_paged(ie_context* c, int seq_len, int start_pos, const ie_bf16* d_q,
                               const void* kv_pages, int n_pages, const int* block_table,
                               int layer, ie_bf16* d_out) {
  CTX_OK(c);
  IE_REQUIRE(d_q && kv_pages && block_table && d_out, "attn_prefill_core_paged: null pointer");
  IE_REQUIRE(n_pages >= 1 && layer >= 0 && layer < kLayers,
             "attn_prefill_core_paged: n_pages %d, layer %d", n_pages, layer);
  const uint16_t* kl = static_cast<const uint16_t*>(kv_pages) + (size_t)layer * kPageLayer;
  AttnPrefillParams a{d_q, kl, kl + (size_t)kKVHeads * kPageHead, d_out, seq_len, start_pos,
                      block_table, n_pages};
  return launch_attn_prefill(a, c->stream);
}

int ie_gemm_ex(ie_context* c, int epilogue, int m, int k, int n, const ie_bf16* d_x,
               const ie_bf16* d_w0, const ie_bf16* d_w1, void* d_y) {
  CTX_OK(c);
  IE_REQUIRE(d_x && d_w0 && d_y, "gemm_ex: null pointer");
  IE_REQUIRE(epilogue >= IE_GEMM_BF16 && epilogue <= IE_GEMM_SWIGLU, "gemm_ex: bad epilogue %d",
             epilogue);
  IE_REQUIRE(epilogue != IE_GEMM_SWIGLU || d_w1, "gemm_ex: SwiGLU needs the up matrix");
  static_assert(IE_GEMM_BF16 == kGemmBf16 && IE_GEMM_RESID == kGemmResid &&
                    IE_GEMM_F32 == kGemmF32 && IE_GEMM_SWIGLU == kGemmSwiglu,
                "epilogue codes");
  GemmParams g{};
  g.x = d_x;
  g.w0 = d_w0;
  g.w1 = d_w1;
  g.n0 = n;
  if (epilogue == IE_GEMM_F32) g.yf = static_cast<float*>(d_y);
  else g.y = static_cast<uint16_t*>(d_y);
  g.M = m;
  g.N = n;
  g.K = k;
  g.ldy = n;
  // split K's partials: a context-owned scratch, grown on first use (op-level entry; the
  // engine passes its own workspace)
  const size_t need = epilogue == IE_GEMM_F32 ? 0 : gemm_split_bytes(m, epilogue == IE_GEMM_SWIGLU ? 2 * n : n);
  if (need > c->gemm_ws_bytes) {
    IE_CHECK_HIP(hipStreamSynchronize(c->stream));
    if (c->gemm_ws) IE_CHECK_HIP(hipFree(c->gemm_ws));
    c->gemm_ws = nullptr;
    c->gemm_ws_bytes = 0;
    IE_CHECK_HIP(hipMalloc(reinterpret_cast<void**>(&c->gemm_ws), need));
    c->gemm_ws_bytes = need;
  }
  g.split_ws = c->gemm_ws;
  g.split_ws_bytes = (long long)c->gemm_ws_bytes;
  skinny_split(c, epilogue, g, c->d_sk_part);
  return launch_gemm(epilogue, g, c->stream);
}

int ie_ffn(ie_context* c, int seq_len, const ie_bf16* d_in, ie_bf16* d_out, const ie_bf16* d_wup,
           const ie_bf16* d_wdown, const ie_bf16* d_wgate, void* workspace) {
  CTX_OK(c);
  IE_REQUIRE(d_in && d_out && d_wup && d_wdown && d_wgate && workspace, "ffn: null pointer");
  IE_REQUIRE(seq_len >= 1, "ffn: seq_len=%d", seq_len);
  hipStream_t st = c->stream;
  if (seq_len == 1) {
    const DecodeWs w = decode_ws(workspace, 1);
    IE_TRY(gemv_plain(kHidden, kEpiSwiglu, d_in, nullptr, d_wgate, d_wup, kFFN, w.h, nullptr, 1, 0,
                      st));
    return gemv_plain(kFFN, kEpiBf16, w.h, nullptr, d_wdown, nullptr, kHidden / 2, d_out, nullptr,
                      1, kHidden, st);
  }
  uint16_t* h = static_cast<uint16_t*>(workspace);
  GemmParams gu{};
  gu.x = d_in;
  gu.w0 = d_wgate;
  gu.w1 = d_wup;
  gu.y = h;
  gu.M = seq_len;
  gu.N = kFFN;
  gu.K = kHidden;
  gu.ldy = kFFN;
  skinny_split(c, kGemmSwiglu, gu, c->d_sk_part);
  IE_TRY(launch_gemm(kGemmSwiglu, gu, st));
  GemmParams dn{};
  dn.x = h;
  dn.w0 = d_wdown;
  dn.n0 = kHidden;
  dn.y = d_out;
  dn.M = seq_len;
  dn.N = kHidden;
  dn.K = kFFN;
  dn.ldy = kHidden;
  skinny_split(c, kGemmBf16, dn, c->d_sk_part);
  return launch_gemm(kGemmBf16, dn, st);
}

int ie_attn(ie_context* c, const float* d_rope_cos, const float* d_rope_sin, int seq_len,
            const ie_bf16* d_input, const ie_bf16* d_qproj, const ie_bf16* d_kproj,
            const ie_bf16* d_vproj, const ie_bf16* d_oproj, ie_bf16* d_output, void* workspace,
            void* kv_cache, int layer_idx) {
  CTX_OK(c);
  IE_REQUIRE(d_rope_cos && d_rope_sin && d_input && d_qproj && d_kproj && d_vproj && d_oproj &&
                 d_output && workspace && kv_cache,
             "attn: null pointer");
  IE_REQUIRE(seq_len >= 1 && seq_len <= kMaxCtx, "attn: seq_len %d out of [1, %d]", seq_len,
             kMaxCtx);
  IE_REQUIRE(layer_idx >= 0 && layer_idx < kLayers, "attn: layer %d", layer_idx);
  hipStream_t st = c->stream;
  const int S = seq_len;
  char* wsb = static_cast<char*>(workspace);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(wsb);
  uint16_t* qrot = reinterpret_cast<uint16_t*>(wsb + align256((size_t)S * kQKVDim * 2));
  uint16_t* kvl = kv_layer(kv_cache, layer_idx);
  GemmParams g{};
  g.x = d_input;
  g.w0 = d_qproj;
  g.w1 = d_kproj;
  g.w2 = d_vproj;
  g.n0 = kHidden;
  g.n1 = kKVDim;
  g.y = qkv;
  g.M = S;
  g.N = kQKVDim;
  g.K = kHidden;
  g.ldy = kQKVDim;
  // split-K partials (both projections) after q/k/v and the rotated q
  g.split_ws = reinterpret_cast<float*>(wsb + prefill_attn_bytes(S));
  g.split_ws_bytes = (long long)(ie_attn_workspace_size(S) - prefill_attn_bytes(S));
  skinny_split(c, kGemmBf16, g, c->d_sk_part);
  IE_TRY(launch_gemm(kGemmBf16, g, st));
  IE_TRY(launch_qkv_rope_scatter(S, 0, qkv, d_rope_cos, d_rope_sin, qrot, kvl,
                                 kvl + (size_t)kKVHeads * kKVPlane, nullptr, 0, st));
  uint16_t* att = qkv;  // the projection is dead once scattered
  AttnPrefillParams a{qrot, kvl, kvl + (size_t)kKVHeads * kKVPlane, att, S, 0};
  IE_TRY(launch_attn_prefill(a, st));
  GemmParams o{};
  o.x = att;
  o.w0 = d_oproj;
  o.n0 = kHidden;
  o.y = d_output;
  o.M = S;
  o.N = kHidden;
  o.K = kHidden;
  o.ldy = kHidden;
  o.split_ws = g.split_ws;
  o.split_ws_bytes = g.split_ws_bytes;
  skinny_split(c, kGemmBf16, o, c->d_sk_part);
  return launch_gemm(kGemmBf16, o, st);
}

int ie_decode_attn(ie_context* c, const float* d_rope_cos, const float* d_rope_sin, int seq_len,
                   const ie_bf16* d_input, const ie_bf16* d_qproj, const ie_bf16* d_kproj,
                   const ie_bf16* d_vproj, const ie_bf16* d_oproj, ie_bf16* d_output,
                   void* workspace, void* kv_cache, int layer_idx) {
  CTX_OK(c);
  IE_REQUIRE(d_rope_cos && d_rope_sin && d_input && d_qproj && d_kproj && d_vproj && d_oproj &&
                 d_output && workspace && kv_cache,
             "decode_attn: null pointer");
  IE_REQUIRE(seq_len >= 1 && seq_len <= kMaxCtx, "decode_attn: seq_len %d out of [1, %d]",
             seq_len, kMaxCtx);
  IE_REQUIRE(layer_idx >= 0 && layer_idx < kLayers, "decode_attn: layer %d", layer_idx);
  hipStream_t st = c->stream;
  const DecodeWs w = decode_ws(workspace, 1);
  uint16_t* kvl = kv_layer(kv_cache, layer_idx);
  ie_layer L{};
  L.transformer.w_q = const_cast<ie_bf16*>(d_qproj);
  L.transformer.w_k = const_cast<ie_bf16*>(d_kproj);
  L.transformer.w_v = const_cast<ie_bf16*>(d_vproj);
  ie_rope_weights rope{const_cast<float*>(d_rope_cos), const_cast<float*>(d_rope_sin)};
  IE_TRY(qkv_rope_gemv(L, rope, d_input, nullptr, w.q, kvl, nullptr, seq_len - 1, st));
  IE_TRY(attn_decode(w.q, kvl, w.attn1, w, nullptr, seq_len, seq_len, 1, 0, true, st));
  return gemv_plain(kHidden, kEpiBf16, w.attn1, nullptr, d_oproj, nullptr, kHidden / 2, d_output,
                    nullptr, 1, kHidden, st);
}

int ie_lm_head(ie_context* c, int seq_len, const ie_bf16* d_input, const ie_bf16* d_weight,
               float* d_output) {
  CTX_OK(c);
  IE_REQUIRE(d_input && d_weight && d_output, "lm_head: null pointer");
  IE_REQUIRE(seq_len >= 1, "lm_head: seq_len=%d", seq_len);
  return gemv_plain(kHidden, kEpiF32, d_input + (size_t)(seq_len - 1) * kHidden, nullptr,
                    d_weight, nullptr, kVocab / 2, nullptr, d_output, 1, kVocab, c->stream);
}

int ie_sample_token_amax(ie_context* c, const float* d_logits, int* d_output) {
  CTX_OK(c);
  IE_REQUIRE(d_logits && d_output, "sample_token_amax: null pointer");
  return launch_argmax_rows(1, kVocab, d_logits, d_output, c->d_slots,
                            c->d_counters + kCntArgmax, c->stream);
}

int ie_sample_argmax_rows(ie_context* c, int rows, int vocab, const float* d_logits,
                          int* d_output) {
  CTX_OK(c);
  IE_REQUIRE(d_logits && d_output, "sample_argmax_rows: null pointer");
  return launch_argmax_rows(rows, vocab, d_logits, d_output, c->d_slots,
                            c->d_counters + kCntArgmax, c->stream);
}

size_t ie_top_p_workspace_size(int rows, int vocab) {
  return top_p_workspace_bytes(rows < 1 ? 1 : rows, vocab < 1 ? 1 : vocab);
}

int ie_sample_top_p(ie_context* c, int rows, int vocab, const float* d_logits, float temperature,
                    float top_p, uint64_t seed, uint64_t step, int* d_output, void* workspace) {
  CTX_OK(c);
  IE_REQUIRE(d_logits && d_output && workspace, "sample_top_p: null pointer");
  return launch_top_p(rows, vocab, d_logits, temperature, top_p, seed, step, d_output,
                      static_cast<float*>(workspace), c->stream);
}

// No allocation: the exponentials go to the library's static per-device scratch
// (top_p_scratch), resolved when a context was created on this device.  Calls that overlap on
// one GPU share that scratch and race.
int ie_sample_top_p_noalloc(ie_context* c, int rows, int vocab, const float* d_logits,
                            float temperature, float top_p, uint64_t seed, uint64_t step,
                            int* d_output) {
  CTX_OK(c);
  IE_REQUIRE(d_logits && d_output, "sample_top_p_noalloc: null pointer");
  IE_REQUIRE(rows >= 1 && vocab >= 1, "sample_top_p_noalloc: rows=%d vocab=%d", rows, vocab);
  IE_REQUIRE(rows <= kTopPNoallocRows && (size_t)rows * (size_t)vocab <= kTopPScratchFloats &&
                 top_p_workspace_bytes(rows, vocab) <= kTopPScratchBytes,
             "sample_top_p_noalloc: rows x vocab = %d x %d exceeds the static scratch (%d rows, "
             "%zu logits; use ie_sample_top_p with a workspace)",
             rows, vocab, kTopPNoallocRows, kTopPScratchFloats);
  float* ws = top_p_scratch(c->device);
  IE_REQUIRE(ws != nullptr, "sample_top_p_noalloc: scratch of device %d not initialised",
             c->device);
  return launch_top_p(rows, vocab, d_logits, temperature, top_p, seed, step, d_output, ws,
                      c->stream);
}

int ie_ffn_block_decode(ie_context* c, ie_bf16* d_x_resid, const ie_bf16* d_norm_w,
                        const ie_bf16* d_wgate, const ie_bf16* d_wup, const ie_bf16* d_wdown,
                        void* workspace) {
  CTX_OK(c);
  IE_REQUIRE(d_x_resid && d_norm_w && d_wgate && d_wup && d_wdown && workspace,
             "ffn_block_decode: null pointer");
  const DecodeWs w = decode_ws(workspace, 1);
  IE_TRY(gemv_plain(kHidden, kEpiSwiglu, d_x_resid, d_norm_w, d_wgate, d_wup, kFFN, w.h, nullptr,
                    1, 0, c->stream));
  return gemv_plain(kFFN, kEpiResid, w.h, nullptr, d_wdown, nullptr, kHidden / 2, d_x_resid,
                    nullptr, 1, 0, c->stream);
}

int ie_ffn_gate_up_decode(ie_context* c, const ie_bf16* d_x, const ie_bf16* d_norm_w,
                          const ie_bf16* d_wgate, const ie_bf16* d_wup, ie_bf16* d_h) {
  CTX_OK(c);
  IE_REQUIRE(d_x && d_norm_w && d_wgate && d_wup && d_h, "ffn_gate_up_decode: null pointer");
  return gemv_plain(kHidden, kEpiSwiglu, d_x, d_norm_w, d_wgate, d_wup, kFFN, d_h, nullptr, 1, 0,
                    c->stream);
}

int ie_decoder_layer_decode(ie_context* c, const ie_model_weights* weights, int layer_idx,
                            int seq_len, ie_bf16* d_x, ie_bf16* d_attn_out, void* workspace,
                            void* kv_cache) {
  CTX_OK(c);
  IE_REQUIRE(weights && d_x && d_attn_out && workspace && kv_cache,
             "decoder_layer_decode: null pointer");
  IE_REQUIRE(layer_idx >= 0 && layer_idx < kLayers, "decoder_layer_decode: layer %d", layer_idx);
  IE_REQUIRE(seq_len >= 1 && seq_len <= kMaxCtx, "decoder_layer_decode: seq_len %d", seq_len);
  return decoder_layer_decode(c, c->stream, *weights, layer_idx, d_x, d_attn_out,
                              decode_ws(workspace, 1), kv_cache, nullptr, seq_len);
}

int ie_final_norm_lm_head(ie_context* c, int rows, const ie_bf16* d_x, const ie_bf16* d_norm_w,
                          const ie_bf16* d_lm_head, float* d_logits) {
  CTX_OK(c);
  IE_REQUIRE(d_x && d_norm_w && d_lm_head && d_logits, "final_norm_lm_head: null pointer");
  IE_REQUIRE(rows >= 1 && rows <= 64, "final_norm_lm_head: rows %d out of [1, 64]", rows);
  return gemv_plain(kHidden, kEpiF32, d_x, d_norm_w, d_lm_head, nullptr, kVocab / 2, nullptr,
                    d_logits, rows, kVocab, c->stream);
}

int ie_model_weights_from_safetensors(ie_model_weights* out, const char* const* paths,
                                      int n_paths) {
  return ie::load_safetensors(out, paths, n_paths);
}

}  // extern "C"
