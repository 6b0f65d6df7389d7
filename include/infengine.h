/*
 * infengine.h — C-ABI of the MI355X (gfx950) per-token Llama-3.1-8B hot path.
 *
 * Every entry point is `extern "C"`, takes plain device pointers and sizes, and
 * returns an int status (IE_OK == 0, negative on error; ie_last_error() gives
 * the message).  Token-returning entry points (ie_prefill, ie_decode_step)
 * return the token id (>= 0) on success.
 *
 * Storage type is bf16 (IEEE binary32 truncated to the top 16 bits, passed as
 * uint16_t); accumulation is fp32 everywhere; logits are fp32.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   config.h:5-27                     -> IE_* shape constants below
 *   kernels/model_weights.cuh:7-34    -> ie_model_weights and its sub-structs
 *   prefill.cuh:6-9                   -> ie_prefill
 *   decode.cuh:6-9                    -> ie_decode_step
 *   kernels/<op>.cuh host launchers   -> ie_<op> launchers (one per reference op)
 * cublasHandle_t is replaced by an opaque ie_context (owns the HIP stream and
 * the small device-side counters some kernels use); `half` becomes bf16.
 */
#ifndef INFENGINE_H
#define INFENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IE_API __attribute__((visibility("default")))

/* config.h:5-27 (InfEngineConfig) */
#define IE_MAX_CONTEXT_LENGTH 8192
/* Positions the paged KV paths (ie_prefill_paged*, ie_decode_step_batched_paged) and the RoPE
 * tables cover: Llama-3.1's 131072 (max_position_embeddings).  No reference counterpart: the
 * reference's cache and tables stop at IE_MAX_CONTEXT_LENGTH (config.h:7, attn.cu:304-307,
 * rope.cu:68-103), which the reference-layout entry points keep. */
#define IE_MAX_LONG_CONTEXT 131072
#define IE_VOCAB_SIZE 128256
#define IE_NUM_LAYERS 32
#define IE_HIDDEN_SIZE 4096
#define IE_NUM_Q_HEADS 32
#define IE_NUM_KV_HEADS 8
#define IE_HEAD_DIM 128
#define IE_FFN_DIM 14336
#define IE_BF16_SIZE 2

/* status codes */
#define IE_OK 0
#define IE_ERR_INVALID_ARG (-1)
#define IE_ERR_HIP (-2)
#define IE_ERR_UNSUPPORTED (-3)
#define IE_ERR_IO (-4)
#define IE_ERR_FORMAT (-5)
#define IE_ERR_OOM (-6)

typedef uint16_t ie_bf16;

/* kernels/model_weights.cuh:7-9 — same field names and order, bf16 storage */
typedef struct ie_transformer_block_weights {
  ie_bf16* w_k; /* [1024, 4096] */
  ie_bf16* w_q; /* [4096, 4096], rows grouped per head (attn.cu:25) */
  ie_bf16* w_v; /* [1024, 4096] */
  ie_bf16* w_o; /* [4096, 4096] */
} ie_transformer_block_weights;

typedef struct ie_ffn_block_weights {
  ie_bf16* w_up;   /* [14336, 4096] */
  ie_bf16* w_gate; /* [14336, 4096] */
  ie_bf16* w_down; /* [4096, 14336] */
} ie_ffn_block_weights;

typedef struct ie_rope_weights {
  float* cos; /* [rope_rows, 64] fp32 (rows 0..8191: the reference's [8192, 64] table) */
  float* sin; /* [rope_rows, 64] fp32 */
} ie_rope_weights;

/* kernels/model_weights.cuh:11-19 */
typedef struct ie_layer {
  ie_bf16* input_layernorm; /* [4096] */
  ie_transformer_block_weights transformer;
  ie_bf16* post_attention_layernorm; /* [4096] */
  ie_ffn_block_weights ffn_block;
} ie_layer;

/* kernels/model_weights.cuh:21-34.  `storage` is the library-owned arena that
 * backs every pointer when the weights were made by ie_model_weights_random_init
 * or ie_model_weights_from_safetensors; NULL when the caller owns them.
 * `rope_rows` (no reference counterpart) is the number of rows of rope.cos and
 * rope.sin: 0 means IE_MAX_CONTEXT_LENGTH, the reference's 8192.  The library's
 * constructors set IE_MAX_LONG_CONTEXT; a caller assembling its own weights with
 * ie_init_rope_buffer's tables may set that too.  Every entry point refuses
 * positions at or past it. */
typedef struct ie_model_weights {
  ie_bf16* emb_lookup; /* [128256, 4096] */
  ie_layer layers[IE_NUM_LAYERS];
  ie_bf16* final_norm; /* [4096] */
  ie_bf16* lm_head;    /* [128256, 4096] (untied) */
  ie_rope_weights rope;
  void* storage;
  int rope_rows;
} ie_model_weights;

typedef struct ie_context ie_context;

/* ---- context / errors (replaces cublasCreate/cublasDestroy, manager.cpp:58-59,107) ---- */
/* stream: the hipStream_t every call on this context runs on; NULL means the
 * legacy default stream (the reference's implicit ordering).  device: a device
 * index, or IE_CURRENT_DEVICE for the calling thread's current device. */
#define IE_CURRENT_DEVICE (-1)
IE_API int ie_context_create(ie_context** out, int device, void* stream);
IE_API int ie_context_destroy(ie_context* ctx);
IE_API void* ie_context_stream(ie_context* ctx);
/* Replay decode steps through a captured hipGraph (default on). */
IE_API int ie_context_set_graph(ie_context* ctx, int enable);
IE_API const char* ie_last_error(void);

/* ---- sizing (attn.cu:295-307, ffn.cu:35-37) ---- */
IE_API size_t ie_attn_workspace_size(int max_seq_len);
IE_API size_t ie_ffn_workspace_size(int max_seq_len);
IE_API size_t ie_kv_cache_size(void); /* [32][2][8][8192][128] bf16 = 1 GiB */

/* ---- engine entry points (prefill.cuh:6-9, decode.cuh:6-9) ----
 * Same 11 parameters, order and meaning as the reference; returns the greedy
 * (argmax) token id, also written to *output_token (device).  output_distr
 * receives fp32 logits [128256] of the last position.  seq_len counts the
 * tokens in tokenid_buff; decode_step embeds tokenid_buff[seq_len-1] and writes
 * its K/V at cache row seq_len-1. */
IE_API int ie_prefill(ie_context* ctx, const ie_model_weights* weights, int seq_len,
                      int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                      ie_bf16* attn_buffer, float* output_distr, int* output_token,
                      void* workspace, void* kv_cache);
IE_API int ie_decode_step(ie_context* ctx, const ie_model_weights* weights, int seq_len,
                          int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                          ie_bf16* attn_buffer, float* output_distr, int* output_token,
                          void* workspace, void* kv_cache);
/* manager.cpp:31-86 (Manager::handle_request) without the tokenizer: copies the prompt ids to
 * tokenid_buff, runs ie_prefill, then decode steps, writing each token back to tokenid_buff on
 * the device (manager.cpp:75, 84) before the next step reads it.  out_tokens (host,
 * max_new_tokens) receives the prefill's token then each step's.  The loop ends after
 * max_new_tokens tokens, or right after a token equal to eos_token (kept in out_tokens; a
 * negative eos_token never matches).  timed_ms (optional) receives the host wall time of decode
 * steps timed_from .. the last one (0 when none ran).  Returns the number of tokens produced
 * or a negative status. */
IE_API int ie_generate(ie_context* ctx, const ie_model_weights* weights, const int* prompt,
                       int prompt_len, int max_new_tokens, int eos_token, int timed_from,
                       int* out_tokens, int* tokenid_buff, ie_bf16* data_buffer,
                       ie_bf16* aux_buffer, ie_bf16* attn_buffer, float* output_distr,
                       int* output_token, void* workspace, void* kv_cache, double* timed_ms);

/* Batched decode (no reference counterpart: manager.h:19-24 RequestContext is
 * unused there).  `batch` independent sequences; seq_lens is a HOST array;
 * tokenid_buffs is a device array [batch][8192]; row b's K/V live in
 * kv_caches + b * ie_kv_cache_size().  data/attn buffers are [batch, 4096];
 * output_distr [batch, 128256]; output_tokens (device) [batch]; tokens_out
 * (host, may be NULL) receives the greedy ids. */
IE_API size_t ie_batch_workspace_size(int batch);
IE_API int ie_decode_step_batched(ie_context* ctx, const ie_model_weights* weights, int batch,
                                  const int* seq_lens, int* tokenid_buffs,
                                  ie_bf16* data_buffer, ie_bf16* attn_buffer,
                                  float* output_distr, int* output_tokens, int* tokens_out,
                                  void* workspace, void* kv_caches);

/* Paged KV cache for the batched step (no reference counterpart; the step toward a
 * paged cache that manager.h:19-24's per-request RequestContext leads to).  A page
 * holds 64 positions of every layer, [32 layers][K|V][8 kv heads][64][128] bf16
 * (ie_kv_page_size() = 8 MiB); kv_pages is a pool of n_pages pages.  block_tables
 * is a DEVICE int array [batch][table_stride]: entry i of row b is the page that
 * holds positions 64*i .. 64*i+63 of sequence b; entries 0 .. (seq_lens[b]-1)/64
 * must be set (the step writes the new K/V row at position seq_lens[b]-1).  Page
 * ids outside [0, n_pages) read as zero and are not written.  Results are
 * bit-identical to ie_decode_step_batched on the same rows. */
IE_API size_t ie_kv_page_size(void);
/* ie_prefill writing the prompt's K/V rows into pages: block_table (device) is the
 * sequence's page per 64-position block, entries 0 .. (seq_len-1)/64 set.  Same arguments and
 * results as ie_prefill otherwise (bit-identical logits / token); seq_len may reach
 * IE_MAX_LONG_CONTEXT (buffers and workspace sized for seq_len rows). */
IE_API int ie_prefill_paged(ie_context* ctx, const ie_model_weights* weights, int seq_len,
                            int* tokenid_buff, ie_bf16* data_buffer, ie_bf16* aux_buffer,
                            ie_bf16* attn_buffer, float* output_distr, int* output_token,
                            void* workspace, void* kv_pages, int n_pages,
                            const int* block_table);
/* Chunked prefill over pages (no reference counterpart): the n_tokens prompt tokens at
 * positions start_pos .. start_pos + n_tokens - 1 (tokenid_buff indexed by position) attend to
 * the K/V of positions 0 .. start_pos - 1 already in the sequence's pages and to each other
 * causally; their K/V rows are written into the pages.  data/aux/attn buffers and the workspace
 * are sized for n_tokens rows.  Returns the greedy token after the chunk's last position
 * (logits in output_distr).  start_pos = 0 is ie_prefill_paged. */
IE_API int ie_prefill_paged_chunk(ie_context* ctx, const ie_model_weights* weights, int start_pos,
                                  int n_tokens, int* tokenid_buff, ie_bf16* data_buffer,
                                  ie_bf16* aux_buffer, ie_bf16* attn_buffer, float* output_distr,
                                  int* output_token, void* workspace, void* kv_pages, int n_pages,
                                  const int* block_table);
/* Positions [first_pos, first_pos + n_pos) of every layer of a reference-layout
 * KV cache (e.g. just written by ie_prefill) into the pages that block_table
 * (device, one sequence's row) maps them to; ids outside [0, n_pages) skipped.
 * Runs on the context's stream. */
IE_API int ie_kv_cache_to_pages(ie_context* ctx, const void* kv_cache, int first_pos, int n_pos,
                                void* kv_pages, int n_pages, const int* block_table);
/* The batched step over pages.  tokenid_buffs is [batch][tokens_stride] (row b holds sequence
 * b's ids by position; tokens_stride >= every seq_lens[b]); seq_lens[b] <= IE_MAX_LONG_CONTEXT
 * and <= 64 * table_stride. */
IE_API int ie_decode_step_batched_paged(ie_context* ctx, const ie_model_weights* weights,
                                        int batch, const int* seq_lens, int* tokenid_buffs,
                                        int tokens_stride, ie_bf16* data_buffer,
                                        ie_bf16* attn_buffer, float* output_distr,
                                        int* output_tokens, int* tokens_out, void* workspace,
                                        void* kv_pages, int n_pages, const int* block_tables,
                                        int table_stride);

/* ---- weights (model_weights.cu:142-172) ---- */
/* Random-init Llama-3.1-8B: matrices ~N(0,std), norms ~1+N(0,0.02), rope tables. */
IE_API int ie_model_weights_random_init(ie_model_weights* out, uint64_t seed, float std);
IE_API int ie_model_weights_from_safetensors(ie_model_weights* out, const char* const* paths,
                                             int n_paths);
IE_API int ie_model_weights_free(ie_model_weights* w);
/* rope.cu:68-103: Llama-3 scaled RoPE tables, fp32 [131072, 64] (the reference's [8192, 64]
 * continued to IE_MAX_LONG_CONTEXT positions by the same formula); allocates. */
IE_API int ie_init_rope_buffer(float** cu_rope_cos, float** cu_rope_sin);
IE_API int ie_cleanup_rope_buffer(float* cu_rope_cos, float* cu_rope_sin);
/* Deterministic synthetic tensor: out[i] = bf16(mean + std * z_i), z_i an
 * integer-exact approximate normal keyed by (seed, tensor_id, i). */
IE_API int ie_fill_synthetic_bf16(ie_bf16* out, size_t n, uint64_t seed, uint64_t tensor_id,
                                  float mean, float std, void* stream);

/* ---- op launchers (one per reference host launcher); stream may be NULL ---- */
/* emblookup.cu:7-10 */
IE_API int ie_emblookup(int seq_len, const int* d_input, const ie_bf16* d_weights,
                        ie_bf16* d_output, void* stream);
/* rmsnorm.cu:7-10 (eps 1e-5, hidden 4096) */
IE_API int ie_rmsnorm(int seq_len, const ie_bf16* d_input, const ie_bf16* d_weight,
                      ie_bf16* d_output, void* stream);
/* residual_add.cu:5-8: x += delta */
IE_API int ie_residual_add(int rows, int cols, ie_bf16* d_x, const ie_bf16* d_delta,
                           void* stream);
/* swiglu.cu:8-14: out = silu(gate) * up over [seq_len, 14336] */
IE_API int ie_swiglu(int seq_len, const ie_bf16* d_gate, const ie_bf16* d_up,
                     ie_bf16* d_output, void* stream);
/* rope.cu:20-22: rotate-half pairs (j, j+64) of [num_heads, seq_len|8192, 128] */
IE_API int ie_apply_rope(int start_pos, int num_heads, int seq_len, const float* d_rope_cos,
                         const float* d_rope_sin, const ie_bf16* d_input, ie_bf16* d_output,
                         int is_kv_cache, void* stream);
/* softmax.cu:10-20: softmax(x / sqrt(128)) over rows of [32, seq_len, seq_len]
 * (causal) or [32, seq_len] (is_row) */
IE_API int ie_scale_causal_softmax(int seq_len, const ie_bf16* d_input, ie_bf16* d_output,
                                   int is_row, void* stream);
/* ffn.cu:7-33: Y[m,n] = X[m,k] . W[n,k]^T, bf16 out, fp32 accumulate */
IE_API int ie_multiply_by_weight(ie_context* ctx, int m, int k, int n, const ie_bf16* d_in,
                                 const ie_bf16* d_w, ie_bf16* d_out);
/* ffn.cu:39-64: out = down(silu(gate . x) * (up . x)) */
IE_API int ie_ffn(ie_context* ctx, int seq_len, const ie_bf16* d_in, ie_bf16* d_out,
                  const ie_bf16* d_wup, const ie_bf16* d_wdown, const ie_bf16* d_wgate,
                  void* workspace);
/* attn.cu:309-371: causal GQA self-attention of seq_len rows from position 0;
 * K/V written to the cache rows 0..seq_len-1 of layer_idx. */
IE_API int ie_attn(ie_context* ctx, const float* d_rope_cos, const float* d_rope_sin,
                   int seq_len, const ie_bf16* d_input, const ie_bf16* d_qproj,
                   const ie_bf16* d_kproj, const ie_bf16* d_vproj, const ie_bf16* d_oproj,
                   ie_bf16* d_output, void* workspace, void* kv_cache, int layer_idx);
/* attn.cu:373-439: one decode row at position seq_len-1 */
IE_API int ie_decode_attn(ie_context* ctx, const float* d_rope_cos, const float* d_rope_sin,
                          int seq_len, const ie_bf16* d_input, const ie_bf16* d_qproj,
                          const ie_bf16* d_kproj, const ie_bf16* d_vproj,
                          const ie_bf16* d_oproj, ie_bf16* d_output, void* workspace,
                          void* kv_cache, int layer_idx);
/* lm_head.cu:5-20: logits (fp32) of row seq_len-1 */
IE_API int ie_lm_head(ie_context* ctx, int seq_len, const ie_bf16* d_input,
                      const ie_bf16* d_weight, float* d_output);
/* sampling.cu:54-58: argmax over 128256 fp32 logits (first maximal index,
 * NaN counts as the maximum, -0.0 == +0.0) */
IE_API int ie_sample_token_amax(ie_context* ctx, const float* d_logits, int* d_output);
/* Row-wise argmax over [rows, vocab]. */
IE_API int ie_sample_argmax_rows(ie_context* ctx, int rows, int vocab, const float* d_logits,
                                 int* d_output);
/* Temperature + top-p (nucleus) sampling over [rows, vocab] fp32 logits; no
 * reference counterpart (sampling.cu has argmax only).  Deterministic:
 * uniform u = counter RNG(seed, row, step); inverse CDF in token-id order over
 * the kept set.  workspace: ie_top_p_workspace_size(rows, vocab) bytes. */
IE_API size_t ie_top_p_workspace_size(int rows, int vocab);
IE_API int ie_sample_top_p(ie_context* ctx, int rows, int vocab, const float* d_logits,
                           float temperature, float top_p, uint64_t seed, uint64_t step,
                           int* d_output, void* workspace);
/* No reference counterpart: ie_sample_top_p without the workspace, for callers that cannot
 * allocate (HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * allocates nothing: its workspace is a static device array of the library, one per GPU, of
 * 10 MiB (rows <= IE_TOP_P_NOALLOC_ROWS and rows * vocab <= 16 * 131072 =
 * IE_TOP_P_NOALLOC_MAX; larger calls return IE_ERR_INVALID_ARG).  Same results as
 * ie_sample_top_p.  Calls that overlap on one GPU (any context, any stream) share that array
 * and race. */
#define IE_TOP_P_NOALLOC_MAX (16 * 131072)
#define IE_TOP_P_NOALLOC_ROWS 16
IE_API int ie_sample_top_p_noalloc(ie_context* ctx, int rows, int vocab, const float* d_logits,
                                   float temperature, float top_p, uint64_t seed, uint64_t step,
                                   int* d_output);

/* ---- fused decode kernels (building blocks of ie_decode_step, exposed for tests) ---- */
/* x_resid += W_down . (silu(W_gate . rmsnorm(x_resid)) * (W_up . rmsnorm(x_resid))) */
IE_API int ie_ffn_block_decode(ie_context* ctx, ie_bf16* d_x_resid, const ie_bf16* d_norm_w,
                               const ie_bf16* d_wgate, const ie_bf16* d_wup,
                               const ie_bf16* d_wdown, void* workspace);
/* h = silu(W_gate . rmsnorm(x)) * (W_up . rmsnorm(x)), one kernel: the dominant
 * decode kernel (two 117 MB weight streams per layer). */
IE_API int ie_ffn_gate_up_decode(ie_context* ctx, const ie_bf16* d_x, const ie_bf16* d_norm_w,
                                 const ie_bf16* d_wgate, const ie_bf16* d_wup, ie_bf16* d_h);
/* One full decoder layer for a single token at position seq_len-1 (in place on d_x). */
IE_API int ie_decoder_layer_decode(ie_context* ctx, const ie_model_weights* weights,
                                   int layer_idx, int seq_len, ie_bf16* d_x,
                                   ie_bf16* d_attn_out, void* workspace, void* kv_cache);
/* One iteration of prefill.cu:17-38's layer loop: decoder layer layer_idx of ie_prefill over
 * seq_len rows (positions 0 .. seq_len-1) of data_buffer [seq_len][4096], in place, writing
 * that layer's K/V rows 0 .. seq_len-1 of kv_cache; aux/attn buffers and workspace
 * (max(ie_attn_workspace_size, ie_ffn_workspace_size)(seq_len) bytes) as ie_prefill.
 * ie_prefill is the embedding, 31 of these calls, ie_decoder_layer_prefill_last_row for layer
 * 31, then final norm + lm_head on the last row and argmax, bit for bit. */
IE_API int ie_decoder_layer_prefill(ie_context* ctx, const ie_model_weights* weights,
                                    int layer_idx, int seq_len, ie_bf16* data_buffer,
                                    ie_bf16* aux_buffer, ie_bf16* attn_buffer, void* workspace,
                                    void* kv_cache);
/* Decoder layer layer_idx of a prefill whose output is needed for the last row only (no
 * reference counterpart: prefill.cu:17-38 runs every layer over all rows, but only the last
 * row reaches the final norm and lm_head, prefill.cu:41-43): K/V rows 0 .. seq_len-1 as
 * ie_decoder_layer_prefill writes them, the last row of data_buffer as a decode step at
 * position seq_len-1 computes it (attention over the cache, O projection + residual, FFN);
 * rows 0 .. seq_len-2 keep the layer's input.  ie_prefill runs it for its last layer. */
IE_API int ie_decoder_layer_prefill_last_row(ie_context* ctx, const ie_model_weights* weights,
                                             int layer_idx, int seq_len, ie_bf16* data_buffer,
                                             ie_bf16* aux_buffer, ie_bf16* attn_buffer,
                                             void* workspace, void* kv_cache);
/* One decoder layer of ie_decode_step_batched (no reference counterpart: the reference decodes
 * one sequence) over batch rows [batch][4096] of data_buffer, in place; row b is sequence b at
 * position seq_lens[b]-1 of cache b (kv_caches as ie_decode_step_batched), workspace
 * ie_batch_workspace_size(batch) bytes.  Synchronous.  The step's residual rows after its 32
 * layers equal the embedding followed by these 32 calls, bit for bit. */
IE_API int ie_decoder_layer_batched(ie_context* ctx, const ie_model_weights* weights,
                                    int layer_idx, int batch, const int* seq_lens,
                                    ie_bf16* data_buffer, ie_bf16* attn_buffer, void* workspace,
                                    void* kv_caches);
/* final RMSNorm + lm_head GEMV to fp32 logits for `rows` rows of [rows, 4096]. */
IE_API int ie_final_norm_lm_head(ie_context* ctx, int rows, const ie_bf16* d_x,
                                 const ie_bf16* d_norm_w, const ie_bf16* d_lm_head,
                                 float* d_logits);
/* Tuning (no reference counterpart): force the decode GEMV's row pairs per wave
 * (0 restores the built-in per-shape choice).  Affects kernels launched after
 * the call, on every context of the process. */
IE_API int ie_tune_gemv_pairs_per_wave(int ppw);
/* Tuning (no reference counterpart): force the decode GEMV's waves per workgroup
 * (4, 8 or 16; 0 restores the built-in choice).  Same scope as above. */
IE_API int ie_tune_gemv_waves(int waves);
/* Tuning (no reference counterpart): the kernel of the prefill GEMM's bf16 tiles of
 * 128 or 256 rows: 0 the DMA-ring kernels, 1 the ping-pong kernel for the 256-row
 * tiles only, 2 (default) the ping-pong kernel for both, 3 as 2 with 4 weight ring
 * slots on the 256 x 128 and 192 x 256 tiles.  Results are bit-identical above 128
 * rows.  At 17-128 rows schedules 2 and 3 run the 64-weight-row streaming kernel,
 * 0 and 1 the older 17-48-row and split-K kernels (other K splits: results agree to
 * bf16 rounding).  Same scope as above. */
IE_API int ie_tune_gemm_schedule(int schedule);
/* Plain GEMM Y[m,n] = X[m,k] . W[n,k]^T on the MFMA path (any m >= 1). */
IE_API int ie_gemm_bf16(ie_context* ctx, int m, int k, int n, const ie_bf16* d_x,
                        const ie_bf16* d_w, ie_bf16* d_y);
/* The MFMA GEMM with a selectable fused epilogue (no reference counterpart; the
 * prefill path uses each of them):
 *   IE_GEMM_BF16    y[m,n] = bf16(X . W0^T)                         (d_y bf16)
 *   IE_GEMM_RESID   y[m,n] = bf16(y + bf16(X . W0^T))               (d_y bf16, read+written)
 *   IE_GEMM_F32     y[m,n] = X . W0^T                               (d_y fp32)
 *   IE_GEMM_SWIGLU  y[m,n] = swiglu(bf16(X . W0^T), bf16(X . W1^T)) (d_y bf16; W0 gate, W1 up)
 * W0/W1 are [n][k]; n % 4 == 0, k % 64 == 0. */
#define IE_GEMM_BF16 0
#define IE_GEMM_RESID 1
#define IE_GEMM_F32 2
#define IE_GEMM_SWIGLU 3
IE_API int ie_gemm_ex(ie_context* ctx, int epilogue, int m, int k, int n, const ie_bf16* d_x,
                      const ie_bf16* d_w0, const ie_bf16* d_w1, void* d_y);
/* The causal GQA attention core of prefill on its own (the softmax(QK^T / sqrt(128)) V step of
 * kernels/attn.cu:309-371, without the projections): d_q [seq_len][32][128] (RoPE applied),
 * d_k / d_v one layer's K and V planes [8][8192][128] holding key rows 0..start_pos+seq_len-1,
 * d_out [seq_len][4096] bf16 in the [s][h][d] layout of attn_permute.cu:15-31.  Query row i sits
 * at position start_pos + i and sees keys 0..start_pos+i. */
IE_API int ie_attn_prefill_core(ie_context* ctx, int seq_len, int start_pos, const ie_bf16* d_q,
                                const ie_bf16* d_k, const ie_bf16* d_v, ie_bf16* d_out);
/* The same attention core over a page pool (ie_kv_page_size() pages; block_table (device) maps
 * 64-key block i to a page): the keys of page-layout layer `layer`, positions 0 ..
 * start_pos + seq_len - 1 <= IE_MAX_LONG_CONTEXT - 1. */
IE_API int ie_attn_prefill_core_paged(ie_context* ctx, int seq_len, int start_pos,
                                      const ie_bf16* d_q, const void* kv_pages, int n_pages,
                                      const int* block_table, int layer, ie_bf16* d_out);

#ifdef __cplusplus
}
#endif

#endif /* INFENGINE_H */
