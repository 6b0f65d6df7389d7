// Host-side launchers of the gfx950 kernels (internal to the library).
#pragma once

#include "ie_common.h"

namespace ie {

// ------------------------------------------------------------ GEMV (m = 1 rows)
enum GemvEpi : int {
  kEpiBf16 = 0,    // out[r] = bf16(acc)
  kEpiF32 = 1,     // out_f32[r] = acc
  kEpiResid = 2,   // out[r] = bf16(out[r] + bf16(acc))              (residual_add.cu:17-19)
  kEpiSwiglu = 3,  // out[r] = bf16(silu(bf16(g)) * bf16(u))          (swiglu.cu:24-29)
  kEpiQkvRope = 4  // q/k/v rows (j, j+64) of a head, RoPE on q,k, k/v -> cache (attn.cu:411-420)
};

struct GemvParams {
  const uint16_t* x;       // input rows [rows][K]
  const uint16_t* norm_w;  // [K] RMSNorm weight applied to x first, or nullptr
  const uint16_t* w0;      // weight [N][K] (gate for SwiGLU, w_q for QKV)
  const uint16_t* w1;      // up (SwiGLU) / w_k (QKV)
  const uint16_t* w2;      // w_v (QKV)
  uint16_t* out;           // bf16 output / residual stream / q output
  float* out_f32;          // fp32 output
  uint16_t* k_cache;       // QKV: this layer's K plane base [8][8192][128]
  uint16_t* v_cache;       // QKV: this layer's V plane base
  const float* rope_cos;   // [8192][64]
  const float* rope_sin;
  const int* d_seq_len;    // QKV: position = *d_seq_len - 1 when set
  int pos;                 // QKV: position when d_seq_len == nullptr (attention input: length)
  int n_pairs;             // row pairs per input row
  int ppw;                 // pairs per wave
  long long x_stride;      // elements between input rows
  long long out_stride;    // elements between output rows (kEpiBf16 / kEpiF32)
  // K = 4096 residual GEMV only: the input row is the decode attention output, built in the
  // prologue from the split partials (part_o / part_ml of batch row 0, splits of d_seq_len)
  const float* attn_part_o;
  const float* attn_part_ml;
  int attn_max_splits;
};

// K must be 4096 or 14336.  rows > 1 re-reads the weights once per row.
int launch_gemv(int K, int epi, bool norm, GemvParams p, int rows, hipStream_t st);
int default_ppw(int n_pairs);
int gemv_waves(int K, int epi, int n_pairs);

// ------------------------------------------------------------ decode attention
struct AttnDecodeParams {
  const uint16_t* q;        // [batch][32][128] bf16, RoPE applied
  const uint16_t* k_cache;  // batch 0 layer K base [8][8192][128]
  const uint16_t* v_cache;  // batch 0 layer V base
  long long cache_batch_stride;  // elements between batch rows' caches
  const int* block_table;   // paged KV: [batch][table_stride] page ids; k/v_cache = the layer's
  int table_stride;         // head-0 K/V planes in page 0 (pages kPageElems apart); ids outside
  int n_pages;              // [0, n_pages) read as empty
  uint16_t* out;            // [batch][32][128] bf16
  float* part_o;            // [batch][8][splits][4][128]
  float* part_ml;           // [batch][8][splits][4][2]
  const int* d_seq_len;     // [batch] device seq lens, or nullptr
  int seq_len;              // used when d_seq_len == nullptr (batch must be 1)
  int max_splits;           // splits per kv head cap: kAttnFusedSplits or kAttnSplits (1: the
                            // kernel writes the normalised bf16 output itself)
};
// Splits per (sequence, kv head) for a context of ntiles 64-row tiles: four tiles per split
// (one per wave of the split workgroup) up to the cap.  Device and host must agree on it.
__host__ __device__ inline int attn_decode_splits(int ntiles, int max_splits) {
  const int n = (ntiles + 3) / 4;
  return n < 1 ? 1 : (n < max_splits ? n : max_splits);
}
// The O projection merges the partials itself (up to kAttnFusedMaxCtx).  Every O-projection
// workgroup reads all the slots it merges, so the cap is small: 4 splits up to
// kAttnFusedShortCtx (4 measured 0.5% faster per decode step than 8 at p = 600, and 4% on the
// bs=16 batched step); beyond, 8 (at p = 2047 the 4-split attention took 9.2 us, twice its time
// at p = 600, on 32 CUs).
constexpr int kAttnFusedSplits = 4;
constexpr int kAttnFusedSplitsLong = 8;
constexpr int kAttnFusedShortCtx = 1024;
inline int attn_fused_splits(int max_len) {
  return max_len <= kAttnFusedShortCtx ? kAttnFusedSplits : kAttnFusedSplitsLong;
}
constexpr int kAttnFusedMaxCtx = 4096;  // beyond: merge kernel + up to kAttnSplits splits
constexpr int kAttnDirectMaxCtx = 2048; // batched contexts up to this: one split, output written directly
// merge = also launch the merge kernel (bf16 output in p.out)
int launch_attn_decode(const AttnDecodeParams& p, int batch, bool merge, hipStream_t st);
size_t attn_decode_partials_bytes(int batch);

// ------------------------------------------------------------ elementwise
int launch_emblookup(int rows, const int* ids, const uint16_t* table, uint16_t* out,
                     const int* d_seq_len, int ids_stride, hipStream_t st);
// For a skinny GEMM that normalises its X rows: the sums of squares of rows 0..15 as 4 partials
// per row (ss[m][4]: the row's sum, then zeros; rows >= `rows` all zero).
// Partial sums of squares per row handed to an RMSNorm folded into the next projection: one per
// producer workgroup of a 4096-column skinny GEMM (16 columns each).
constexpr int kNormParts = kHidden / 16;
int launch_rmsnorm_prep(int rows, const uint16_t* x, float* ss, hipStream_t st);
int launch_rmsnorm(int rows, const uint16_t* x, const uint16_t* w, uint16_t* out,
                   hipStream_t st);
int launch_residual_add(size_t n, uint16_t* x, const uint16_t* d, hipStream_t st);
int launch_swiglu(size_t n, const uint16_t* g, const uint16_t* u, uint16_t* out,
                  hipStream_t st);
int launch_rope(int start_pos, int heads, int seq_len, const float* cos, const float* sin,
                const uint16_t* in, uint16_t* out, int is_kv, hipStream_t st);
int launch_softmax(int seq_len, const uint16_t* in, uint16_t* out, int is_row, hipStream_t st);
int launch_fill_synthetic(uint16_t* out, size_t n, uint64_t seed, uint64_t tensor_id,
                          float mean, float std, hipStream_t st);
// Rotate q,k of a [S][6144] QKV block, write k,v to cache rows start..start+S-1
// (or, with d_seq_lens, row t to position d_seq_lens[t]-1 of cache t) and the
// rotated q to q_out [S][4096].
int launch_kv_to_pages(const uint16_t* kv, int first, int n, uint16_t* pages, int n_pages,
                       const int* table, hipStream_t st);
int launch_qkv_rope_scatter(int S, int start_pos, const uint16_t* qkv, const float* cos,
                            const float* sin, uint16_t* q_out, uint16_t* k_cache,
                            uint16_t* v_cache, const int* d_seq_lens, long long cache_stride,
                            hipStream_t st, const int* block_table = nullptr, int n_pages = 0);

// ------------------------------------------------------------ sampling
// Row 0 extras of the argmax: host_tok (mapped pinned memory) receives the token with a
// system-scope store, and when seq is set, tok_buf[*seq] = token and *seq += 1 (the decode step's
// token write-back and position advance).  All optional.
struct ArgmaxTail {
  int* host_tok = nullptr;
  int* tok_buf = nullptr;
  int* seq = nullptr;
};
int launch_argmax_rows(int rows, int vocab, const float* logits, int* out,
                       unsigned long long* slots, unsigned int* counters, hipStream_t st,
                       ArgmaxTail tail = ArgmaxTail{});
int launch_top_p(int rows, int vocab, const float* logits, float temperature, float top_p,
                 uint64_t seed, uint64_t step, int* out, float* ws, hipStream_t st);
// The no-allocation top-p entry point's scratch (k_sampling.hip): rows * vocab <= this many
// floats.  top_p_scratch_init(device) resolves the device address of that device's copy (the
// device must be current; idempotent); top_p_scratch(device) returns it (nullptr before init).
constexpr size_t kTopPScratchFloats = (size_t)IE_TOP_P_NOALLOC_MAX;
constexpr int kTopPNoallocRows = IE_TOP_P_NOALLOC_ROWS;
// the exponentials plus kTopPNoallocRows per-row blocks of the sampler's state (< 128 KiB each)
constexpr size_t kTopPScratchBytes = kTopPScratchFloats * sizeof(float) + (size_t)kTopPNoallocRows * (128 << 10);
// Workspace of launch_top_p: the [rows][vocab] fp32 exponentials (256-byte aligned), then the
// per-row state.
size_t top_p_workspace_bytes(int rows, int vocab);
int top_p_scratch_init(int device);
float* top_p_scratch(int device);

// ------------------------------------------------------------ MFMA GEMM
enum GemmEpi : int {
  kGemmBf16 = 0,    // Y = bf16(acc)
  kGemmResid = 1,   // Y = bf16(Y + bf16(acc))
  kGemmF32 = 2,     // Yf = acc
  kGemmSwiglu = 3,  // Y[:, j] = bf16(silu(bf16(acc_gate)) * bf16(acc_up)) (two weights)
  // QKV projection with RoPE and the K/V cache write (the [q|k|v] weights as w0/w1/w2):
  // bf16(acc), RoPE on q and k, q to y [M][32][128], k and v to the cache (rope.cu:53-64,
  // attn.cu:345-352).  Batched decode (skinny GEMM, M <= 16): row m at position d_seq_len[m] - 1
  // of sequence m's cache.  Prefill (launch_qkv_rope_prefill, the 192 x 256 ping-pong tiles): row
  // m at position start_pos + m of one sequence's cache.
  kGemmQkvRope = 4,
};
struct GemmParams {
  const uint16_t* x;   // [M][K]
  const uint16_t* w0;  // [N][K]    (first N0 rows)
  const uint16_t* w1;  // rows N0..N0+N1 (or the up matrix for SwiGLU)
  const uint16_t* w2;  // rows N0+N1..
  int n0, n1;          // split points for the concatenated-weights view
  uint16_t* y;         // [M][ldy]
  float* yf;           // [M][ldy]
  int M, N, K;
  int ldy;
  // kGemmQkvRope only
  const float* rope_cos;   // [kMaxCtx][64]
  const float* rope_sin;
  uint16_t* k_cache;       // sequence 0's K plane base of this layer [8][kMaxCtx][128]
  uint16_t* v_cache;
  long long cache_stride;  // elements between sequences' caches
  const int* block_table;  // paged KV: [M][table_stride] page ids; k/v_cache = this layer's K/V
  int table_stride;        // head-0 planes of page 0 (pages kPageElems apart); ids outside
  int n_pages;             // [0, n_pages) are not written
  const int* d_seq_len;    // [M] (batched decode)
  int start_pos;           // prefill: position of row 0 (block_table: one sequence's table)
  // Skinny GEMM (M <= 16) only: RMSNorm of the X rows inside the projection (rmsnorm.cu:49-61).
  // Consumer (SwiGLU / QKV + RoPE): x holds the raw rows, x_norm_w the norm weight [K] and ss_in
  // [16][ss_parts] partial sums of squares of the rows (rows past M zero); the product uses the
  // rows as bf16(bf16(x * r) * w), r = rsqrt(sum / K + eps): the reference's two roundings.
  const float* ss_in;
  int ss_parts;
  const uint16_t* x_norm_w;
  // Producer (kGemmResid, N = 16 kNormParts): also writes the sums of squares of each 16
  // columns of the new rows to ss_out[row][n / 16].
  float* ss_out;
  // Split K (bf16 / residual / SwiGLU epilogues, 16 < M <= kSplitMaxRows): scratch for
  // fp32 partial products [splits][M][N]; when set and the tiles would fill at most half the
  // chip, K is split across workgroups and a reduction applies the epilogue.
  float* split_ws;
  long long split_ws_bytes;
  // Residual epilogue with K split, N = 4096: when rn_out is set the reduction also writes
  // rmsnorm(y) with weight rn_w to rn_out (the RMSNorm of the rows that follows the product in
  // the layer) and sets *rn_done; otherwise the caller runs that RMSNorm itself.
  const uint16_t* rn_w;
  uint16_t* rn_out;
  int* rn_done;
  int k_splits;  // set by the launcher for the wide kernel (0 / 1: no split)
  // Skinny GEMM (M <= 16): the last sk_tail of its tiles (16 rows; 32 for the fp32 epilogue
  // at K = 4096 or 14336) run as two workgroups each, one per K half, so that every CU gets the
  // same share of the weight stream (gemm_skinny_split gives the count).  sk_part: fp32
  // partials [sk_tail][2][2][64][4]; sk_cnt: one zeroed arrival counter per tile, kCntStride
  // apart (reset by the tile's finisher).
  float* sk_part;
  unsigned int* sk_cnt;
  int sk_tail;
};
// Bytes of sk_part for up to kSkTailMax split tiles.
constexpr size_t kSkPartBytes = (size_t)kSkTailMax * 2 * 2 * 64 * 4 * sizeof(float);
constexpr int kSplitMaxRows = 1024;
// Scratch bytes split K may use for an M-row product with n output columns (SwiGLU: 2 x the
// output columns): 2048 partial rows, i.e. up to 16 planes at M <= 128, 4 at M = 512.
inline size_t gemm_split_bytes(int M, int n) {
  return M <= kSplitMaxRows ? (size_t)(4 * M > 2048 ? 4 * M : 2048) * n * sizeof(float) : 0;
}
int launch_gemm(int epi, const GemmParams& p, hipStream_t st);
// Prefill QKV projection with RoPE and the K/V scatter in the GEMM epilogue (kGemmQkvRope,
// start_pos): launched when the bf16 product would run as one launch of the 192 x 256
// ping-pong tiles; returns 1 without launching otherwise (the caller then runs the bf16
// product and the scatter kernel, with the same results bit for bit).
int launch_qkv_rope_prefill(const GemmParams& p, hipStream_t st);

// ------------------------------------------------------------ weight arena (engine.hip)
constexpr int kLayerFields = 9;
ie_bf16** layer_field(ie_layer& L, int f);
size_t layer_field_elems(int f);
size_t weights_arena_bytes();
void weights_arena_assign(ie_model_weights* w, void* arena);
int weights_upload_rope(ie_model_weights* w);
// model_weights.cu:80-154 (weights_io.cpp)
int load_safetensors(ie_model_weights* out, const char* const* paths, int n_paths);
// M <= 16 streaming variant (batched decode); launch_gemm routes to it when it fits.
bool gemm_skinny_fits(const GemmParams& p);
int launch_gemm_skinny(int epi, const GemmParams& p, hipStream_t st);
// Tiles of an N-column skinny product to split in K halves (the part of the last round of
// tiles that would leave CUs idle), 0 for none.
int gemm_skinny_tail(int N);
// The same for any skinny epilogue at its own tile size (the fp32 epilogue's 32-row tiles at
// K = 4096 or 14336; 0 for the other plain epilogues).
int gemm_skinny_split(int epi, int N, int K);
// 16 < M <= 48 (short prompts): the streaming kernel over 2-3 X row-blocks
bool gemm_skinny_mb_fits(int epi, const GemmParams& p);
int launch_gemm_skinny_mb(int epi, const GemmParams& p, hipStream_t st);

// ------------------------------------------------------------ prefill attention
struct AttnPrefillParams {
  const uint16_t* q;   // [S][32][128] rotated
  const uint16_t* k;   // layer K plane base [8][8192][128]
  const uint16_t* v;
  uint16_t* out;       // [S][4096]
  int S;
  int start_pos;       // absolute position of q row 0 (keys 0..start_pos+S-1)
  const int* block_table = nullptr;  // paged KV: page of each 64-key block; k / v = the layer's
  int n_pages = 0;                   // head-0 K / V planes in page 0 (ids outside: empty)
};
int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t st);

}  // namespace ie
