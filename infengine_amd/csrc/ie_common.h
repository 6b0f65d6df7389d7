// Shared device helpers, error plumbing and the engine context for the gfx950
// hot path.  bf16 values travel as raw uint16_t; conversions are explicit so the
// rounding points are the same as the CPU oracle's (round-to-nearest-even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "infengine.h"

namespace ie {

constexpr int kMaxCtx = IE_MAX_CONTEXT_LENGTH;       // reference-layout KV cache positions
constexpr int kMaxLongCtx = IE_MAX_LONG_CONTEXT;    // paged KV paths and RoPE table rows
constexpr int kVocab = IE_VOCAB_SIZE;
constexpr int kLayers = IE_NUM_LAYERS;
constexpr int kHidden = IE_HIDDEN_SIZE;
constexpr int kQHeads = IE_NUM_Q_HEADS;
constexpr int kKVHeads = IE_NUM_KV_HEADS;
constexpr int kHeadDim = IE_HEAD_DIM;
constexpr int kFFN = IE_FFN_DIM;
constexpr int kGQA = kQHeads / kKVHeads;             // q heads per kv head (attn.cu:51-53)
constexpr int kKVDim = kKVHeads * kHeadDim;          // 1024
constexpr int kQKVDim = kHidden + 2 * kKVDim;        // 6144
constexpr float kRmsEps = 1e-5f;                     // rmsnorm.cu:5
// Per-layer KV-cache plane: [2][8][8192][128] (attn.cu:304-307, 334-337).
constexpr size_t kKVPlane = (size_t)kMaxCtx * kHeadDim;              // one head, K or V
constexpr size_t kKVLayer = 2 * (size_t)kKVHeads * kKVPlane;         // elements per layer
// Paged KV cache: a page holds kPagePos positions of every layer, [layer][K|V][kv head]
// [kPagePos][128] bf16; a sequence's block table maps position block i (positions
// kPagePos*i ..) to a page.
constexpr int kPagePos = 64;
constexpr size_t kPageHead = (size_t)kPagePos * kHeadDim;              // one head, K or V
constexpr size_t kPageLayer = 2 * (size_t)kKVHeads * kPageHead;        // one layer in a page
constexpr size_t kPageElems = (size_t)kLayers * kPageLayer;            // elements per page

// Decode attention splits the context of each KV head over this many blocks.
constexpr int kAttnSplits = 32;
constexpr int kAttnTile = 64;

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* get_error();

#define IE_CHECK_HIP(expr)                                                              \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess) {                                                             \
      ::ie::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                      __LINE__);                                                        \
      return IE_ERR_HIP;                                                                \
    }                                                                                   \
  } while (0)

#define IE_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      ::ie::set_error(__VA_ARGS__);    \
      return IE_ERR_INVALID_ARG;       \
    }                                  \
  } while (0)

#define IE_CHECK_LAUNCH()                                                                \
  do {                                                                                   \
    hipError_t _e = hipGetLastError();                                                   \
    if (_e != hipSuccess) {                                                              \
      ::ie::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(_e), __FILE__, \
                      __LINE__);                                                         \
      return IE_ERR_HIP;                                                                 \
    }                                                                                    \
  } while (0)

#define IE_TRY(expr)             \
  do {                           \
    int _rc = (expr);            \
    if (_rc < 0) return _rc;     \
  } while (0)

// ---------------------------------------------------------------- bf16
__host__ __device__ __forceinline__ float bf2f(uint16_t h) {
  union { uint32_t u; float f; } c;
  c.u = (uint32_t)h << 16;
  return c.f;
}

__host__ __device__ __forceinline__ uint16_t f2bf(float f) {
  union { uint32_t u; float f; } c;
  c.f = f;
  uint32_t u = c.u;
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to bf16 in one gfx950 v_cvt_pk_bf16_f32 (round to nearest even, as f2bf; NaN becomes
// a quiet NaN).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// acc + a.lo*b.lo + a.hi*b.hi on the gfx950 dot2 unit (bf16 inputs, fp32 accumulate)
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

__device__ __forceinline__ float dot8(const uint4& w, const uint4& x, float acc) {
  acc = dot2(w.x, x.x, acc);
  acc = dot2(w.y, x.y, acc);
  acc = dot2(w.z, x.z, acc);
  acc = dot2(w.w, x.w, acc);
  return acc;
}

// RoPE of the pair (a, b) = (x_j, x_{j+64}) by angle (c, s) = (cos, sin) (rope.cu:59-64):
// a c - b s and a s + b c, each as one fused multiply-add over the other product, so the result
// does not depend on which product the compiler would have contracted (nvcc, compiling the
// reference, contracts a*b - c*d the same way by default).
__host__ __device__ __forceinline__ float rope_lo(float a, float b, float c, float s) {
  return fmaf(a, c, -(b * s));
}
__host__ __device__ __forceinline__ float rope_hi(float a, float b, float c, float s) {
  return fmaf(a, s, b * c);
}

// Native 4 x u32 vector.  Register arrays use it instead of HIP's uint4 (a
// struct with a union, which SROA does not split into registers).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot8(const u32x4_t& w, const u32x4_t& x, float acc) {
  acc = dot2(w[0], x[0], acc);
  acc = dot2(w[1], x[1], acc);
  acc = dot2(w[2], x[2], acc);
  acc = dot2(w[3], x[3], acc);
  return acc;
}

// Streaming (non-temporal) 128-bit load for data read exactly once.
__device__ __forceinline__ u32x4_t ld_stream(const u32x4_t* p) {
  return __builtin_nontemporal_load(p);
}

// ---------------------------------------------------------------- wave reductions
// DPP controls (GCN3+ encoding): quad_perm, row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each 16-lane row; every lane of the row receives the row's sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  return v;
}

// x[l] op x[l ^ 16] and x[l] op x[l ^ 32] on every lane, with gfx950's v_permlane16_swap /
// v_permlane32_swap given x twice: the two results hold x[l & ~m] and x[l | m] (measured on the
// device), so one VALU swap replaces an LDS-crossbar shuffle, and both lanes of a pair combine
// the same two values in the same order.
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wave64 sum; the result is uniform across the wave.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
               fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// ---------------------------------------------------------------- synthetic data
// splitmix64 finaliser (Steele, Lea, Flood 2014).
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__host__ __device__ __forceinline__ uint64_t synth_base(uint64_t seed, uint64_t tensor_id) {
  return splitmix64(splitmix64(seed) ^ (tensor_id * 0xD1B54A32D192ED03ull));
}

// Integer-exact approximate standard normal: centred sum of four uniform
// 16-bit draws (Irwin-Hall, n=4), returned as an exact integer in [-131070, 131070].
__host__ __device__ __forceinline__ int synth_centered(uint64_t base, uint64_t index) {
  uint64_t h = splitmix64(base + index);
  int s = (int)(h & 0xFFFF) + (int)((h >> 16) & 0xFFFF) + (int)((h >> 32) & 0xFFFF) +
          (int)(h >> 48);
  return s - 131070;
}
// Standard deviation of synth_centered: sqrt(4 * (65536^2 - 1) / 12).
constexpr double kSynthStd = 37837.22627754049;

// ---------------------------------------------------------------- context
struct Context {
  int device = 0;
  hipStream_t stream = nullptr;    // nullptr = the legacy default stream
  hipStream_t capture = nullptr;   // private stream the decode graph is captured on
  unsigned int* d_counters = nullptr;       // self-resetting last-block counters
  unsigned long long* d_slots = nullptr;    // 64-bit reduction slots (argmax)
  int* d_params = nullptr;                  // device copy of per-step scalars
  int* h_params = nullptr;                  // pinned staging for d_params
  int* h_token = nullptr;                   // pinned, mapped token read-back
  int* h_token_dev = nullptr;               // device address of h_token (the argmax writes it)
  int next_seq = -1;                        // d_params[0] as the last decode step left it
  bool use_graph = true;
  // captured decode-step graph and the arguments it was captured with
  hipGraphExec_t graph_exec = nullptr;
  const void* graph_key[12] = {};
  // captured batched steps, least recently used replaced first (a serving loop alternates
  // between a few batch compositions)
  struct BatchGraph {
    hipGraphExec_t exec = nullptr;
    const void* key[16] = {};
    unsigned long long used = 0;
  } bgraph[4];
  unsigned long long bgraph_tick = 0;
  // the skinny GEMM's K-half partials (kSkPartBytes) for launches outside the batched step
  float* d_sk_part = nullptr;
  // split-K partials of the op-level GEMM entry (allocated on first use)
  float* gemm_ws = nullptr;
  size_t gemm_ws_bytes = 0;
};

// Per-row reduction state sits one 128-byte line apart: device-scope atomics on one line
// serialise (the bs=16 argmax, 64 workgroups per row, took 15.5 us with the 16 rows' slots and
// counters on 3 lines, 5.4 us with a line per row).
constexpr int kSlotStride = 16;  // 64-bit slots per row
constexpr int kCntStride = 32;   // 32-bit counters per row
constexpr int kNumSlots = 64;
// Counter bank offsets.
constexpr int kCntArgmax = 0;  // [64][kCntStride] argmax rows
// The skinny GEMM's split tail tiles: one arrival counter per tile (two K halves), at most
// kSkTailMax tiles per launch.
constexpr int kSkTailMax = 256;
constexpr int kCntSkinny = kCntArgmax + kNumSlots * kCntStride;  // [kSkTailMax][kCntStride]
constexpr int kNumCounters = kCntSkinny + kSkTailMax * kCntStride;

inline hipStream_t stream_of(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace ie
