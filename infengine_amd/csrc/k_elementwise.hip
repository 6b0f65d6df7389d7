// Row-wise and elementwise kernels: embedding gather, RMSNorm, residual add,
// SwiGLU, RoPE, scaled (causal) softmax, prefill q/k/v scatter, and the
// deterministic synthetic-tensor generator.  All are HBM-bound byte movers:
// 128-bit loads/stores, one 256-thread workgroup per row where a row-wide
// reduction is needed.
#include "ie_kernels.h"

namespace ie {

namespace {

// ---------------------------------------------------------------- emblookup
// emblookup.cu:12-25: out[t, :] = E[ids[t], :].  With d_seq_len set (decode)
// row t gathers ids[t * ids_stride + d_seq_len[t] - 1], the last token of
// sequence t.  Ids outside [0, vocab) produce a zero row instead of an
// out-of-bounds read.
__global__ __launch_bounds__(256) void emblookup_kernel(const int* ids, const uint16_t* table,
                                                        uint16_t* out, const int* d_seq_len,
                                                        int ids_stride) {
  const int t = blockIdx.x;
  const int id = d_seq_len ? ids[(size_t)t * ids_stride + d_seq_len[t] - 1] : ids[t];
  uint4* dst = reinterpret_cast<uint4*>(out + (size_t)t * kHidden);
  if (id < 0 || id >= kVocab) {
    for (int i = threadIdx.x; i < kHidden / 8; i += 256) dst[i] = make_uint4(0, 0, 0, 0);
    return;
  }
  const uint4* src = reinterpret_cast<const uint4*>(table + (size_t)id * kHidden);
  // both loads before either store (the compiler cannot tell the row from the output apart)
  static_assert(kHidden / 8 == 2 * 256, "two 16-byte chunks per thread");
  const uint4 a = src[threadIdx.x], b = src[threadIdx.x + 256];
  dst[threadIdx.x] = a;
  dst[threadIdx.x + 256] = b;
}

// ---------------------------------------------------------------- rmsnorm
// rmsnorm.cu:31-63: fp32 sum of squares, r = rsqrt(mean + 1e-5),
// out = bf16(bf16(x * r) * w).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, const uint16_t* w,
                                                      uint16_t* out) {
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint4* x4 = reinterpret_cast<const uint4*>(x + (size_t)row * kHidden);
  const uint4* w4 = reinterpret_cast<const uint4*>(w);
  uint4 v[2], wv[2];
  // every load up front (the weight's with the row's): one memory latency, not two
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    v[k] = x4[tid + k * 256];
    wv[k] = w4[tid + k * 256];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ss = fmaf(bf_lo(e[q]), bf_lo(e[q]), ss);
      ss = fmaf(bf_hi(e[q]), bf_hi(e[q]), ss);
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float r = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)kHidden + kRmsEps);
  uint4* o4 = reinterpret_cast<uint4*>(out + (size_t)row * kHidden);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
    const uint32_t f[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = bf2f(f2bf(bf_lo(e[q]) * r)) * bf_lo(f[q]);
      const float hi = bf2f(f2bf(bf_hi(e[q]) * r)) * bf_hi(f[q]);
      o[q] = pack_bf2(lo, hi);
    }
    o4[tid + k * 256] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---------------------------------------------------------------- residual / swiglu
__global__ void residual_add_kernel(uint16_t* x, const uint16_t* d, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t n8 = n / 8;
  if (i < n8) {
    uint4 a = reinterpret_cast<uint4*>(x)[i];
    const uint4 b = reinterpret_cast<const uint4*>(d)[i];
    a.x = pack_bf2(bf_lo(a.x) + bf_lo(b.x), bf_hi(a.x) + bf_hi(b.x));
    a.y = pack_bf2(bf_lo(a.y) + bf_lo(b.y), bf_hi(a.y) + bf_hi(b.y));
    a.z = pack_bf2(bf_lo(a.z) + bf_lo(b.z), bf_hi(a.z) + bf_hi(b.z));
    a.w = pack_bf2(bf_lo(a.w) + bf_lo(b.w), bf_hi(a.w) + bf_hi(b.w));
    reinterpret_cast<uint4*>(x)[i] = a;
  } else if (i == n8) {
    for (size_t j = n8 * 8; j < n; ++j) x[j] = f2bf(bf2f(x[j]) + bf2f(d[j]));
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * (1.0f / (1.0f + expf(-g))) * u;
}

__global__ void swiglu_kernel(const uint16_t* g, const uint16_t* u, uint16_t* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t n8 = n / 8;
  if (i < n8) {
    const uint4 a = reinterpret_cast<const uint4*>(g)[i];
    const uint4 b = reinterpret_cast<const uint4*>(u)[i];
    uint4 o;
    o.x = pack_bf2(silu_mul(bf_lo(a.x), bf_lo(b.x)), silu_mul(bf_hi(a.x), bf_hi(b.x)));
    o.y = pack_bf2(silu_mul(bf_lo(a.y), bf_lo(b.y)), silu_mul(bf_hi(a.y), bf_hi(b.y)));
    o.z = pack_bf2(silu_mul(bf_lo(a.z), bf_lo(b.z)), silu_mul(bf_hi(a.z), bf_hi(b.z)));
    o.w = pack_bf2(silu_mul(bf_lo(a.w), bf_lo(b.w)), silu_mul(bf_hi(a.w), bf_hi(b.w)));
    reinterpret_cast<uint4*>(out)[i] = o;
  } else if (i == n8) {
    for (size_t j = n8 * 8; j < n; ++j) out[j] = f2bf(silu_mul(bf2f(g[j]), bf2f(u[j])));
  }
}

// ---------------------------------------------------------------- rope
// rope.cu:30-66: block per (head, token), lane j rotates the pair (j, j+64)
// with angle table[pos][j]; heads are strided by 8192 rows when is_kv.
__global__ __launch_bounds__(64) void rope_kernel(int start_pos, int seq_len, const float* cos_t,
                                                  const float* sin_t, const uint16_t* in,
                                                  uint16_t* out, int is_kv) {
  const int head = blockIdx.x / seq_len, tok = blockIdx.x % seq_len, j = threadIdx.x;
  const size_t off = ((size_t)head * (is_kv ? kMaxCtx : seq_len) + tok) * kHeadDim;
  const int pos = start_pos + tok;
  const float c = cos_t[pos * 64 + j], s = sin_t[pos * 64 + j];
  const float a = bf2f(in[off + j]), b = bf2f(in[off + j + 64]);
  out[off + j] = f2bf(rope_lo(a, b, c, s));
  out[off + j + 64] = f2bf(rope_hi(a, b, c, s));
}

// ---------------------------------------------------------------- prefill q/k/v scatter
// One block per token row of the fused [S][6144] projection: q heads are
// rotated into q_out [S][32][128], k heads rotated into the cache, v copied.
// Same pairing and rounding as rope.cu:53-64 and attn.cu:345-352.  Row t sits at
// position start_pos + t of one cache, or (d_seq_lens set: batched decode) at
// position d_seq_lens[t] - 1 of cache t, cache_stride elements apart.
__global__ __launch_bounds__(256) void qkv_rope_scatter_kernel(int start_pos, const uint16_t* qkv,
                                                               const float* cos_t,
                                                               const float* sin_t,
                                                               uint16_t* q_out, uint16_t* kc,
                                                               uint16_t* vc,
                                                               const int* d_seq_lens,
                                                               long long cache_stride,
                                                               const int* block_table,
                                                               int n_pages) {
  const int t = blockIdx.x;
  const int pos = d_seq_lens ? d_seq_lens[t] - 1 : start_pos + t;
  if (d_seq_lens) {
    kc += (size_t)t * cache_stride;
    vc += (size_t)t * cache_stride;
  }
  const uint16_t* src = qkv + (size_t)t * kQKVDim;
  // 48 heads x 64 pairs = 3072 pairs; 256 threads -> 12 pairs each
  for (int pr = threadIdx.x; pr < (kQHeads + 2 * kKVHeads) * 64; pr += 256) {
    const int head = pr >> 6, j = pr & 63;
    const uint16_t* hs = src + head * kHeadDim;
    float a = bf2f(hs[j]), b = bf2f(hs[j + 64]);
    if (head < kQHeads + kKVHeads) {
      const float c = cos_t[pos * 64 + j], s = sin_t[pos * 64 + j];
      const float a2 = rope_lo(a, b, c, s), b2 = rope_hi(a, b, c, s);
      a = a2;
      b = b2;
    }
    uint16_t* dst;
    if (head < kQHeads) {
      dst = q_out + ((size_t)t * kQHeads + head) * kHeadDim;
    } else {
      const bool is_k = head < kQHeads + kKVHeads;
      const int kvh = head - kQHeads - (is_k ? 0 : kKVHeads);
      uint16_t* const plane = is_k ? kc : vc;
      if (block_table) {  // paged: row pos % kPagePos of the page holding block pos / kPagePos
        const int page = block_table[pos / kPagePos];
        if (page < 0 || page >= n_pages) continue;
        dst = plane + (size_t)page * kPageElems + ((size_t)kvh * kPagePos + pos % kPagePos) * kHeadDim;
      } else {
        dst = plane + ((size_t)kvh * kMaxCtx + pos) * kHeadDim;
      }
    }
    dst[j] = f2bf(a);
    dst[j + 64] = f2bf(b);
  }
}

// ---------------------------------------------------------------- contiguous cache -> pages
// Positions [first, first + n) of every (layer, K|V, kv head) plane of a reference-layout cache
// into the pages of one sequence's block table; 16 bytes per thread.  Page ids outside
// [0, n_pages) are skipped.
__global__ __launch_bounds__(256) void kv_to_pages_kernel(const uint16_t* kv, int first, int n,
                                                          uint16_t* pages, int n_pages,
                                                          const int* table) {
  constexpr int kPlanes = kLayers * 2 * kKVHeads;
  const size_t total = (size_t)n * kPlanes * 16;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(i & 15);
    const size_t rest = i >> 4;
    const int plane = (int)(rest % kPlanes);
    const int pos = first + (int)(rest / kPlanes);
    const int page = table[pos / kPagePos];
    if (page < 0 || page >= n_pages) continue;
    const u32x4_t v =
        *reinterpret_cast<const u32x4_t*>(kv + ((size_t)plane * kMaxCtx + pos) * kHeadDim + 8 * c);
    *reinterpret_cast<u32x4_t*>(pages + (size_t)page * kPageElems +
                                ((size_t)plane * kPagePos + pos % kPagePos) * kHeadDim + 8 * c) = v;
  }
}

// ---------------------------------------------------------------- softmax
// softmax.cu:55-160: softmax(x / sqrt(128)) per row, entries right of the
// diagonal masked (causal) and written as 0.  fp32 throughout.
__global__ __launch_bounds__(256) void softmax_kernel(int seq_len, const uint16_t* in,
                                                      uint16_t* out, int causal) {
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int valid = causal ? (row % seq_len) + 1 : seq_len;
  const uint16_t* x = in + (size_t)row * seq_len;
  uint16_t* y = out + (size_t)row * seq_len;
  const float scale = 0.08838834764831845f;
  float mx = -INFINITY;
  for (int i = tid; i < valid; i += 256) mx = fmaxf(mx, bf2f(x[i]) * scale);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int i = tid; i < valid; i += 256) sum += expf(bf2f(x[i]) * scale - mx);
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  const float inv = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
  for (int i = tid; i < seq_len; i += 256)
    y[i] = (i < valid) ? f2bf(expf(bf2f(x[i]) * scale - mx) * inv) : (uint16_t)0;
}

// ---------------------------------------------------------------- synthetic data
__global__ void fill_synthetic_kernel(uint16_t* out, size_t n, uint64_t base, float mean,
                                      float scale) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int c = synth_centered(base, i);
    out[i] = f2bf(__builtin_fmaf((float)c, scale, mean));
  }
}

}  // namespace

int launch_emblookup(int rows, const int* ids, const uint16_t* table, uint16_t* out,
                     const int* d_seq_len, int ids_stride, hipStream_t st) {
  IE_REQUIRE(rows >= 1, "emblookup: rows=%d", rows);
  hipLaunchKernelGGL(emblookup_kernel, dim3(rows), dim3(256), 0, st, ids, table, out, d_seq_len,
                     ids_stride);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

// One block per row of 16 (rows past `rows` write zero sums); thread t writes partial t, the
// sum of squares of columns 16t .. 16t+15 exactly as the skinny GEMM's residual epilogue forms
// it for its 16-column tile t (lane group q's four columns 16t + 4q .. +3 as one fma chain, then
// (q0 + q1) + (q2 + q3)), so a step's later layers, which read that epilogue's partials, and a
// layer started from this kernel see the same bits.
static_assert(kNormParts == 256 && kNormParts * 16 == kHidden, "one 16-column partial per thread");
__global__ __launch_bounds__(256) void rmsnorm_prep_kernel(int rows, const uint16_t* x,
                                                           float* ss) {
  const int row = blockIdx.x, tid = threadIdx.x;
  float part = 0.f;
  if (row < rows) {
    const uint4* x4 = reinterpret_cast<const uint4*>(x + (size_t)row * kHidden + 16 * tid);
    const uint4 a = x4[0], b = x4[1];
    const uint32_t e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float sq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float v0 = bf_lo(e[2 * q]), v1 = bf_hi(e[2 * q]), v2 = bf_lo(e[2 * q + 1]),
                  v3 = bf_hi(e[2 * q + 1]);
      sq[q] = fmaf(v0, v0, fmaf(v1, v1, fmaf(v2, v2, v3 * v3)));
    }
    part = (sq[0] + sq[1]) + (sq[2] + sq[3]);
  }
  ss[row * kNormParts + tid] = part;
}

int launch_rmsnorm_prep(int rows, const uint16_t* x, float* ss, hipStream_t st) {
  IE_REQUIRE(rows >= 1 && rows <= 16, "rmsnorm_prep: rows %d out of [1, 16]", rows);
  hipLaunchKernelGGL(rmsnorm_prep_kernel, dim3(16), dim3(256), 0, st, rows, x, ss);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_rmsnorm(int rows, const uint16_t* x, const uint16_t* w, uint16_t* out,
                   hipStream_t st) {
  IE_REQUIRE(rows >= 1, "rmsnorm: rows=%d", rows);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, st, x, w, out);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_residual_add(size_t n, uint16_t* x, const uint16_t* d, hipStream_t st) {
  if (n == 0) return IE_OK;
  const size_t threads = n / 8 + 1;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, x, d, n);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_swiglu(size_t n, const uint16_t* g, const uint16_t* u, uint16_t* out,
                  hipStream_t st) {
  if (n == 0) return IE_OK;
  const size_t threads = n / 8 + 1;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, g,
                     u, out, n);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_rope(int start_pos, int heads, int seq_len, const float* cos, const float* sin,
                const uint16_t* in, uint16_t* out, int is_kv, hipStream_t st) {
  IE_REQUIRE(heads >= 1 && seq_len >= 1, "rope: heads=%d seq_len=%d", heads, seq_len);
  IE_REQUIRE(start_pos >= 0 && start_pos + seq_len <= kMaxCtx,
             "rope: positions [%d, %d) exceed the %d-row table", start_pos, start_pos + seq_len,
             kMaxCtx);
  hipLaunchKernelGGL(rope_kernel, dim3(heads * seq_len), dim3(64), 0, st, start_pos, seq_len, cos,
                     sin, in, out, is_kv);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_kv_to_pages(const uint16_t* kv, int first, int n, uint16_t* pages, int n_pages,
                       const int* table, hipStream_t st) {
  IE_REQUIRE(kv && pages && table && n_pages >= 1, "kv_to_pages: null buffer");
  IE_REQUIRE(first >= 0 && n >= 0 && first + n <= kMaxCtx, "kv_to_pages: positions [%d, %d)",
             first, first + n);
  if (n == 0) return IE_OK;
  const size_t total = (size_t)n * kLayers * 2 * kKVHeads * 16;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(kv_to_pages_kernel, dim3(blocks), dim3(256), 0, st, kv, first, n, pages,
                     n_pages, table);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_qkv_rope_scatter(int S, int start_pos, const uint16_t* qkv, const float* cos,
                            const float* sin, uint16_t* q_out, uint16_t* k_cache,
                            uint16_t* v_cache, const int* d_seq_lens, long long cache_stride,
                            hipStream_t st, const int* block_table, int n_pages) {
  IE_REQUIRE(S >= 1 && start_pos >= 0 &&
                 (d_seq_lens || start_pos + S <= (block_table ? kMaxLongCtx : kMaxCtx)),
             "qkv scatter: rows [%d, %d) exceed the KV cache", start_pos, start_pos + S);
  IE_REQUIRE(!block_table || !d_seq_lens, "qkv scatter: paged rows are one sequence's");
  hipLaunchKernelGGL(qkv_rope_scatter_kernel, dim3(S), dim3(256), 0, st, start_pos, qkv, cos, sin,
                     q_out, k_cache, v_cache, d_seq_lens, cache_stride, block_table, n_pages);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_softmax(int seq_len, const uint16_t* in, uint16_t* out, int is_row, hipStream_t st) {
  IE_REQUIRE(seq_len >= 1, "softmax: seq_len=%d", seq_len);
  const int rows = is_row ? kQHeads : kQHeads * seq_len;
  hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, st, seq_len, in, out,
                     is_row ? 0 : 1);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_fill_synthetic(uint16_t* out, size_t n, uint64_t seed, uint64_t tensor_id,
                          float mean, float std, hipStream_t st) {
  if (n == 0) return IE_OK;
  const float scale = (float)((double)std / kSynthStd);
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_synthetic_kernel, dim3((unsigned)blocks), dim3(256), 0, st, out, n,
                     synth_base(seed, tensor_id), mean, scale);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
