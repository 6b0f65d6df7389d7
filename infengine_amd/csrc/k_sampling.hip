// Token selection over fp32 logits.
//
// argmax — reference sample_token_amax (kernels/sampling.cu:28-58) is a single
// 1024-thread block whose tie rule depends on thread layout.  Here the rule is
// torch.argmax's: the largest value wins, ties go to the smallest index, NaN
// counts as larger than everything, -0.0 equals +0.0.  Each (value, index) is
// packed into one 64-bit key whose unsigned order is exactly that rule, so the
// reduction is a plain max: per-workgroup max, then a device-scope atomicMax
// into a slot; the last workgroup of a row (counter) reads and clears the slot.
//
// top-p — no reference counterpart (the reference samples greedily).  The kept
// set follows HF TopPLogitsWarper (logits/T, drop the ascending-cumulative mass
// <= 1-p, keep >= 1 token): token i is kept iff the probability mass of tokens
// with a strictly larger scaled logit is < p.  Masses are exp(l/T - max) in
// fixed point (2^-40 units, uint64), so every sum is exact and order-free:
//   1. max of l/T; e_i = expf(l_i/T - max) cached in the workspace; Z = sum q_i
//   2. the cut key kappa with mass(key > kappa) < target <= mass(key >= kappa): the positive
//      masses binned by distance to the max locate its bin, then a radix select (4 x 8-bit
//      digits of the order-preserving key of l_i/T) over that bin's tokens
//   3. Z_kept = mass(key >= kappa); t = floor(Z_kept * u), u a 24-bit counter-RNG
//      uniform of (seed, row, step)
//   4. the sampled token is the smallest id whose kept prefix mass exceeds t
//      (inverse CDF in token-id order), found with a block-wide exclusive scan.
#include <mutex>

#include "ie_kernels.h"

namespace ie {

namespace {

__device__ __forceinline__ uint32_t order_key(float v) {
  if (v != v) return 0xFFFFFFFFu;
  if (v == 0.f) v = 0.f;
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned idx) {
  return ((unsigned long long)order_key(v) << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

constexpr int kArgmaxBlocks = 64;

__global__ __launch_bounds__(256) void argmax_kernel(const float* logits, int vocab, int* out,
                                                     unsigned long long* slots,
                                                     unsigned int* counters, ArgmaxTail tail) {
  __shared__ unsigned long long red[4];
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* L = logits + (size_t)row * vocab;
  const int chunk = (vocab + gridDim.x - 1) / gridDim.x;
  const int beg = blockIdx.x * chunk;
  const int end = min(vocab, beg + chunk);
  unsigned long long best = 0ull;
  // 8 loads in flight per thread per round (a chunk of the 128256-entry vocabulary is one
  // round): indices past the chunk load its last element and count as key 0
  for (int i0 = beg + tid; i0 < end; i0 += 8 * 256) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = L[min(i0 + u * 256, end - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 256;
      // (masked arithmetically: a select let the compiler move a load under a branch)
      const unsigned long long k =
          argmax_key(v[u], (unsigned)i) & (0ull - (unsigned long long)(i < end));
      best = k > best ? k : best;
    }
  }
  best = wave_max_u64(best);
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (tid == 0) {
    unsigned long long b = red[0];
    for (int w = 1; w < 4; ++w) b = red[w] > b ? red[w] : b;
    // Device-scope atomics on one address are coherent across the XCDs; waiting for the max
    // to be performed before counting in orders the two, so the workgroup that counts last
    // exchanges out the final max.  (No __threadfence: on this part it writes back the L2.)
    unsigned long long* slot = slots + row * kSlotStride;
    unsigned int* counter = counters + row * kCntStride;
    atomicMax(slot, b);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (atomicAdd(counter, 1u) == gridDim.x - 1) {
      const unsigned long long fin = atomicExch(slot, 0ull);
      const int tok = (int)(0xFFFFFFFFu - (unsigned)(fin & 0xFFFFFFFFull));
      out[row] = tok;
      atomicExch(counter, 0u);
      if (row == 0) {
        if (tail.host_tok)
          __hip_atomic_store(tail.host_tok, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (tail.seq) {
          const int s = *tail.seq;
          if (tail.tok_buf) tail.tok_buf[s] = tok;
          *tail.seq = s + 1;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- top-p
constexpr int kTopPThreads = 1024;
constexpr float kFix = 1099511627776.0f;  // 2^40

__device__ __forceinline__ unsigned long long fix_mass(float e) {
  return (unsigned long long)(e * kFix);
}

template <typename T>
__device__ __forceinline__ T wave_sum_u64(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Tokens with a positive fixed-point mass lie within 28 nats of the largest scaled logit
// (exp(-27.8) * 2^40 < 1), and only they can be kept (the cut token has positive mass, and every
// zero-mass token's key is below its key).  They are binned by their distance d = max - l/T into
// kTopPBins bins: bin(d) is non-decreasing in d, so every key of a lower bin is strictly larger
// than every key of a higher one and equal keys share a bin.  The bin where the cumulative mass
// from the top reaches the target holds the cut; the radix select runs over its tokens only.
//
// Each row is split into kTopPChunks chunks, one workgroup each, over six launches (the row's
// state, histogram and candidates sit in a TopPRow after the exponentials in the workspace):
//   tp_max     chunk maxima of l (the max of l/T is fl(max l / T): division by T > 0 is
//              monotone); the row's histogram and candidate count are cleared
//   tp_hist    e = expf(l/T - max) (cached), chunk mass, the chunk's positive masses binned in
//              LDS and added to the row's histogram
//   tp_gather  every workgroup scans the histogram for the cut bin (identical results), then
//              appends its chunk's tokens of that bin to the candidates
//   tp_select  one workgroup per row: radix select of the cut key over the candidates (over the
//              row's tokens of the cut bin when there are more than kTopPCandMax)
//   tp_kept    chunk masses of the kept tokens
//   tp_walk    one workgroup per row: t from the kept total, the chunk holding t, then its
//              token by a scan over the chunk in token-id order
constexpr int kTopPBins = 2048;
constexpr float kTopPBinScale = kTopPBins / 28.0f;
constexpr int kTopPChunks = 64;
constexpr int kTopPChunkThreads = 256;
constexpr int kTopPCandMax = 8192;

struct TopPRow {
  unsigned long long hist[kTopPBins];
  unsigned long long zpart[kTopPChunks];
  unsigned long long kpart[kTopPChunks];
  float pmax[kTopPChunks];
  unsigned int ncand;
  int bcut;
  uint32_t kappa;
  unsigned int pad;
  unsigned long long above, target;
  uint32_t cand_key[kTopPCandMax];
  unsigned long long cand_q[kTopPCandMax];
};

__device__ __forceinline__ int top_p_bin(float d) {
  return min(kTopPBins - 1, (int)(d * kTopPBinScale));
}

__device__ __forceinline__ int tp_chunk_len(int vocab) {
  return (vocab + kTopPChunks - 1) / kTopPChunks;
}

// Block-wide sum / max for kTopPChunkThreads threads (red: 4 entries).
__device__ __forceinline__ unsigned long long tp_block_sum(unsigned long long v,
                                                           unsigned long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One 256-bin digit step of the radix select (wave 0): the highest digit whose cumulative mass
// from the top reaches t_rem; sets *bin and *above (the mass of the digits above it).
__device__ __forceinline__ void top_p_digit(const unsigned long long* hist, unsigned long long t_rem,
                                            int* s_bin, unsigned long long* s_above) {
  const int lane = threadIdx.x & 63;
  // lane l owns bins 255-4l .. 252-4l (descending digit order)
  unsigned long long hb[4], loc = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hb[j] = hist[255 - 4 * lane - j];
    loc += hb[j];
  }
  unsigned long long inc = loc;  // inclusive scan over lanes
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  const unsigned long long exc = inc - loc;
  const unsigned long long hit = __ballot(inc >= t_rem);
  const int first = hit ? __ffsll((long long)hit) - 1 : 63;
  if (lane == first) {
    unsigned long long cum = exc;
    int bin = 252 - 4 * lane;
    unsigned long long above = cum;
    for (int j = 0; j < 4; ++j) {
      if (cum + hb[j] >= t_rem || j == 3) {
        bin = 255 - 4 * lane - j;
        above = cum;
        break;
      }
      cum += hb[j];
    }
    *s_bin = bin;
    *s_above = above;
  }
}

__global__ __launch_bounds__(kTopPChunkThreads) void tp_max_kernel(const float* logits, int vocab,
                                                                   TopPRow* rows) {
  __shared__ float redf[4];
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  TopPRow& R = rows[row];
  const float* L = logits + (size_t)row * vocab;
  const int cl = tp_chunk_len(vocab), beg = c * cl, end = min(vocab, beg + cl);
  for (int b = c * (kTopPBins / kTopPChunks) + tid; b < (c + 1) * (kTopPBins / kTopPChunks);
       b += kTopPChunkThreads)
    R.hist[b] = 0;
  if (c == 0 && tid == 0) R.ncand = 0;
  float m = -INFINITY;
  for (int i = beg + tid; i < end; i += kTopPChunkThreads) m = fmaxf(m, L[i]);
  m = wave_max(m);
  if (lane == 0) redf[wave] = m;
  __syncthreads();
  if (tid == 0) R.pmax[c] = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
}

__device__ __forceinline__ float tp_row_max(const TopPRow& R, float temperature) {
  float m = R.pmax[0];
  for (int c = 1; c < kTopPChunks; ++c) m = fmaxf(m, R.pmax[c]);
  return m / temperature;
}

__global__ __launch_bounds__(kTopPChunkThreads) void tp_hist_kernel(const float* logits, int vocab,
                                                                    float temperature, TopPRow* rows,
                                                                    float* ws) {
  __shared__ unsigned long long hist[kTopPBins];
  __shared__ unsigned long long red[4];
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  TopPRow& R = rows[row];
  const float* L = logits + (size_t)row * vocab;
  float* E = ws + (size_t)row * vocab;
  const int cl = tp_chunk_len(vocab), beg = c * cl, end = min(vocab, beg + cl);
  const float mx = tp_row_max(R, temperature);
  for (int b = tid; b < kTopPBins; b += kTopPChunkThreads) hist[b] = 0;
  __syncthreads();
  unsigned long long z = 0;
  for (int i = beg + tid; i < end; i += kTopPChunkThreads) {
    const float sv = L[i] / temperature;
    const float e = expf(sv - mx);
    E[i] = e;
    const unsigned long long q = fix_mass(e);
    z += q;
    if (q) atomicAdd(&hist[top_p_bin(mx - sv)], q);
  }
  z = tp_block_sum(z, red);
  if (tid == 0) R.zpart[c] = z;
  for (int b = tid; b < kTopPBins; b += kTopPChunkThreads)
    if (hist[b]) atomicAdd(&R.hist[b], hist[b]);
}

__global__ __launch_bounds__(kTopPChunkThreads) void tp_gather_kernel(const float* logits, int vocab,
                                                                      float temperature, float top_p,
                                                                      TopPRow* rows, const float* ws) {
  __shared__ unsigned long long red[4];
  __shared__ int s_bin;
  __shared__ unsigned long long s_above;
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  TopPRow& R = rows[row];
  const float* L = logits + (size_t)row * vocab;
  const float* E = ws + (size_t)row * vocab;
  const int cl = tp_chunk_len(vocab), beg = c * cl, end = min(vocab, beg + cl);
  const float mx = tp_row_max(R, temperature);
  unsigned long long z = 0;
  for (int j = 0; j < kTopPChunks; ++j) z += R.zpart[j];
  unsigned long long target = (unsigned long long)((double)z * (double)top_p);
  if (target < 1) target = 1;
  // the cut bin: thread t owns bins 8 t .. 8 t + 7 (ascending distance), block inclusive scan
  unsigned long long hb[8], loc = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    hb[j] = R.hist[8 * tid + j];
    loc += hb[j];
  }
  unsigned long long inc = loc;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  if (lane == 63) red[wave] = inc;
  if (tid == 0) s_bin = -1;
  __syncthreads();
  unsigned long long wb = 0;
  for (int w = 0; w < wave; ++w) wb += red[w];
  inc += wb;
  const unsigned long long exc = inc - loc;
  if (exc < target && inc >= target) {  // exactly one thread
    unsigned long long cum = exc;
    int bin = 8 * tid + 7;
    for (int j = 0; j < 8; ++j) {
      if (cum + hb[j] >= target) {
        bin = 8 * tid + j;
        break;
      }
      cum += hb[j];
    }
    s_bin = bin;
    s_above = cum;
  }
  __syncthreads();
  const int bcut = s_bin;
  if (c == 0 && tid == 0) {
    R.bcut = bcut;
    R.above = s_above;
    R.target = target;
  }
  for (int i = beg + tid; i < end; i += kTopPChunkThreads) {
    const float sv = L[i] / temperature;
    if (top_p_bin(mx - sv) != bcut) continue;
    const unsigned long long q = fix_mass(E[i]);
    if (!q) continue;
    const unsigned int slot = atomicAdd(&R.ncand, 1u);
    if (slot < (unsigned)kTopPCandMax) {
      R.cand_key[slot] = order_key(sv);
      R.cand_q[slot] = q;
    }
  }
}

__global__ __launch_bounds__(kTopPThreads) void tp_select_kernel(const float* logits, int vocab,
                                                                 float temperature, TopPRow* rows,
                                                                 const float* ws) {
  __shared__ unsigned long long hist[256];
  __shared__ int s_bin;
  __shared__ unsigned long long s_above;
  const int row = blockIdx.x, tid = threadIdx.x, wave = tid >> 6;
  TopPRow& R = rows[row];
  const float* L = logits + (size_t)row * vocab;
  const float* E = ws + (size_t)row * vocab;
  const int ncand = (int)R.ncand, bcut = R.bcut;
  const bool listed = ncand <= kTopPCandMax;
  const float mx = tp_row_max(R, temperature);
  uint32_t prefix = 0, mask = 0;
  unsigned long long t_rem = R.target - R.above;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    if (listed) {
      for (int j = tid; j < ncand; j += kTopPThreads) {
        const uint32_t k = R.cand_key[j];
        if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], R.cand_q[j]);
      }
    } else {
      for (int i = tid; i < vocab; i += kTopPThreads) {
        const float sv = L[i] / temperature;
        if (top_p_bin(mx - sv) != bcut) continue;
        const unsigned long long q = fix_mass(E[i]);
        const uint32_t k = order_key(sv);
        if (q && (k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], q);
      }
    }
    __syncthreads();
    if (wave == 0) top_p_digit(hist, t_rem, &s_bin, &s_above);
    __syncthreads();
    prefix |= (uint32_t)s_bin << shift;
    mask |= 255u << shift;
    t_rem -= s_above;
    __syncthreads();
  }
  if (tid == 0) R.kappa = prefix;
}

__global__ __launch_bounds__(kTopPChunkThreads) void tp_kept_kernel(const float* logits, int vocab,
                                                                    float temperature, TopPRow* rows,
                                                                    const float* ws) {
  __shared__ unsigned long long red[4];
  const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  TopPRow& R = rows[row];
  const float* L = logits + (size_t)row * vocab;
  const float* E = ws + (size_t)row * vocab;
  const int cl = tp_chunk_len(vocab), beg = c * cl, end = min(vocab, beg + cl);
  const uint32_t kappa = R.kappa;
  unsigned long long m = 0;
  for (int i = beg + tid; i < end; i += kTopPChunkThreads)
    if (order_key(L[i] / temperature) >= kappa) m += fix_mass(E[i]);
  m = tp_block_sum(m, red);
  if (tid == 0) R.kpart[c] = m;
}

__global__ __launch_bounds__(kTopPChunkThreads) void tp_walk_kernel(const float* logits, int vocab,
                                                                    float temperature, uint64_t seed,
                                                                    uint64_t step, TopPRow* rows,
                                                                    const float* ws, int* out) {
  __shared__ unsigned long long red[4];
  __shared__ int s_tok;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const TopPRow& R = rows[row];
  const float* L = logits + (size_t)row * vocab;
  const float* E = ws + (size_t)row * vocab;
  const uint32_t kappa = R.kappa;
  unsigned long long zk = 0;
  for (int j = 0; j < kTopPChunks; ++j) zk += R.kpart[j];
  const uint64_t bits = splitmix64(synth_base(seed, 0x70707070ull + (uint64_t)row) + step) >> 40;
  const unsigned long long t = (zk >> 24) * bits + (((zk & 0xFFFFFFull) * bits) >> 24);
  // the chunk holding t (kept masses in chunk order = token-id order)
  int c = 0;
  unsigned long long cbase = 0;
  while (c + 1 < kTopPChunks && cbase + R.kpart[c] <= t) cbase += R.kpart[c++];
  const int cl = tp_chunk_len(vocab), cbeg = c * cl, cend = min(vocab, cbeg + cl);
  // thread segments of the chunk, exclusive scan of their kept masses, the owner walks
  const int seg = (cl + kTopPChunkThreads - 1) / kTopPChunkThreads;
  const int beg = min(cend, cbeg + tid * seg), end = min(cend, beg + seg);
  unsigned long long mine = 0;
  for (int i = beg; i < end; ++i)
    if (order_key(L[i] / temperature) >= kappa) mine += fix_mass(E[i]);
  unsigned long long inc = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  if (lane == 63) red[wave] = inc;
  if (tid == 0) s_tok = -1;
  __syncthreads();
  unsigned long long wb = cbase;
  for (int w = 0; w < wave; ++w) wb += red[w];
  const unsigned long long exc = wb + inc - mine;
  if (mine > 0 && exc <= t && t < exc + mine) {
    unsigned long long cum = exc;
    for (int i = beg; i < end; ++i) {
      if (order_key(L[i] / temperature) >= kappa) {
        cum += fix_mass(E[i]);
        if (cum > t) {
          s_tok = i;
          break;
        }
      }
    }
  }
  __syncthreads();
  if (tid == 0) out[row] = s_tok;
}

}  // namespace

static_assert(kTopPScratchBytes >= kTopPScratchFloats * sizeof(float) +
                                    kTopPNoallocRows * sizeof(TopPRow),
              "the static scratch holds the largest no-allocation workspace");

// ---------------------------------------------------------------- no-allocation scratch
// The top-p sampler's workspace (the [rows][vocab] fp32 exponentials, then a TopPRow per row)
// for the entry point that takes none: a file-scope device array of kTopPScratchBytes (8 MiB of
// exponentials for up to kTopPNoallocRows rows of 131072, and their TopPRows), one copy per GPU
// for the life of the process.  Host code never passes `scratch` itself to a kernel (on the
// host the name is only a stand-in, not the device address): top_p_scratch_init looks up each
// device's address once with hipGetSymbolAddress and the launcher passes that.
static __device__ __align__(256) float scratch[kTopPScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
float* g_scratch_addr[kMaxDevices] = {};
std::mutex g_scratch_mu;
}  // namespace

int top_p_scratch_init(int device) {
  IE_REQUIRE(device >= 0 && device < kMaxDevices, "top_p scratch: device %d out of [0, %d)",
             device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[device]) return IE_OK;
  int cur = -1;
  IE_CHECK_HIP(hipGetDevice(&cur));
  IE_REQUIRE(cur == device, "top_p scratch: device %d is not current (%d is)", device, cur);
  void* addr = nullptr;
  IE_CHECK_HIP(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
  IE_REQUIRE(addr != nullptr, "top_p scratch: no device address for device %d", device);
  g_scratch_addr[device] = static_cast<float*>(addr);
  return IE_OK;
}

float* top_p_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_addr[device];
}

int launch_argmax_rows(int rows, int vocab, const float* logits, int* out,
                       unsigned long long* slots, unsigned int* counters, hipStream_t st,
                       ArgmaxTail tail) {
  IE_REQUIRE(rows >= 1 && rows <= kNumSlots, "argmax: rows=%d out of range [1,%d]", rows,
             kNumSlots);
  IE_REQUIRE(vocab >= 1, "argmax: vocab=%d", vocab);
  int blocks = kArgmaxBlocks;
  if (vocab < blocks * 256) blocks = (vocab + 255) / 256;
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks, rows), dim3(256), 0, st, logits, vocab, out,
                     slots, counters, tail);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

size_t top_p_workspace_bytes(int rows, int vocab) {
  const size_t e = ((size_t)rows * (size_t)vocab * sizeof(float) + 255) & ~(size_t)255;
  return e + (size_t)rows * sizeof(TopPRow);
}

int launch_top_p(int rows, int vocab, const float* logits, float temperature, float top_p,
                 uint64_t seed, uint64_t step, int* out, float* ws, hipStream_t st) {
  IE_REQUIRE(rows >= 1 && rows <= 65535, "top_p: rows=%d", rows);
  IE_REQUIRE(vocab >= 1, "top_p: vocab=%d", vocab);
  IE_REQUIRE(temperature > 0.f, "top_p: temperature must be > 0 (got %g)", (double)temperature);
  IE_REQUIRE(top_p > 0.f && top_p <= 1.f, "top_p: top_p must be in (0, 1] (got %g)",
             (double)top_p);
  TopPRow* R = reinterpret_cast<TopPRow*>(reinterpret_cast<char*>(ws) +
                                          (top_p_workspace_bytes(rows, vocab) -
                                           (size_t)rows * sizeof(TopPRow)));
  const dim3 chunks(kTopPChunks, rows);
  hipLaunchKernelGGL(tp_max_kernel, chunks, dim3(kTopPChunkThreads), 0, st, logits, vocab, R);
  hipLaunchKernelGGL(tp_hist_kernel, chunks, dim3(kTopPChunkThreads), 0, st, logits, vocab,
                     temperature, R, ws);
  hipLaunchKernelGGL(tp_gather_kernel, chunks, dim3(kTopPChunkThreads), 0, st, logits, vocab,
                     temperature, top_p, R, ws);
  hipLaunchKernelGGL(tp_select_kernel, dim3(rows), dim3(kTopPThreads), 0, st, logits, vocab,
                     temperature, R, ws);
  hipLaunchKernelGGL(tp_kept_kernel, chunks, dim3(kTopPChunkThreads), 0, st, logits, vocab,
                     temperature, R, ws);
  hipLaunchKernelGGL(tp_walk_kernel, dim3(rows), dim3(kTopPChunkThreads), 0, st, logits, vocab,
                     temperature, seed, step, R, ws, out);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
