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
//   2. radix select (4 x 8-bit digits of the order-preserving key of l_i/T) for
//      the cut key kappa with mass(key > kappa) < ceil-target <= mass(key >= kappa)
//   3. Z_kept = mass(key >= kappa); t = floor(Z_kept * u), u a 24-bit counter-RNG
//      uniform of (seed, row, step)
//   4. the sampled token is the smallest id whose kept prefix mass exceeds t
//      (inverse CDF in token-id order), found with a block-wide exclusive scan.
#include <mutex>

#include "ie_kernels.h"

namespace ie {

// ---------------------------------------------------------------- no-allocation scratch
// The top-p sampler's [rows][vocab] fp32 exponentials, for the entry point that takes no
// workspace: a file-scope device array of kTopPScratchFloats floats (8 MiB), one copy per GPU
// for the life of the process.  Host code never passes `scratch` itself to a kernel (on the
// host the name is only a stand-in, not the device address): top_p_scratch_init looks up each
// device's address once with hipGetSymbolAddress and the launcher passes that.
static __device__ __align__(256) float scratch[kTopPScratchFloats];

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
constexpr int kTopPWaves = kTopPThreads / 64;
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

__device__ unsigned long long block_sum_u64(unsigned long long v, unsigned long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  unsigned long long t = 0;
  for (int w = 0; w < kTopPWaves; ++w) t += red[w];
  return t;
}

__device__ float block_max_f(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
  for (int w = 1; w < kTopPWaves; ++w) t = fmaxf(t, red[w]);
  return t;
}

__global__ __launch_bounds__(kTopPThreads) void top_p_kernel(const float* logits, int vocab,
                                                             float temperature, float top_p,
                                                             uint64_t seed, uint64_t step,
                                                             int* out, float* ws) {
  __shared__ unsigned long long hist[256];
  __shared__ unsigned long long red64[kTopPWaves];
  __shared__ float redf[kTopPWaves];
  __shared__ int s_bin;
  __shared__ unsigned long long s_above;
  __shared__ int s_tok;

  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* L = logits + (size_t)row * vocab;
  float* E = ws + (size_t)row * vocab;

  // 1. max of l/T, cached exponentials, total mass
  float mx = -INFINITY;
  for (int i = tid; i < vocab; i += kTopPThreads) mx = fmaxf(mx, L[i] / temperature);
  mx = block_max_f(mx, redf);
  unsigned long long z = 0;
  for (int i = tid; i < vocab; i += kTopPThreads) {
    const float e = expf(L[i] / temperature - mx);
    E[i] = e;
    z += fix_mass(e);
  }
  z = block_sum_u64(z, red64);
  unsigned long long target = (unsigned long long)((double)z * (double)top_p);
  if (target < 1) target = 1;

  // 2. radix select of the cut key, most significant digit first
  uint32_t prefix = 0, mask = 0;
  unsigned long long t_rem = target;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < vocab; i += kTopPThreads) {
      const uint32_t k = order_key(L[i] / temperature);
      if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], fix_mass(E[i]));
    }
    __syncthreads();
    if (wave == 0) {
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
        s_bin = bin;
        s_above = above;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)s_bin << shift;
    mask |= 255u << shift;
    t_rem -= s_above;
    __syncthreads();
  }
  const uint32_t kappa = prefix;

  // 3. kept mass and the sampled point
  const int seg = (vocab + kTopPThreads - 1) / kTopPThreads;
  const int beg = min(vocab, tid * seg), end = min(vocab, beg + seg);
  unsigned long long mine = 0;
  for (int i = beg; i < end; ++i)
    if (order_key(L[i] / temperature) >= kappa) mine += fix_mass(E[i]);
  const unsigned long long zk = block_sum_u64(mine, red64);
  const uint64_t bits = splitmix64(synth_base(seed, 0x70707070ull + (uint64_t)row) + step) >> 40;
  const unsigned long long t = (zk >> 24) * bits + (((zk & 0xFFFFFFull) * bits) >> 24);

  // 4. exclusive scan of segment masses, then the owning thread walks its segment
  unsigned long long inc = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  __syncthreads();
  if (lane == 63) red64[wave] = inc;
  if (tid == 0) s_tok = -1;
  __syncthreads();
  unsigned long long wbase = 0;
  for (int w = 0; w < wave; ++w) wbase += red64[w];
  const unsigned long long exc = wbase + inc - mine;
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

int launch_top_p(int rows, int vocab, const float* logits, float temperature, float top_p,
                 uint64_t seed, uint64_t step, int* out, float* ws, hipStream_t st) {
  IE_REQUIRE(rows >= 1 && rows <= 65535, "top_p: rows=%d", rows);
  IE_REQUIRE(vocab >= 1, "top_p: vocab=%d", vocab);
  IE_REQUIRE(temperature > 0.f, "top_p: temperature must be > 0 (got %g)", (double)temperature);
  IE_REQUIRE(top_p > 0.f && top_p <= 1.f, "top_p: top_p must be in (0, 1] (got %g)",
             (double)top_p);
  hipLaunchKernelGGL(top_p_kernel, dim3(rows), dim3(kTopPThreads), 0, st, logits, vocab,
                     temperature, top_p, seed, step, out, ws);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
