// Decode GEMV family (m = 1): y = W . x with bf16 weights streamed from HBM.
//
// Reference: multiply_by_weight (kernels/ffn.cu:7-33) computes Y = X . W^T through
// cublasGemmEx with fp32 compute.  Here every launch is a hand-written kernel in
// which one wave64 owns a PAIR of weight rows at a time: each lane loads 16 bytes
// (8 bf16) of both rows per step, so a wave-wide load covers 1 KiB of one row and
// the two rows of a pair give 2 x (K/512) independent 128-bit loads in flight per
// lane.  The dot products run on the gfx950 dot2 unit (bf16 x bf16 -> fp32) and
// the wave reduction is DPP within 16-lane rows plus 4 readlanes.
//
// Pairing the rows lets the epilogue see both outputs a fused op needs:
//   * SwiGLU:  (gate row r, up row r)                    -> h[r]        (ffn.cu:53-58)
//   * RoPE:    (row j, row j+64) of one q/k head          -> rotated pair (rope.cu:53-64)
//   * others:  rows (2p, 2p+1)                            -> bf16 / fp32 / residual add
// The input vector is staged once per workgroup in LDS; with `norm` the staging
// applies RMSNorm (rmsnorm.cu:31-63) on the way in, so no normalised copy of the
// activations is ever written to HBM.
#include "ie_kernels.h"

namespace ie {

namespace {

__device__ __forceinline__ float sumsq8(const uint4& v) {
  float s = 0.f;
  s = fmaf(bf_lo(v.x), bf_lo(v.x), s); s = fmaf(bf_hi(v.x), bf_hi(v.x), s);
  s = fmaf(bf_lo(v.y), bf_lo(v.y), s); s = fmaf(bf_hi(v.y), bf_hi(v.y), s);
  s = fmaf(bf_lo(v.z), bf_lo(v.z), s); s = fmaf(bf_hi(v.z), bf_hi(v.z), s);
  s = fmaf(bf_lo(v.w), bf_lo(v.w), s); s = fmaf(bf_hi(v.w), bf_hi(v.w), s);
  return s;
}

// bf16(bf16(x * r) * w): the two rounding points of rmsnorm.cu:61 / HF LlamaRMSNorm.
__device__ __forceinline__ uint32_t norm2(uint32_t x, uint32_t w, float r) {
  float lo = bf2f(f2bf(bf_lo(x) * r)) * bf_lo(w);
  float hi = bf2f(f2bf(bf_hi(x) * r)) * bf_hi(w);
  return pack_bf2(lo, hi);
}

__device__ __forceinline__ uint4 norm8(const uint4& x, const uint4& w, float r) {
  return make_uint4(norm2(x.x, w.x, r), norm2(x.y, w.y, r), norm2(x.z, w.z, r),
                    norm2(x.w, w.w, r));
}

template <int EPI, int K>
__device__ __forceinline__ void rows_of_pair(const GemvParams& p, int pair, const uint16_t*& r0,
                                             const uint16_t*& r1) {
  if constexpr (EPI == kEpiSwiglu) {
    r0 = p.w0 + (size_t)pair * K;
    r1 = p.w1 + (size_t)pair * K;
  } else if constexpr (EPI == kEpiQkvRope) {
    const int head = pair >> 6, j = pair & 63;
    const uint16_t* base;
    if (head < kQHeads) base = p.w0 + (size_t)head * kHeadDim * K;
    else if (head < kQHeads + kKVHeads) base = p.w1 + (size_t)(head - kQHeads) * kHeadDim * K;
    else base = p.w2 + (size_t)(head - kQHeads - kKVHeads) * kHeadDim * K;
    r0 = base + (size_t)j * K;
    r1 = base + (size_t)(j + 64) * K;
  } else {
    r0 = p.w0 + (size_t)(2 * pair) * K;
    r1 = r0 + K;
  }
}

template <int EPI>
__device__ __forceinline__ void gemv_epilogue(const GemvParams& p, int pair, int row, float a0,
                                              float a1) {
  if constexpr (EPI == kEpiBf16) {
    uint16_t* o = p.out + (size_t)row * p.out_stride + 2 * pair;
    *reinterpret_cast<uint32_t*>(o) = pack_bf2(a0, a1);
  } else if constexpr (EPI == kEpiF32) {
    float* o = p.out_f32 + (size_t)row * p.out_stride + 2 * pair;
    *reinterpret_cast<float2*>(o) = make_float2(a0, a1);
  } else if constexpr (EPI == kEpiResid) {
    uint32_t* o = reinterpret_cast<uint32_t*>(p.out + 2 * pair);
    const uint32_t old = *o;
    const float y0 = bf2f(f2bf(a0)), y1 = bf2f(f2bf(a1));
    *o = pack_bf2(bf_lo(old) + y0, bf_hi(old) + y1);
  } else if constexpr (EPI == kEpiSwiglu) {
    const float g = bf2f(f2bf(a0)), u = bf2f(f2bf(a1));
    p.out[pair] = f2bf(g * (1.0f / (1.0f + expf(-g))) * u);
  } else {  // kEpiQkvRope
    const int head = pair >> 6, j = pair & 63;
    const int pos = p.d_seq_len ? (*p.d_seq_len - 1) : p.pos;
    float y0 = bf2f(f2bf(a0)), y1 = bf2f(f2bf(a1));
    if (head < kQHeads + kKVHeads) {
      const float c = p.rope_cos[pos * (kHeadDim / 2) + j];
      const float s = p.rope_sin[pos * (kHeadDim / 2) + j];
      const float o0 = y0 * c - y1 * s;
      const float o1 = y0 * s + y1 * c;
      y0 = o0;
      y1 = o1;
    }
    uint16_t* dst;
    if (head < kQHeads) {
      dst = p.out + head * kHeadDim;
    } else {
      const int kvh = (head - kQHeads) & (kKVHeads - 1);
      uint16_t* plane = head < kQHeads + kKVHeads ? p.k_cache : p.v_cache;
      dst = plane + ((size_t)kvh * kMaxCtx + pos) * kHeadDim;
    }
    dst[j] = f2bf(y0);
    dst[j + 64] = f2bf(y1);
  }
}

template <int K, int EPI, bool NORM>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  constexpr int NC = K / 512;                // 16-byte chunks per lane per row
  constexpr int G = (NC % 8 == 0) ? 8 : 7;   // chunks per load group
  static_assert(NC % G == 0, "K must be a multiple of 512*G");
  __shared__ uint4 xs[K / 8];
  __shared__ float red[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.y;
  const uint4* x4 = reinterpret_cast<const uint4*>(p.x + (size_t)row * p.x_stride);

  if constexpr (NORM) {
    float ss = 0.f;
    for (int i = tid; i < K / 8; i += 256) {
      const uint4 v = x4[i];
      xs[i] = v;
      ss += sumsq8(v);
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = rsqrtf(tot / (float)K + kRmsEps);
    const uint4* w4 = reinterpret_cast<const uint4*>(p.norm_w);
    for (int i = tid; i < K / 8; i += 256) xs[i] = norm8(xs[i], w4[i], r);
  } else {
    for (int i = tid; i < K / 8; i += 256) xs[i] = x4[i];
  }
  __syncthreads();

  const int first = (blockIdx.x * 4 + wave) * p.ppw;
  for (int i = 0; i < p.ppw; ++i) {
    const int pair = first + i;
    if (pair >= p.n_pairs) break;
    const uint16_t *r0, *r1;
    rows_of_pair<EPI, K>(p, pair, r0, r1);
    const uint4* a = reinterpret_cast<const uint4*>(r0) + lane;
    const uint4* b = reinterpret_cast<const uint4*>(r1) + lane;
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll 1
    for (int g = 0; g < NC; g += G) {
      uint4 wa[G], wb[G];
#pragma unroll
      for (int c = 0; c < G; ++c) {
        wa[c] = ld_stream(a + (g + c) * 64);
        wb[c] = ld_stream(b + (g + c) * 64);
      }
#pragma unroll
      for (int c = 0; c < G; ++c) {
        const uint4 xv = xs[(g + c) * 64 + lane];
        acc0 = dot8(wa[c], xv, acc0);
        acc1 = dot8(wb[c], xv, acc1);
      }
    }
    acc0 = wave_sum(acc0);
    acc1 = wave_sum(acc1);
    if (lane == 0) gemv_epilogue<EPI>(p, pair, row, acc0, acc1);
  }
}

template <int K, int EPI, bool NORM>
int launch_t(const GemvParams& p, int rows, hipStream_t st) {
  const int waves = (p.n_pairs + p.ppw - 1) / p.ppw;
  dim3 grid((waves + 3) / 4, rows);
  hipLaunchKernelGGL((gemv_kernel<K, EPI, NORM>), grid, dim3(256), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int K>
int launch_k(int epi, bool norm, const GemvParams& p, int rows, hipStream_t st) {
  switch (epi) {
    case kEpiBf16: return norm ? launch_t<K, kEpiBf16, true>(p, rows, st)
                               : launch_t<K, kEpiBf16, false>(p, rows, st);
    case kEpiF32: return norm ? launch_t<K, kEpiF32, true>(p, rows, st)
                              : launch_t<K, kEpiF32, false>(p, rows, st);
    case kEpiResid: return norm ? launch_t<K, kEpiResid, true>(p, rows, st)
                                : launch_t<K, kEpiResid, false>(p, rows, st);
    case kEpiSwiglu: return norm ? launch_t<K, kEpiSwiglu, true>(p, rows, st)
                                 : launch_t<K, kEpiSwiglu, false>(p, rows, st);
    case kEpiQkvRope: return norm ? launch_t<K, kEpiQkvRope, true>(p, rows, st)
                                  : launch_t<K, kEpiQkvRope, false>(p, rows, st);
  }
  set_error("launch_gemv: bad epilogue %d", epi);
  return IE_ERR_INVALID_ARG;
}

}  // namespace

int default_ppw(int n_pairs) {
  // Aim for ~2048 waves in flight (256 CUs x 8) so each wave amortises the
  // staging of x over several row pairs without starving the chip.
  int ppw = n_pairs / 2048;
  if (ppw < 1) ppw = 1;
  if (ppw > 32) ppw = 32;
  return ppw;
}

int launch_gemv(int K, int epi, bool norm, GemvParams p, int rows, hipStream_t st) {
  IE_REQUIRE(rows >= 1 && rows <= 65535, "launch_gemv: rows=%d out of range", rows);
  IE_REQUIRE(p.n_pairs >= 1, "launch_gemv: no rows");
  IE_REQUIRE(rows == 1 || epi == kEpiBf16 || epi == kEpiF32,
             "launch_gemv: epilogue %d supports one row only", epi);
  if (p.ppw <= 0) p.ppw = default_ppw(p.n_pairs);
  if (K == 4096) return launch_k<4096>(epi, norm, p, rows, st);
  if (K == 14336) return launch_k<14336>(epi, norm, p, rows, st);
  set_error("launch_gemv: unsupported K=%d (4096 or 14336)", K);
  return IE_ERR_UNSUPPORTED;
}

}  // namespace ie
