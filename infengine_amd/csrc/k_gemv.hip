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

__device__ __forceinline__ float sumsq8(const u32x4_t& v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s = fmaf(bf_lo(v[i]), bf_lo(v[i]), s);
    s = fmaf(bf_hi(v[i]), bf_hi(v[i]), s);
  }
  return s;
}

// bf16(bf16(x * r) * w): the two rounding points of rmsnorm.cu:61 / HF LlamaRMSNorm.
__device__ __forceinline__ uint32_t norm2(uint32_t x, uint32_t w, float r) {
  float lo = bf2f(f2bf(bf_lo(x) * r)) * bf_lo(w);
  float hi = bf2f(f2bf(bf_hi(x) * r)) * bf_hi(w);
  return pack_bf2(lo, hi);
}

__device__ __forceinline__ u32x4_t norm8(const u32x4_t& x, const u32x4_t& w, float r) {
  return u32x4_t{norm2(x[0], w[0], r), norm2(x[1], w[1], r), norm2(x[2], w[2], r),
                 norm2(x[3], w[3], r)};
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

// Operands an epilogue reads from memory (the residual, the RoPE position and angle), loaded in
// the prologue with the inputs when the wave owns a single pair, so that the epilogue does not end
// the wave on a load latency.  `have` = false: the epilogue loads them itself.
struct EpiPre {
  uint32_t old = 0;
  float c = 0.f, s = 0.f;
  int pos = 0;
  bool have = false;
};

template <int EPI>
__device__ __forceinline__ EpiPre epi_preload(const GemvParams& p, int pair) {
  EpiPre e;
  e.have = true;
  if constexpr (EPI == kEpiResid) {
    e.old = *reinterpret_cast<const uint32_t*>(p.out + 2 * pair);
  } else if constexpr (EPI == kEpiQkvRope) {
    // V heads take no rotation; their (valid) table entries are loaded and unused
    const int j = pair & 63;
    e.pos = p.d_seq_len ? (*p.d_seq_len - 1) : p.pos;
    e.c = p.rope_cos[e.pos * (kHeadDim / 2) + j];
    e.s = p.rope_sin[e.pos * (kHeadDim / 2) + j];
  }
  return e;
}

template <int EPI>
__device__ __forceinline__ void gemv_epilogue(const GemvParams& p, int pair, int row, float a0,
                                              float a1, const EpiPre& e) {
  if constexpr (EPI == kEpiBf16) {
    uint16_t* o = p.out + (size_t)row * p.out_stride + 2 * pair;
    *reinterpret_cast<uint32_t*>(o) = pack_bf2(a0, a1);
  } else if constexpr (EPI == kEpiF32) {
    float* o = p.out_f32 + (size_t)row * p.out_stride + 2 * pair;
    *reinterpret_cast<float2*>(o) = make_float2(a0, a1);
  } else if constexpr (EPI == kEpiResid) {
    uint32_t* o = reinterpret_cast<uint32_t*>(p.out + 2 * pair);
    const uint32_t old = e.have ? e.old : *o;
    const float y0 = bf2f(f2bf(a0)), y1 = bf2f(f2bf(a1));
    *o = pack_bf2(bf_lo(old) + y0, bf_hi(old) + y1);
  } else if constexpr (EPI == kEpiSwiglu) {
    const float g = bf2f(f2bf(a0)), u = bf2f(f2bf(a1));
    p.out[pair] = f2bf(g * (1.0f / (1.0f + expf(-g))) * u);
  } else {  // kEpiQkvRope
    const int head = pair >> 6, j = pair & 63;
    const int pos = e.have ? e.pos : (p.d_seq_len ? (*p.d_seq_len - 1) : p.pos);
    float y0 = bf2f(f2bf(a0)), y1 = bf2f(f2bf(a1));
    if (head < kQHeads + kKVHeads) {
      const float c = e.have ? e.c : p.rope_cos[pos * (kHeadDim / 2) + j];
      const float s = e.have ? e.s : p.rope_sin[pos * (kHeadDim / 2) + j];
      const float o0 = rope_lo(y0, y1, c, s);
      const float o1 = rope_hi(y0, y1, c, s);
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

// Loads of one pipeline step: G 16-byte chunks of each row of a pair.
template <int G>
__device__ __forceinline__ void load_step(const u32x4_t* a, const u32x4_t* b, int g0,
                                          u32x4_t (&wa)[G], u32x4_t (&wb)[G]) {
#pragma unroll
  for (int c = 0; c < G; ++c) {
    wa[c] = ld_stream(a + (g0 + c) * 64);
    wb[c] = ld_stream(b + (g0 + c) * 64);
  }
}

// The decode attention output for the O projection, merged from the split partials straight
// into the staged input vector: 8 dims of one q head per item, same arithmetic as the merge
// kernel (weights exp(m_s - max m), o = sum_s w_s o_s / sum_s w_s l_s).  The loads of an item
// are issued before the weight stream (attn_load) and merged after it is in flight (attn_merge).
template <int MS>
struct AttnItem {
  float2 ml[MS];
  float4 oa[MS], ob[MS];
};

// All MS slots are loaded (they lie inside the partials buffer, which holds kAttnSplits per kv
// head; attn_merge reads only the first ns).  The loads neither branch nor depend on ns (a
// device value in graph replays): either would let the compiler issue them after the weight
// stream, or make its wait at the merge conservative, and the staging would then wait for the
// weights.
template <int MS>
__device__ __forceinline__ void attn_load(const GemvParams& p, int i, AttnItem<MS>& a) {
  const int h = i >> 4, c = i & 15;
  const size_t slot0 = ((size_t)(h / kGQA) * kAttnSplits) * kGQA + (h % kGQA);
#pragma unroll
  for (int sp = 0; sp < MS; ++sp) {
    const size_t slot = slot0 + (size_t)sp * kGQA;
    a.ml[sp] = *reinterpret_cast<const float2*>(p.attn_part_ml + slot * 2);
    const float4* po = reinterpret_cast<const float4*>(p.attn_part_o + slot * kHeadDim + c * 8);
    a.oa[sp] = po[0];
    a.ob[sp] = po[1];
  }
}

template <int MS>
__device__ __forceinline__ u32x4_t attn_merge(const AttnItem<MS>& a, int ns) {
  float M = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < MS; ++sp)
    if (sp < ns) M = fmaxf(M, a.ml[sp].x);
  float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < MS; ++sp) {
    if (sp < ns) {
      const float w = a.ml[sp].y > 0.f ? __expf(a.ml[sp].x - M) : 0.f;
      L = fmaf(a.ml[sp].y, w, L);
      o[0] = fmaf(a.oa[sp].x, w, o[0]);
      o[1] = fmaf(a.oa[sp].y, w, o[1]);
      o[2] = fmaf(a.oa[sp].z, w, o[2]);
      o[3] = fmaf(a.oa[sp].w, w, o[3]);
      o[4] = fmaf(a.ob[sp].x, w, o[4]);
      o[5] = fmaf(a.ob[sp].y, w, o[5]);
      o[6] = fmaf(a.ob[sp].z, w, o[6]);
      o[7] = fmaf(a.ob[sp].w, w, o[7]);
    }
  }
  const float inv = 1.0f / L;
  return u32x4_t{pack_bf2(o[0] * inv, o[1] * inv), pack_bf2(o[2] * inv, o[3] * inv),
                 pack_bf2(o[4] * inv, o[5] * inv), pack_bf2(o[6] * inv, o[7] * inv)};
}

// Loads of step t of this wave's (pair, chunk-group) sequence into (wa, wb).  The pair index
// is clamped to the last pair, so a wave past the end loads valid rows it never stores.
template <int K, int EPI, int G, int NG>
__device__ __forceinline__ void issue_step(const GemvParams& p, int first, int lane, int t,
                                           u32x4_t (&wa)[G], u32x4_t (&wb)[G]) {
  const uint16_t *r0, *r1;
  rows_of_pair<EPI, K>(p, min(first + t / NG, p.n_pairs - 1), r0, r1);
  load_step<G>(reinterpret_cast<const u32x4_t*>(r0) + lane,
               reinterpret_cast<const u32x4_t*>(r1) + lane, (t % NG) * G, wa, wb);
}

// Dot products of step t against the staged input; the row pair's epilogue after its last step.
template <int EPI, int G, int NG>
__device__ __forceinline__ void consume_step(const GemvParams& p, const u32x4_t* xs, int first,
                                             int row, int lane, int t, const u32x4_t (&wa)[G],
                                             const u32x4_t (&wb)[G], float& acc0, float& acc1,
                                             const EpiPre& e) {
  const int g = t % NG;
#pragma unroll
  for (int c = 0; c < G; ++c) {
    const u32x4_t xv = xs[(g * G + c) * 64 + lane];
    acc0 = dot8(wa[c], xv, acc0);
    acc1 = dot8(wb[c], xv, acc1);
  }
  if (g == NG - 1) {
    const float a0 = wave_sum(acc0), a1 = wave_sum(acc1);
    if (lane == 0 && first + t / NG < p.n_pairs)
      gemv_epilogue<EPI>(p, first + t / NG, row, a0, a1, e);
    acc0 = 0.f;
    acc1 = 0.f;
  }
}

// ONE: one pair per wave (the default), unrolled at compile time so every wait is exact; the
// general loop for more pairs per wave is a separate instance because its conditional loads
// more than double the register count.
// ATTN: 0, or the split slots (kAttnFusedSplits / kAttnFusedSplitsLong) the O projection merges
// into its input.
template <int K, int EPI, bool NORM, int WAVES, int ATTN, bool ONE>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvParams p) {
  constexpr int T = WAVES * 64;
  constexpr int NC = K / 512;                 // 16-byte chunks per lane per row
  constexpr int G = (K == 4096) ? 4 : 7;      // chunks per pipeline step
  constexpr int NG = NC / G;                  // steps per row pair
  static_assert(NC % G == 0 && NG % 2 == 0, "K must be a multiple of 1024*G");
  constexpr int XC = (K / 8 + T - 1) / T;     // input chunks staged per thread
  constexpr int AI = (kQHeads * kHeadDim / 8 + T - 1) / T;  // attention items per thread
  __shared__ u32x4_t xs[K / 8];
  __shared__ float red[WAVES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.y;
  const int first = (blockIdx.x * WAVES + wave) * p.ppw;
  const int npairs = max(0, min(p.ppw, p.n_pairs - first));
  const int nsteps = npairs * NG;

  // Memory operations return in issue order, so the input (activations, norm weight, attention
  // partials) is loaded first: it lands while the weight stream is still in flight, and the
  // staging below waits for it alone.  These loads and the first two weight steps are
  // unconditional (indices clamped): a load under a branch makes the compiler's wait at the
  // join conservative, which would stall the staging until the weights arrive.
  const u32x4_t* x4 = reinterpret_cast<const u32x4_t*>(p.x + (size_t)row * p.x_stride);
  u32x4_t xin[XC], nwin[XC];
  AttnItem<ATTN ? ATTN : 1> ai[ATTN ? AI : 1];
  int ns = 0;
  if constexpr (ATTN != 0) {
    static_assert(K == kQHeads * kHeadDim && !NORM, "attention input: the O projection only");
#pragma unroll
    for (int j = 0; j < AI; ++j) attn_load(p, min(tid + j * T, kQHeads * kHeadDim / 8 - 1), ai[j]);
    const int S = p.d_seq_len ? *p.d_seq_len : p.pos;
    ns = attn_decode_splits((S + kAttnTile - 1) / kAttnTile, p.attn_max_splits);
  } else {
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int i = min(tid + j * T, K / 8 - 1);
      xin[j] = x4[i];
      if constexpr (NORM) nwin[j] = reinterpret_cast<const u32x4_t*>(p.norm_w)[i];
    }
  }

  EpiPre epre;
  if constexpr (ONE) epre = epi_preload<EPI>(p, min(first, p.n_pairs - 1));
  __builtin_amdgcn_sched_barrier(0);  // keep every input load ahead of the weight stream

  // Weight stream: two steps in flight in two register buffers (B0: even steps, B1: odd).
  u32x4_t a0[G], b0[G], a1[G], b1[G];
  issue_step<K, EPI, G, NG>(p, first, lane, 0, a0, b0);
  issue_step<K, EPI, G, NG>(p, first, lane, 1, a1, b1);

  if constexpr (ATTN != 0) {
#pragma unroll
    for (int j = 0; j < AI; ++j)
      if (tid + j * T < kQHeads * kHeadDim / 8) xs[tid + j * T] = attn_merge(ai[j], ns);
  } else if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < XC; ++j)
      if (tid + j * T < K / 8) ss += sumsq8(xin[j]);
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) tot += red[w];
    const float r = rsqrtf(tot / (float)K + kRmsEps);
#pragma unroll
    for (int j = 0; j < XC; ++j)
      if (tid + j * T < K / 8) xs[tid + j * T] = norm8(xin[j], nwin[j], r);
  } else {
#pragma unroll
    for (int j = 0; j < XC; ++j)
      if (tid + j * T < K / 8) xs[tid + j * T] = xin[j];
  }
  __syncthreads();

  // Step t+2 is issued into the buffer step t has just been consumed from.
  float acc0 = 0.f, acc1 = 0.f;
  if constexpr (ONE) {
#pragma unroll
    for (int t = 0; t < NG; t += 2) {
      consume_step<EPI, G, NG>(p, xs, first, row, lane, t, a0, b0, acc0, acc1, epre);
      if (t + 2 < NG) issue_step<K, EPI, G, NG>(p, first, lane, t + 2, a0, b0);
      consume_step<EPI, G, NG>(p, xs, first, row, lane, t + 1, a1, b1, acc0, acc1, epre);
      if (t + 3 < NG) issue_step<K, EPI, G, NG>(p, first, lane, t + 3, a1, b1);
    }
  } else {
    for (int t = 0; t < nsteps; t += 2) {
      consume_step<EPI, G, NG>(p, xs, first, row, lane, t, a0, b0, acc0, acc1, epre);
      if (t + 2 < nsteps) issue_step<K, EPI, G, NG>(p, first, lane, t + 2, a0, b0);
      consume_step<EPI, G, NG>(p, xs, first, row, lane, t + 1, a1, b1, acc0, acc1, epre);
      if (t + 3 < nsteps) issue_step<K, EPI, G, NG>(p, first, lane, t + 3, a1, b1);
    }
  }
}

template <int K, int EPI, bool NORM, int WAVES, bool ONE>
int launch_o(const GemvParams& p, int rows, hipStream_t st) {
  const int waves = (p.n_pairs + p.ppw - 1) / p.ppw;
  dim3 grid((waves + WAVES - 1) / WAVES, rows);
  if constexpr (K == kQHeads * kHeadDim && EPI == kEpiResid && !NORM) {
    if (p.attn_part_o) {
      if (p.attn_max_splits <= kAttnFusedSplits)
        hipLaunchKernelGGL((gemv_kernel<K, EPI, NORM, WAVES, kAttnFusedSplits, ONE>), grid,
                           dim3(WAVES * 64), 0, st, p);
      else
        hipLaunchKernelGGL((gemv_kernel<K, EPI, NORM, WAVES, kAttnFusedSplitsLong, ONE>), grid,
                           dim3(WAVES * 64), 0, st, p);
      IE_CHECK_LAUNCH();
      return IE_OK;
    }
  }
  hipLaunchKernelGGL((gemv_kernel<K, EPI, NORM, WAVES, 0, ONE>), grid, dim3(WAVES * 64), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int K, int EPI, bool NORM, int WAVES>
int launch_w(const GemvParams& p, int rows, hipStream_t st) {
  return p.ppw == 1 ? launch_o<K, EPI, NORM, WAVES, true>(p, rows, st)
                    : launch_o<K, EPI, NORM, WAVES, false>(p, rows, st);
}

template <int K, int EPI, bool NORM>
int launch_t(const GemvParams& p, int rows, hipStream_t st) {
  const int waves = gemv_waves(K, EPI, p.n_pairs);
  if constexpr (EPI == kEpiQkvRope) {
    if (waves == 12) return launch_w<K, EPI, NORM, 12>(p, rows, st);
  }
  switch (waves) {
    case 8: return launch_w<K, EPI, NORM, 8>(p, rows, st);
    case 16: return launch_w<K, EPI, NORM, 16>(p, rows, st);
    default: return launch_w<K, EPI, NORM, 4>(p, rows, st);
  }
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

namespace {
int g_ppw_override = 0;
int g_waves_override = 0;
}  // namespace

// Waves per workgroup: each workgroup stages (and for RMSNorm ops normalises) the whole input
// vector once, so more waves per workgroup means less of that per weight byte, at the price of
// coarser occupancy.  8 by default; the fused QKV GEMV (3072 row pairs) uses 12, which makes
// its grid exactly one workgroup per CU (measured 1.0 us faster per launch than 384 workgroups
// of 8 waves, whose 1.5 workgroups per CU finish unevenly).
int gemv_waves(int K, int epi, int n_pairs) {
  if (g_waves_override > 0) return g_waves_override;
  (void)K;
  (void)n_pairs;
  return epi == kEpiQkvRope ? 12 : 8;
}

int default_ppw(int n_pairs) {
  if (g_ppw_override > 0) return g_ppw_override;
  // One row pair per wave measured fastest on MI355X for every decode shape
  // (QKV, O, gate/up, down, lm_head): the most waves, hence the most 16-byte
  // loads in flight per CU, while the software pipeline already hides the
  // x staging behind the first loads.
  (void)n_pairs;
  return 1;
}

int launch_gemv(int K, int epi, bool norm, GemvParams p, int rows, hipStream_t st) {
  IE_REQUIRE(rows >= 1 && rows <= 65535, "launch_gemv: rows=%d out of range", rows);
  IE_REQUIRE(p.n_pairs >= 1, "launch_gemv: no rows");
  IE_REQUIRE(rows == 1 || epi == kEpiBf16 || epi == kEpiF32,
             "launch_gemv: epilogue %d supports one row only", epi);
  IE_REQUIRE(!p.attn_part_o || (K == kQHeads * kHeadDim && epi == kEpiResid && !norm && rows == 1 &&
                                p.attn_part_ml && p.attn_max_splits >= 1 &&
                                p.attn_max_splits <= kAttnFusedSplitsLong &&
                                (p.d_seq_len || (p.pos >= 1 && p.pos <= kMaxCtx))),
             "launch_gemv: attention-partials input is for the O projection only");
  if (p.ppw <= 0) p.ppw = default_ppw(p.n_pairs);
  if (K == 4096) return launch_k<4096>(epi, norm, p, rows, st);
  if (K == 14336) return launch_k<14336>(epi, norm, p, rows, st);
  set_error("launch_gemv: unsupported K=%d (4096 or 14336)", K);
  return IE_ERR_UNSUPPORTED;
}

}  // namespace ie

extern "C" int ie_tune_gemv_waves(int waves) {
  IE_REQUIRE(waves == 0 || waves == 4 || waves == 8 || waves == 16,
             "tune_gemv_waves: %d not one of 0 (default), 4, 8, 16", waves);
  ie::g_waves_override = waves;
  return IE_OK;
}

extern "C" int ie_tune_gemv_pairs_per_wave(int ppw) {
  IE_REQUIRE(ppw >= 0 && ppw <= 64, "tune_gemv_pairs_per_wave: %d out of [0, 64]", ppw);
  ie::g_ppw_override = ppw;
  return IE_OK;
}
