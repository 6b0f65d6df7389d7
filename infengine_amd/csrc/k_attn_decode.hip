// GQA decode attention for one new token per sequence.
//
// Reference: decode_attn (kernels/attn.cu:373-439) runs QK^T and A.V as two
// cuBLAS batched GEMVs over device pointer arrays plus a separate row softmax
// (softmax.cu:109-160) with half-precision intermediates.  Here softmax(q.K^T /
// sqrt(128)) . V for all 32 q heads runs in fp32 as split-context ("flash
// decoding") attention:
//
//   grid  = (kAttnSplits, 8 kv heads, batch), block = 8 waves
//   split s of kv head g owns a contiguous run of 64-row tiles of the context
//   0..S-1; its 8 waves take 16-row slices of that run in turn and each computes
//   all 4 q heads of the kv head (GQA: q head h reads kv head h/4, attn.cu:51-53)
//   for its rows, so every K/V byte is fetched once per workgroup and each wave
//   does 64 (row, head) dot products per slice.  Each wave keeps an online softmax
//   (running max m, sum l, unnormalised output) per head over its slices; the 8
//   waves are merged in LDS and the split writes one partial (m, l, o) per q head.
//
// The number of splits ns = min(max_splits, ceil(tiles / 2)) follows the context
// length (two tiles, i.e. one slice per wave, per split while that fits).  The
// partials of the ns splits are merged either by the O projection itself (its
// input-staging prologue reads them; decode with max_splits = 8, no extra launch)
// or by a small merge kernel writing bf16 [h][128] (attn.cu:433-438) for the
// batched GEMM path and long contexts (max_splits = 32).  A device-scope "last
// workgroup merges" scheme is not used: its fence (L2 write-back / invalidate on
// this multi-XCD part) per workgroup cost more than a launch.
#include "ie_kernels.h"

namespace ie {

namespace {

constexpr int kSplitWaves = 8;
constexpr int kSlice = 16;  // rows per wave per step

// Wave-local ordering of this wave's own LDS slice (waves run different slice counts, so no
// workgroup barrier may sit inside the slice loop).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Online-softmax attention of the 4 q heads of one kv head over the 16-row slices
// first, first + stride, ... of rows [row0, row1) (row1 <= S).  Lane (sub = lane/16, dl =
// lane%16) loads 16 bytes (dims 8dl..8dl+7) of rows 4it + sub, it = 0..3, of a slice.
// Returns, in the lanes of 16-lane group h, head h's running max and sum (m_me, l_me), and in
// every lane the unnormalised outputs acc[h][8] of dims 8dl.. summed over its rows.
__device__ __forceinline__ void attend_slices(const uint16_t* Kh, const uint16_t* Vh,
                                              const u32x4_t (&qv)[kGQA], int S, int row0,
                                              int row1, int first, int stride, float* sc,
                                              float& m_me, float& l_me, float (&acc)[kGQA][8]) {
  const int lane = threadIdx.x & 63;
  const int sub = lane >> 4, dl = lane & 15;
  const float scale = 0.08838834764831845f;  // 1/sqrt(128), softmax.cu:79
  m_me = -INFINITY;
  l_me = 0.f;
#pragma unroll
  for (int h = 0; h < kGQA; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;

  for (int base = row0 + first * kSlice; base < row1; base += stride * kSlice) {
    u32x4_t kk[kSlice / 4], vv[kSlice / 4];
#pragma unroll
    for (int it = 0; it < kSlice / 4; ++it) {
      const int r = min(base + it * 4 + sub, S - 1);
      kk[it] = reinterpret_cast<const u32x4_t*>(Kh + (size_t)r * kHeadDim)[dl];
      vv[it] = reinterpret_cast<const u32x4_t*>(Vh + (size_t)r * kHeadDim)[dl];
    }
    // ---- scores: (head h, slice row j) -> sc[16h + j]; rows past row1 get -inf
#pragma unroll
    for (int it = 0; it < kSlice / 4; ++it) {
      const int r = base + it * 4 + sub;
#pragma unroll
      for (int h = 0; h < kGQA; ++h) {
        const float d = row16_sum(dot8(kk[it], qv[h], 0.f));
        if (dl == 0) sc[h * kSlice + it * 4 + sub] = (r < row1) ? d * scale : -INFINITY;
      }
    }
    wave_lds_sync();
    // ---- online softmax, lane <-> (head lane/16, row lane%16); row `base` is always < row1
    const float s = sc[lane];
    const float mn = fmaxf(m_me, row16_max(s));
    const float alpha = __expf(m_me - mn);
    const float pr = __expf(s - mn);
    l_me = l_me * alpha + row16_sum(pr);
    m_me = mn;
    sc[lane] = pr;
#pragma unroll
    for (int h = 0; h < kGQA; ++h) {
      const float a = readlane_f(alpha, h * kSlice);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= a;
    }
    wave_lds_sync();
    // ---- P . V: each lane accumulates 8 dims of each head over its 4 rows
#pragma unroll
    for (int it = 0; it < kSlice / 4; ++it) {
#pragma unroll
      for (int h = 0; h < kGQA; ++h) {
        const float w = sc[h * kSlice + it * 4 + sub];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[h][2 * q] = fmaf(w, bf_lo(vv[it][q]), acc[h][2 * q]);
          acc[h][2 * q + 1] = fmaf(w, bf_hi(vv[it][q]), acc[h][2 * q + 1]);
        }
      }
    }
    wave_lds_sync();
  }
  // fold the 4 row groups of the wave: lanes dl, dl+16, dl+32, dl+48
#pragma unroll
  for (int h = 0; h < kGQA; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc[h][i] = xor32_sum(xor16_sum(acc[h][i]));
    }
}

static_assert(kAttnSplits <= 64, "the merge gives each split one lane");

// Phase 1: split s of (batch b, kv head g) attends its run of tiles and writes the
// unnormalised partial (m, l, o) of each of the 4 q heads.
__global__ __launch_bounds__(kSplitWaves * 64) void attn_decode_split_kernel(AttnDecodeParams p) {
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dl = lane & 15;
  const int S = p.d_seq_len ? p.d_seq_len[b] : p.seq_len;
  const int ntiles = (S + kAttnTile - 1) / kAttnTile;
  const int ns = attn_decode_splits(ntiles, p.max_splits);
  if (split >= ns) return;  // whole workgroup: nobody reads a partial past ns
  const int tps = (ntiles + ns - 1) / ns;
  const int row0 = split * tps * kAttnTile;
  const int row1 = min(S, row0 + tps * kAttnTile);

  __shared__ float sc[kSplitWaves][kGQA * kSlice];
  __shared__ float xo[kSplitWaves][kGQA][kHeadDim];
  __shared__ float xml[kSplitWaves][kGQA][2];
  const uint16_t* Kh = p.k_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  const uint16_t* Vh = p.v_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  u32x4_t qv[kGQA];
#pragma unroll
  for (int h = 0; h < kGQA; ++h)
    qv[h] = reinterpret_cast<const u32x4_t*>(p.q + ((size_t)b * kQHeads + g * kGQA + h) * kHeadDim)[dl];
  float m_me, l_me, acc[kGQA][8];
  attend_slices(Kh, Vh, qv, S, row0, row1, wave, kSplitWaves, sc[wave], m_me, l_me, acc);

  // merge the 8 waves' partials of each head (a wave without rows has l = 0: weight 0)
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < kGQA; ++h) {
      float4* d = reinterpret_cast<float4*>(&xo[wave][h][dl * 8]);
      d[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      d[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  if ((lane & 15) == 0) {
    xml[wave][lane >> 4][0] = m_me;
    xml[wave][lane >> 4][1] = l_me;
  }
  __syncthreads();
  if (wave >= kGQA) return;
  const int h = wave;  // wave h merges q head 4g + h; lane d owns dims 2d, 2d+1
  const float mw = lane < kSplitWaves ? xml[lane][h][0] : -INFINITY;
  const float lw = lane < kSplitWaves ? xml[lane][h][1] : 0.f;
  const float M = wave_max(mw);
  const float wl = lw > 0.f ? __expf(mw - M) : 0.f;
  const float L = wave_sum(lw * wl);
  float o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int w = 0; w < kSplitWaves; ++w) {
    const float ww = readlane_f(wl, w);
    o0 = fmaf(xo[w][h][2 * lane], ww, o0);
    o1 = fmaf(xo[w][h][2 * lane + 1], ww, o1);
  }
  const size_t slot = (((size_t)b * kKVHeads + g) * kAttnSplits + split) * kGQA + h;
  *reinterpret_cast<float2*>(p.part_o + slot * kHeadDim + 2 * lane) = make_float2(o0, o1);
  if (lane == 0) *reinterpret_cast<float2*>(p.part_ml + slot * 2) = make_float2(M, L);
}

// Phase 2 (next kernel on the stream, so phase 1's writes are visible): one
// workgroup per (batch, kv head), wave w merges q head 4g + w.  Lane s holds
// split s's (m, l); every partial load is issued up front (one memory latency).
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(AttnDecodeParams p) {
  const int g = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = g * kGQA + wave;
  const int S = p.d_seq_len ? p.d_seq_len[b] : p.seq_len;
  const int ns = attn_decode_splits((S + kAttnTile - 1) / kAttnTile, p.max_splits);
  __shared__ float wsh[4][64];
  const size_t slot0 = (((size_t)b * kKVHeads + g) * kAttnSplits) * kGQA + wave;
  float ms = -INFINITY, ls = 0.f;
  if (lane < ns) {
    const float2 v = *reinterpret_cast<const float2*>(p.part_ml + (slot0 + lane * kGQA) * 2);
    ms = v.x;
    ls = v.y;
  }
  float2 ov[kAttnSplits];
#pragma unroll
  for (int sp = 0; sp < kAttnSplits; ++sp)
    ov[sp] = sp < ns ? *reinterpret_cast<const float2*>(p.part_o + (slot0 + sp * kGQA) * kHeadDim +
                                                        2 * lane)
                     : make_float2(0.f, 0.f);
  const float M = wave_max(ms);
  const float wl = (ls > 0.f) ? __expf(ms - M) : 0.f;
  const float L = wave_sum(ls * wl);
  wsh[wave][lane] = wl;
  __syncthreads();
  float o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int sp = 0; sp < kAttnSplits; ++sp) {
    const float w = wsh[wave][sp];
    o0 = fmaf(ov[sp].x, w, o0);
    o1 = fmaf(ov[sp].y, w, o1);
  }
  const float inv = 1.0f / L;
  uint32_t* dst = reinterpret_cast<uint32_t*>(p.out + ((size_t)b * kQHeads + h) * kHeadDim);
  dst[lane] = pack_bf2(o0 * inv, o1 * inv);
}

}  // namespace

size_t attn_decode_partials_bytes(int batch) {
  const size_t slots = (size_t)batch * kKVHeads * kAttnSplits * kGQA;
  return slots * kHeadDim * sizeof(float) + slots * 2 * sizeof(float);
}

int launch_attn_decode(const AttnDecodeParams& p, int batch, bool merge, hipStream_t st) {
  IE_REQUIRE(batch >= 1 && batch <= 16, "attn_decode: batch %d out of range [1,16]", batch);
  IE_REQUIRE(p.d_seq_len || (p.seq_len >= 1 && p.seq_len <= kMaxCtx && batch == 1),
             "attn_decode: seq_len %d out of range [1,%d]", p.seq_len, kMaxCtx);
  IE_REQUIRE(p.max_splits >= 1 && p.max_splits <= kAttnSplits, "attn_decode: max_splits %d",
             p.max_splits);
  // one workgroup per possible split: idle ones would still cost dispatch (at batch 16 and
  // 32 splits, 4096 mostly empty workgroups took 52 us)
  hipLaunchKernelGGL(attn_decode_split_kernel, dim3(p.max_splits, kKVHeads, batch),
                     dim3(kSplitWaves * 64), 0, st, p);
  IE_CHECK_LAUNCH();
  if (merge) {
    IE_REQUIRE(p.out, "attn_decode: merge needs an output buffer");
    hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(kKVHeads, batch), dim3(256), 0, st, p);
    IE_CHECK_LAUNCH();
  }
  return IE_OK;
}

}  // namespace ie
