// GQA decode attention for one new token per sequence.
//
// Reference: decode_attn (kernels/attn.cu:373-439) runs QK^T and A.V as two
// cuBLAS batched GEMVs over device pointer arrays plus a separate row softmax
// (softmax.cu:109-160) with half-precision intermediates.  Here one kernel does
// softmax(q.K^T / sqrt(128)) . V for all 32 q heads in fp32:
//
//   grid  = (kAttnSplits, 8 kv heads, batch), block = 4 waves
//   wave w of block (s, g) is q head 4g + w (GQA: q head h reads kv head h/4,
//   attn.cu:51-53), so the 4 waves stream the same K/V rows and only the first
//   touches HBM.  The context 0..S-1 is cut into 64-row tiles; split s owns a
//   contiguous run of tiles and keeps an online softmax (running max m, sum l,
//   unnormalised output) across them.
//
// Each split writes (m, l, o) to the workspace and a second, tiny kernel merges
// the partials and writes bf16 output in [h][128] order, which is the [1, 4096]
// row the O projection reads (attn.cu:433-438).  Two launches instead of a
// last-block merge: a device-scope fence per workgroup (L2 write-back and
// invalidate on this multi-XCD part) costs more than one extra launch.
#include "ie_kernels.h"

namespace ie {

namespace {

// Online-softmax attention of one q head (this wave) over cache rows
// [t0*64, min(t1*64, S)); returns the running max m, sum l and the unnormalised
// output slice acc[8] of dims (lane&15)*8.. (summed over the wave's 4 row groups).
// Each 64-row tile issues all of its K and V loads (16 + 16 x 16 bytes per lane)
// before any arithmetic; rows past S are clamped to S-1 for the load and masked
// to probability 0.
__device__ __forceinline__ void attend_tiles(const uint16_t* Kh, const uint16_t* Vh, u32x4_t qv,
                                             int S, int t0, int t1, float (*sc)[kAttnTile],
                                             float& m, float& l, float acc[8]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, dl = lane & 15;
  const float scale = 0.08838834764831845f;  // 1/sqrt(128), softmax.cu:79
  m = -INFINITY;
  l = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;

  for (int t = t0; t < t1; ++t) {
    const int base = t * kAttnTile;
    u32x4_t kk[kAttnTile / 4], vv[kAttnTile / 4];
#pragma unroll
    for (int it = 0; it < kAttnTile / 4; ++it) {
      const int r = min(base + it * 4 + sub, S - 1);
      kk[it] = reinterpret_cast<const u32x4_t*>(Kh + (size_t)r * kHeadDim)[dl];
    }
#pragma unroll
    for (int it = 0; it < kAttnTile / 4; ++it) {
      const int r = min(base + it * 4 + sub, S - 1);
      vv[it] = reinterpret_cast<const u32x4_t*>(Vh + (size_t)r * kHeadDim)[dl];
    }
    // ---- scores for 64 rows: 16 steps of 4 rows, 16 lanes per row
#pragma unroll
    for (int it = 0; it < kAttnTile / 4; ++it) {
      const float d = row16_sum(dot8(kk[it], qv, 0.f));
      const int r = base + it * 4 + sub;
      if (dl == 0) sc[wave][it * 4 + sub] = (r < S) ? d * scale : -INFINITY;
    }
    __syncthreads();
    // ---- online softmax over this tile (lane <-> row)
    const float s = sc[wave][lane];
    const float mt = wave_max(s);
    const float mn = fmaxf(m, mt);
    const float alpha = __expf(m - mn);
    const float pr = __expf(s - mn);
    l = l * alpha + wave_sum(pr);
    m = mn;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    sc[wave][lane] = pr;
    __syncthreads();
    // ---- P . V: each lane accumulates 8 dims over its 16 rows
#pragma unroll
    for (int it = 0; it < kAttnTile / 4; ++it) {
      const float w = sc[wave][it * 4 + sub];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] = fmaf(w, bf_lo(vv[it][q]), acc[2 * q]);
        acc[2 * q + 1] = fmaf(w, bf_hi(vv[it][q]), acc[2 * q + 1]);
      }
    }
    __syncthreads();
  }
  // fold the 4 row groups of the wave: lanes dl, dl+16, dl+32, dl+48
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    acc[i] += __shfl_xor(acc[i], 16, 64);
    acc[i] += __shfl_xor(acc[i], 32, 64);
  }
}

static_assert(kAttnSplits <= 64, "the merge gives each split one lane");

// Phase 1: split s of (batch b, kv head g) attends its run of tiles and writes
// the unnormalised partial (m, l, o) of each of the 4 q heads.
__global__ __launch_bounds__(256) void attn_decode_split_kernel(AttnDecodeParams p) {
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dl = lane & 15;
  const int S = p.d_seq_len ? p.d_seq_len[b] : p.seq_len;
  const int ntiles = (S + kAttnTile - 1) / kAttnTile;
  const int tps = (ntiles + kAttnSplits - 1) / kAttnSplits;
  const int t0 = split * tps;
  const int t1 = min(ntiles, t0 + tps);
  const int h = g * kGQA + wave;
  const size_t slot = (((size_t)b * kKVHeads + g) * kAttnSplits + split) * kGQA + wave;
  if (t0 >= t1) {  // empty split: weight 0 in the merge, zero partial output
    if (lane < 16) {
      float4* po = reinterpret_cast<float4*>(p.part_o + slot * kHeadDim + dl * 8);
      po[0] = make_float4(0.f, 0.f, 0.f, 0.f);
      po[1] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (lane == 0) *reinterpret_cast<float2*>(p.part_ml + slot * 2) = make_float2(-INFINITY, 0.f);
    return;
  }

  __shared__ float sc[4][kAttnTile];
  const uint16_t* Kh = p.k_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  const uint16_t* Vh = p.v_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  const u32x4_t qv =
      reinterpret_cast<const u32x4_t*>(p.q + ((size_t)b * kQHeads + h) * kHeadDim)[dl];
  float m, l, acc[8];
  attend_tiles(Kh, Vh, qv, S, t0, t1, sc, m, l, acc);
  if (lane < 16) {
    float4* po = reinterpret_cast<float4*>(p.part_o + slot * kHeadDim + dl * 8);
    po[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    po[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  if (lane == 0) *reinterpret_cast<float2*>(p.part_ml + slot * 2) = make_float2(m, l);
}

// Phase 2 (next kernel on the stream, so phase 1's writes are visible): one
// workgroup per (batch, kv head), wave w merges q head 4g + w.  Lane s holds
// split s's (m, l); every partial load is issued up front (one memory latency).
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(AttnDecodeParams p) {
  const int g = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = g * kGQA + wave;
  __shared__ float wsh[4][64];
  const size_t slot0 = (((size_t)b * kKVHeads + g) * kAttnSplits) * kGQA + wave;
  float ms = -INFINITY, ls = 0.f;
  if (lane < kAttnSplits) {
    const float2 v = *reinterpret_cast<const float2*>(p.part_ml + (slot0 + lane * kGQA) * 2);
    ms = v.x;
    ls = v.y;
  }
  float2 ov[kAttnSplits];
#pragma unroll
  for (int sp = 0; sp < kAttnSplits; ++sp)
    ov[sp] = *reinterpret_cast<const float2*>(p.part_o + (slot0 + sp * kGQA) * kHeadDim + 2 * lane);
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

int launch_attn_decode(const AttnDecodeParams& p, int batch, hipStream_t st) {
  IE_REQUIRE(batch >= 1 && batch <= 16, "attn_decode: batch %d out of range [1,16]", batch);
  IE_REQUIRE(p.d_seq_len || (p.seq_len >= 1 && p.seq_len <= kMaxCtx && batch == 1),
             "attn_decode: seq_len %d out of range [1,%d]", p.seq_len, kMaxCtx);
  hipLaunchKernelGGL(attn_decode_split_kernel, dim3(kAttnSplits, kKVHeads, batch), dim3(256), 0,
                     st, p);
  IE_CHECK_LAUNCH();
  hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(kKVHeads, batch), dim3(256), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
