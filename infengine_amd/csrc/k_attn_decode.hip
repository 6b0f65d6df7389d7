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
// Each split writes (m, l, o) to the workspace; the last split of a kv head to
// finish (device-scope counter) merges the partials and writes bf16 output in
// [h][128] order, which is the [1, 4096] row the O projection reads
// (attn.cu:433-438).  The counter is reset by that block, so it is zero again
// when the kernel ends.
#include "ie_kernels.h"

namespace ie {

namespace {

// Online-softmax attention of one q head (this wave) over cache rows
// [t0*64, min(t1*64, S)); returns the running max m, sum l and the unnormalised
// output slice acc[8] of dims (lane&15)*8.. (still split over the 4 row groups).
__device__ __forceinline__ void attend_tiles(const uint16_t* Kh, const uint16_t* Vh, uint4 qv,
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
    // ---- scores for 64 rows: 16 steps of 4 rows, 16 lanes per row
#pragma unroll 4
    for (int it = 0; it < kAttnTile / 4; ++it) {
      const int r = base + it * 4 + sub;
      float d = 0.f;
      if (r < S) d = dot8(reinterpret_cast<const uint4*>(Kh + (size_t)r * kHeadDim)[dl], qv, 0.f);
      d = row16_sum(d);
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
    // ---- P . V: 16 steps of 4 rows, each lane accumulates 8 dims
#pragma unroll 4
    for (int it = 0; it < kAttnTile / 4; ++it) {
      const int r = base + it * 4 + sub;
      if (r < S) {
        const float w = sc[wave][it * 4 + sub];
        const uint4 vv = reinterpret_cast<const uint4*>(Vh + (size_t)r * kHeadDim)[dl];
        acc[0] = fmaf(w, bf_lo(vv.x), acc[0]);
        acc[1] = fmaf(w, bf_hi(vv.x), acc[1]);
        acc[2] = fmaf(w, bf_lo(vv.y), acc[2]);
        acc[3] = fmaf(w, bf_hi(vv.y), acc[3]);
        acc[4] = fmaf(w, bf_lo(vv.z), acc[4]);
        acc[5] = fmaf(w, bf_hi(vv.z), acc[5]);
        acc[6] = fmaf(w, bf_lo(vv.w), acc[6]);
        acc[7] = fmaf(w, bf_hi(vv.w), acc[7]);
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

__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeParams p) {
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dl = lane & 15;
  const int S = p.d_seq_len ? p.d_seq_len[b] : p.seq_len;
  const int ntiles = (S + kAttnTile - 1) / kAttnTile;
  const int tps = (ntiles + kAttnSplits - 1) / kAttnSplits;
  const int t0 = split * tps;
  const int t1 = min(ntiles, t0 + tps);
  const int h = g * kGQA + wave;

  __shared__ float sc[4][kAttnTile];
  __shared__ int s_last;

  const uint16_t* Kh = p.k_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  const uint16_t* Vh = p.v_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  const uint4 qv = reinterpret_cast<const uint4*>(p.q + ((size_t)b * kQHeads + h) * kHeadDim)[dl];
  float m, l, acc[8];
  attend_tiles(Kh, Vh, qv, S, t0, t1, sc, m, l, acc);

  const size_t slot = (((size_t)b * kKVHeads + g) * kAttnSplits + split) * kGQA + wave;
  if (lane < 16) {
    float4* po = reinterpret_cast<float4*>(p.part_o + slot * kHeadDim + dl * 8);
    po[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    po[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  if (lane == 0) *reinterpret_cast<float2*>(p.part_ml + slot * 2) = make_float2(m, l);

  // ---- last split of this (batch, kv head) merges
  __threadfence();
  __syncthreads();
  unsigned int* cnt = p.counters + b * kKVHeads + g;
  if (tid == 0) s_last = (atomicAdd(cnt, 1u) == (unsigned)(kAttnSplits - 1));
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const size_t slot0 = (((size_t)b * kKVHeads + g) * kAttnSplits) * kGQA + wave;
  float M = -INFINITY;
  for (int sp = 0; sp < kAttnSplits; ++sp) M = fmaxf(M, p.part_ml[(slot0 + sp * kGQA) * 2]);
  float L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int sp = 0; sp < kAttnSplits; ++sp) {
    const size_t sl = slot0 + sp * kGQA;
    const float ms = p.part_ml[sl * 2], ls = p.part_ml[sl * 2 + 1];
    const float wgt = (ls > 0.f) ? __expf(ms - M) : 0.f;
    const float2 ov = *reinterpret_cast<const float2*>(p.part_o + sl * kHeadDim + 2 * lane);
    L = fmaf(ls, wgt, L);
    o0 = fmaf(ov.x, wgt, o0);
    o1 = fmaf(ov.y, wgt, o1);
  }
  const float inv = 1.0f / L;
  uint32_t* dst = reinterpret_cast<uint32_t*>(p.out + ((size_t)b * kQHeads + h) * kHeadDim);
  dst[lane] = pack_bf2(o0 * inv, o1 * inv);
  if (tid == 0) atomicExch(cnt, 0u);
}

// Causal prefill attention, one workgroup per (query row t, kv head g): q row t
// sits at absolute position start_pos + t and attends to cache rows
// 0..start_pos+t (attn.cu:355-363 with the causal mask of softmax.cu:55-107).
// Output row t is [32 heads][128], the permuted layout of attn_permute.cu:15-31.
__global__ __launch_bounds__(256) void attn_prefill_rows_kernel(AttnPrefillParams p) {
  const int t = blockIdx.x, g = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dl = lane & 15;
  const int h = g * kGQA + wave;
  const int S = p.start_pos + t + 1;
  __shared__ float sc[4][kAttnTile];
  const uint16_t* Kh = p.k + (size_t)g * kKVPlane;
  const uint16_t* Vh = p.v + (size_t)g * kKVPlane;
  const uint4 qv = reinterpret_cast<const uint4*>(p.q + ((size_t)t * kQHeads + h) * kHeadDim)[dl];
  float m, l, acc[8];
  attend_tiles(Kh, Vh, qv, S, 0, (S + kAttnTile - 1) / kAttnTile, sc, m, l, acc);
  if (lane < 16) {
    const float inv = 1.0f / l;
    uint4 o;
    o.x = pack_bf2(acc[0] * inv, acc[1] * inv);
    o.y = pack_bf2(acc[2] * inv, acc[3] * inv);
    o.z = pack_bf2(acc[4] * inv, acc[5] * inv);
    o.w = pack_bf2(acc[6] * inv, acc[7] * inv);
    reinterpret_cast<uint4*>(p.out + (size_t)t * kHidden + h * kHeadDim)[dl] = o;
  }
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
  dim3 grid(kAttnSplits, kKVHeads, batch);
  hipLaunchKernelGGL(attn_decode_kernel, grid, dim3(256), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t st) {
  IE_REQUIRE(p.S >= 1 && p.start_pos >= 0 && p.start_pos + p.S <= kMaxCtx,
             "attn_prefill: rows [%d, %d) exceed the KV cache", p.start_pos, p.start_pos + p.S);
  hipLaunchKernelGGL(attn_prefill_rows_kernel, dim3(p.S, kKVHeads), dim3(256), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
