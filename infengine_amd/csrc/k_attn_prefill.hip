// Causal GQA prefill attention on MFMA (flash style: online softmax, no S x S
// scores in memory).
//
// Reference: attn (kernels/attn.cu:309-371) materialises QK^T for all 32 heads
// ([32, S, S] fp16, cublasGemmBatchedEx), runs a causal softmax kernel
// (softmax.cu:55-107), multiplies by V and permutes [h, s, d] -> [s, h, d].
//
// Here one workgroup owns 16 query rows of the 4 q heads of one kv head (GQA:
// q head h reads kv head h/4, attn.cu:51-53); wave w is q head 4g + w, so every
// K/V tile staged in LDS feeds 4 heads.  Per 64-key tile and wave:
//   S^T[key][q] = K . Q^T      16 x v_mfma_f32_16x16x32_bf16 (A = K from LDS,
//                                B = Q fragments held in registers)
//   online softmax per query column (scale 1/sqrt(128), causal mask key > q)
//   O^T[d][q] += V^T . P^T      16 MFMAs; B = P^T straight from the S^T
//                                accumulators: the 32 contraction slots of one
//                                MFMA are mapped to keys {4G+r, 16+4G+r} of a
//                                32-key half tile, the same permutation on both
//                                operands, so P never goes through LDS
// V is written to LDS transposed ([d][key], 8-byte key quads XOR-swizzled by
// d & 15) so the A operand of the P.V product is two 8-byte LDS reads.  K rows
// are 16 chunks of 16 bytes, chunk c of key r stored at c ^ (r & 15).
// Output rows are [s][h][d] (the attn_permute.cu:15-31 layout), bf16.
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

constexpr int BQ = 16;    // query rows per workgroup
constexpr int BKEY = 64;  // keys per LDS tile

__device__ __forceinline__ uint32_t pack_bf2_rn(float lo, float hi) { return pack_bf2(lo, hi); }

__global__ __launch_bounds__(256) void flash_prefill_kernel(AttnPrefillParams p) {
  __shared__ u32x4_t k_lds[BKEY * 16];          // [key][16 chunks], 16 KiB
  __shared__ u32x2_t vt_lds[kHeadDim * (BKEY / 4)];  // [d][16 key quads], 16 KiB

  const int qt = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, G = lane >> 4;
  const int h = g * kGQA + wave;
  const int row0 = qt * BQ;                       // first query row of the tile
  const int rows = min(BQ, p.S - row0);
  const int q_abs = p.start_pos + row0 + fr;      // this lane's query position
  const int nkeys = p.start_pos + row0 + rows;    // keys 0 .. nkeys-1 are needed
  const int ntiles = (nkeys + BKEY - 1) / BKEY;

  const uint16_t* Kg = p.k + (size_t)g * kKVPlane;
  const uint16_t* Vg = p.v + (size_t)g * kKVPlane;

  // Q^T fragments: lane holds Q[q = row0 + fr][d = 32 ks + 8 G .. +8]
  bf16x8_t qf[4];
  {
    const int qr = row0 + min(fr, rows - 1);
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(p.q + ((size_t)qr * kQHeads + h) * kHeadDim);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = __builtin_bit_cast(bf16x8_t, qrow[4 * ks + G]);
  }

  f32x4_t o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale = 0.08838834764831845f;  // 1/sqrt(128), softmax.cu:79

  for (int t = 0; t < ntiles; ++t) {
    const int key0 = t * BKEY;
    __syncthreads();  // the previous tile is fully consumed
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + i * 256, r = idx >> 4, c = idx & 15;
      const int key = min(key0 + r, nkeys - 1);
      const u32x4_t kv = reinterpret_cast<const u32x4_t*>(Kg + (size_t)key * kHeadDim)[c];
      k_lds[r * 16 + (c ^ (r & 15))] = kv;
      const u32x4_t vv = reinterpret_cast<const u32x4_t*>(Vg + (size_t)key * kHeadDim)[c];
      // transpose: 8 dims of one key -> V^T[c*8 + e][key]
      uint16_t* vt = reinterpret_cast<uint16_t*>(vt_lds);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = c * 8 + e;
        const uint32_t w = vv[e >> 1];
        const uint16_t val = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFF);
        vt[(d * (BKEY / 4) + ((r >> 2) ^ (d & 15))) * 4 + (r & 3)] = val;
      }
    }
    __syncthreads();

    // ---- S^T tiles: s[kt][r] = S[q = fr][key = key0 + 16 kt + 4 G + r]
    f32x4_t s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const int kr = kt * 16 + fr;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, k_lds[kr * 16 + ((4 * ks + G) ^ fr)]);
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[ks], s[kt], 0, 0, 0);
      }
    }
    // ---- online softmax for query column fr (spread over lanes fr, fr+16, fr+32, fr+48)
    float mt = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = key0 + kt * 16 + 4 * G + r;
        const float v = (key <= q_abs && key < nkeys) ? s[kt][r] * scale : -INFINITY;
        s[kt][r] = v;
        mt = fmaxf(mt, v);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m, mt);
    // a query row whose keys in this tile are all masked keeps mn = m (finite
    // after its first tile, which always holds key 0)
    const float alpha = __expf(m - mn);
    float ls = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __expf(s[kt][r] - mn);
        s[kt][r] = e;
        ls += e;
      }
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    l = l * alpha + ls;
    m = mn;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;

    // ---- P^T fragments (contraction slots 8G+r <-> key 32 ks2 + 4G + r,
    //      8G+4+r <-> key 32 ks2 + 16 + 4G + r)
    bf16x8_t pb[2];
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      const u32x4_t w = {pack_bf2_rn(s[2 * ks2][0], s[2 * ks2][1]),
                         pack_bf2_rn(s[2 * ks2][2], s[2 * ks2][3]),
                         pack_bf2_rn(s[2 * ks2 + 1][0], s[2 * ks2 + 1][1]),
                         pack_bf2_rn(s[2 * ks2 + 1][2], s[2 * ks2 + 1][3])};
      pb[ks2] = __builtin_bit_cast(bf16x8_t, w);
    }
    // ---- O^T[d][q] += V^T[d][keys] . P^T[keys][q]
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = dt * 16 + fr;
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        const int kq0 = (8 * ks2 + G) ^ (d & 15);          // keys 32 ks2 + 4G .. +3
        const int kq1 = (8 * ks2 + 4 + G) ^ (d & 15);      // keys 32 ks2 + 16 + 4G .. +3
        const u32x2_t lo = vt_lds[d * (BKEY / 4) + kq0];
        const u32x2_t hi = vt_lds[d * (BKEY / 4) + kq1];
        const u32x4_t av = {lo[0], lo[1], hi[0], hi[1]};
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), pb[ks2],
                                                         o[dt], 0, 0, 0);
      }
    }
  }

  // ---- o[dt][r] = O[q = fr][d = 16 dt + 4 G + r] (unnormalised)
  if (fr < rows) {
    const float inv = 1.0f / l;
    uint16_t* dst = p.out + (size_t)(row0 + fr) * kHidden + h * kHeadDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x2_t w = {pack_bf2(o[dt][0] * inv, o[dt][1] * inv),
                         pack_bf2(o[dt][2] * inv, o[dt][3] * inv)};
      *reinterpret_cast<u32x2_t*>(dst + dt * 16 + 4 * G) = w;
    }
  }
}

}  // namespace

int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t st) {
  IE_REQUIRE(p.S >= 1 && p.start_pos >= 0 && p.start_pos + p.S <= kMaxCtx,
             "attn_prefill: rows [%d, %d) exceed the KV cache", p.start_pos, p.start_pos + p.S);
  hipLaunchKernelGGL(flash_prefill_kernel, dim3((p.S + BQ - 1) / BQ, kKVHeads), dim3(256), 0, st,
                     p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
