// GQA decode attention for one new token per sequence.
//
// Reference: decode_attn (kernels/attn.cu:373-439) runs QK^T and A.V as two
// cuBLAS batched GEMVs over device pointer arrays plus a separate row softmax
// (softmax.cu:109-160) with half-precision intermediates.  Here softmax(q.K^T /
// sqrt(128)) . V for all 32 q heads runs as split-context ("flash decoding")
// attention on MFMA:
//
//   grid  = (max_splits, 8 kv heads, batch), block = NW waves
//   split s of kv head g owns a contiguous run of the context 0..S-1 (at most 256 positions,
//   while the split cap allows), cut into tiles of 64 or 32 keys that its waves take in turn
//   (batch 1: 8 waves on 32-key tiles; batched: 12 waves on 32-key tiles for one split per
//   sequence, 4 on 64-key tiles for several); a wave stages its tile's K and V rows in LDS (K by
//   direct-to-LDS loads; V likewise at batch 1, through registers in the batched forms), and
//   computes, with
//   v_mfma_f32_16x16x32_bf16, S^T = K . Q^T for the 4 GQA q heads of the kv head (GQA: q head h
//   reads kv head h/4, attn.cu:51-53) as 4 of the 16 MFMA columns, an online softmax per head,
//   and O^T += V^T . P^T with P^T taken straight from the S^T accumulators and V^T read with
//   ds_read_b64_tr_b16, as in the prefill kernel.  The waves are merged in LDS and the split
//   writes one partial (m, l, o) per q head.
//
// The partials of the ns splits are merged either by the O projection itself (its
// input-staging prologue reads them; decode with max_splits = 4, no extra launch)
// or by a small merge kernel writing bf16 [h][128] (attn.cu:433-438) for the
// batched GEMM path and long contexts (max_splits = 32).  A device-scope "last
// workgroup merges" scheme is not used: its fence (L2 write-back / invalidate on
// this multi-XCD part) per workgroup cost more than a launch.
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) short4_t lds_short4;

constexpr int kSplitWaves = 4;
constexpr int kRowBytes = kHeadDim * 2;
constexpr int kBufferFlags = 0x00020000;   // buffer descriptor word 3 (raw 32-bit access)
static_assert(kAttnTile == 64, "tile = 4 x 16-key MFMA blocks");

// chunk c of key r of a tile at slot c ^ (r & 15) (LDS bank spread for the fragment reads)
__device__ __forceinline__ int kv_slot(int r, int c) { return r * 16 + (c ^ (r & 15)); }

static_assert(kAttnSplits <= 64, "the merge gives each split one lane");
// A wave preloads the page ids of its tiles, one per lane: with kAttnSplits splits of
// kSplitWaves waves, the longest context keeps that within 64 tiles per wave.
static_assert(kMaxLongCtx / kAttnTile <= 64 * kAttnSplits * 4, "page ids per wave exceed a wave");

// Phase 1: split s of (batch b, kv head g) attends its run of tiles (its NW waves take every
// NW-th tile) and writes the unnormalised partial (m, l, o) of each of the 4 q heads; with one
// split (max_splits = 1, batched: 12 waves on 32-key tiles) it writes the normalised bf16 output
// instead.  VREG: one LDS slice per wave, K through it and V staged in registers then written over
// K (72 KiB per 4-wave workgroup of 64-key tiles, two workgroups per CU: the batched split grid;
// 120 KiB for the 12-wave form); otherwise K and V each have a slice (136 KiB, one workgroup per
// CU; 0.7% faster per decode step at batch 1 than K fragments loaded straight into registers).
// The batched one-split form takes 32-key tiles so that 12 waves (3 per SIMD within the registers)
// cover a context of 17-24 half tiles in two rounds of half the work: 10.6 against 11.8 us per
// layer for 8 waves on 64-key tiles at bs = 16, S = 517-564, where one wave's ninth full tile
// ended each workgroup ~3 us after the others.  The batch-1 split form likewise runs 8 waves on
// 32-key tiles (the same tiles per split, half the work per wave): 4.85 against 5.07 us at
// S = 550-610.  Splits are counted in 64-key tiles whatever the tile, as the merge counts them.
template <bool VREG, int NW, int KT = kAttnTile>
__global__ __launch_bounds__(NW * 64) void attn_decode_split_kernel(AttnDecodeParams p) {
  // KT: keys per tile, 64 or 32 (half tiles: twice the waves on a context's tiles; a page
  // holds two)
  static_assert(KT == 64 || KT == 32, "tile of 64 or 32 keys");
  constexpr int KB = KT / 16;   // 16-key MFMA blocks per tile
  constexpr int KS2 = KT / 32;  // 32-key P.V contraction chunks per tile
  constexpr int NJ = KT / 4;    // 1 KiB loads per tile (4 rows each)
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  // wave id made provably uniform: the tile indices and buffer descriptors derived from it stay
  // in SGPRs (otherwise every buffer load becomes a readfirstlane loop)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 15, G = lane >> 4;
  const int S = p.d_seq_len ? p.d_seq_len[b] : p.seq_len;
  const int ntiles = (S + KT - 1) / KT;
  // (split count in 64-key tiles whatever KT: the merge and the O projection count the same)
  const int ns = attn_decode_splits((S + kAttnTile - 1) / kAttnTile, p.max_splits);
  if (split >= ns) return;  // whole workgroup: nobody reads a partial past ns
  const int tps = (ntiles + ns - 1) / ns;
  const int t0 = split * tps, t1 = min(ntiles, t0 + tps);

  __shared__ u32x4_t kvlds[NW][VREG ? 1 : 2][KT * 16];  // per wave: K tile (then V over it), V tile
  __shared__ float xo[NW][kGQA][kHeadDim];
  __shared__ float xml[NW][kGQA][2];
  const uint16_t* Kh = p.k_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  const uint16_t* Vh = p.v_cache + (size_t)b * p.cache_batch_stride + (size_t)g * kKVPlane;
  // rows past S read as zero (buffer bounds) and are masked below
  const __amdgpu_buffer_rsrc_t krs_seq =
      __builtin_amdgcn_make_buffer_rsrc((void*)Kh, 0, S * kRowBytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs_seq =
      __builtin_amdgcn_make_buffer_rsrc((void*)Vh, 0, S * kRowBytes, kBufferFlags);

  // Q^T fragments: MFMA column fr is q head 4g + fr for fr < 4 (zero elsewhere); lane supplies
  // dims 32 ks + 8 G .. +8
  bf16x8_t qf[4];
  {
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(
        p.q + ((size_t)b * kQHeads + g * kGQA + min(fr, kGQA - 1)) * kHeadDim);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4_t v = qrow[4 * ks + G];
      qf[ks] = __builtin_bit_cast(bf16x8_t, fr < kGQA ? v : u32x4_t{0u, 0u, 0u, 0u});
    }
  }
  const float scale = 0.08838834764831845f;  // 1/sqrt(128), softmax.cu:79
  float m = -INFINITY, l = 0.f;
  f32x4_t o[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4_t* kt = kvlds[wave][0];
  u32x4_t* vt = kvlds[wave][VREG ? 0 : 1];

  // paged KV: lane i holds the page of this wave's i-th tile (one load ahead of the loop)
  const bool paged = p.block_table != nullptr;
  int page_of = 0;
  if (paged) {
    const int t = t0 + wave + NW * lane;
    page_of = t < t1 ? p.block_table[(size_t)b * p.table_stride + t * KT / kAttnTile] : -1;
  }
  int it = 0;
  for (int t = t0 + wave; t < t1; t += NW, ++it) {
    const int key0 = t * KT;
    // the tile's buffers: rows key0.. of the sequence's cache, or rows 0.. of its page (a page
    // id outside the pool reads as zero)
    __amdgpu_buffer_rsrc_t krs = krs_seq, vrs = vrs_seq;
    int kr0 = key0;
    if (paged) {
      const int page = __builtin_amdgcn_readlane(page_of, it);
      const bool ok = page >= 0 && page < p.n_pages;
      const size_t base = (size_t)(ok ? page : 0) * kPageElems + (size_t)g * kPageHead;
      kr0 = key0 % kAttnTile;  // the tile's first row in its page
      const int bytes = ok ? min(kAttnTile, S - (key0 - kr0)) * kRowBytes : 0;
      krs = __builtin_amdgcn_make_buffer_rsrc((void*)(p.k_cache + base), 0, bytes, kBufferFlags);
      vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(p.v_cache + base), 0, bytes, kBufferFlags);
    }
    // Tile to LDS: load j fills rows 4j .. 4j+3; lane fills slot lane%16 of row 4j + lane/16
    // with global chunk (lane%16) ^ (row & 15).  The wave only reads its own slice, so its own
    // vmcnt wait is the whole synchronisation.  VREG (the batched forms, one slice per
    // wave): K goes through the slice by direct-to-LDS loads while V is loaded into registers,
    // row-contiguous, and written over K once the K fragments are in registers.  (Loading the
    // K fragments straight from memory instead reads 64-byte pieces of 16 rows per lane
    // quad and issued ~3x slower than row-contiguous loads.)
    u32x4_t vv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int r = 4 * j + G;
      const uint32_t off = (uint32_t)((kr0 + r) * kRowBytes + ((fr ^ (r & 15)) * 16));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)&kt[64 * j], 16, off, 0, 0, 0);
      if constexpr (!VREG)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)&vt[64 * j], 16, off, 0, 0, 0);
    }
    if constexpr (VREG) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        vv[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
            vrs, (uint32_t)((kr0 + 4 * j + G) * kRowBytes + fr * 16), 0, 0));
    }
    // K fragments kk[kb][ks] = K[key0 + 16 kb + fr][32 ks + 8 G .. +8] from the LDS tile
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(VREG ? NJ : 0) : "memory");
    u32x4_t kk[KB][4];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kk[kb][ks] = kt[kv_slot(16 * kb + fr, 4 * ks + G)];

    // ---- S^T blocks: s[kb][r] = S[q head 4g + fr][key key0 + 16 kb + 4 G + r]
    f32x4_t s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      s[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kk[kb][ks]),
                                                        qf[ks], s[kb], 0, 0, 0);
    }
    // ---- online softmax per q column (spread over lanes fr, fr+16, fr+32, fr+48)
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = key0 + 16 * kb + 4 * G + r;
        const float v = key < S ? s[kb][r] * scale : -INFINITY;
        s[kb][r] = v;
        mt = fmaxf(mt, v);
      }
    mt = xor32_max(xor16_max(mt));   // finite: key key0 < S is in every processed tile
    const float mn = fmaxf(m, mt);
    const float alpha = __expf(m - mn);
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __expf(s[kb][r] - mn);
        s[kb][r] = e;
        ls += e;
      }
    l = l * alpha + xor32_sum(xor16_sum(ls));
    m = mn;
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] *= alpha;
    // P^T fragments: slot 8 G + r <-> key 32 ks2 + 4 G + r, slot 8 G + 4 + r <-> key
    // 32 ks2 + 16 + 4 G + r
    bf16x8_t pb[KS2];
#pragma unroll
    for (int ks2 = 0; ks2 < KS2; ++ks2) {
      const u32x4_t w = {pack_bf2(s[2 * ks2][0], s[2 * ks2][1]), pack_bf2(s[2 * ks2][2], s[2 * ks2][3]),
                         pack_bf2(s[2 * ks2 + 1][0], s[2 * ks2 + 1][1]),
                         pack_bf2(s[2 * ks2 + 1][2], s[2 * ks2 + 1][3])};
      pb[ks2] = __builtin_bit_cast(bf16x8_t, w);
    }
    // ---- O^T[d][q] += V^T[d][keys] . P^T[keys][q]; V^T by transposed LDS reads (source lane
    //      s of a 16-lane group reads V[key0 + s/4][d0 + 4 (s%4) .. +3])
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the V tile has landed (LDS or registers)
    if constexpr (VREG) {
      // every K fragment read has returned (the MFMAs above consumed them): V over K
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < NJ; ++j) vt[kv_slot(4 * j + G, fr)] = vv[j];
    }
    const int kr = fr >> 2, dq = fr & 3;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int c = 2 * db + (dq >> 1), hb = (dq & 1) * 8;
#pragma unroll
      for (int ks2 = 0; ks2 < KS2; ++ks2) {
        const int ka = 32 * ks2 + 4 * G + kr;
        const char* va = reinterpret_cast<const char*>(&vt[kv_slot(ka, c)]) + hb;
        const char* vb = reinterpret_cast<const char*>(&vt[kv_slot(ka + 16, c)]) + hb;
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)va);
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)vb);
        const short4_t both[2] = {lo, hi};
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, both), pb[ks2],
                                                        o[db], 0, 0, 0);
      }
    }
    // the next tile's loads overwrite this slice: every read of it has returned
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // ---- this wave's partial: o[db][r] = O^T[d = 16 db + 4 G + r][head fr] (fr < 4); a wave
  //      without tiles has l = 0 (weight 0 in the merge)
  if (fr < kGQA) {
#pragma unroll
    for (int db = 0; db < 8; ++db)
      *reinterpret_cast<float4*>(&xo[wave][fr][16 * db + 4 * G]) =
          make_float4(o[db][0], o[db][1], o[db][2], o[db][3]);
    if (G == 0) {
      xml[wave][fr][0] = m;
      xml[wave][fr][1] = l;
    }
  }
  __syncthreads();
  if (wave >= kGQA) return;  // (NW > 4) waves past the 4 q heads only contribute partials
  const int h = wave;  // wave h merges q head 4g + h; lane d owns dims 2d, 2d+1
  const float mw = lane < NW ? xml[lane][h][0] : -INFINITY;
  const float lw = lane < NW ? xml[lane][h][1] : 0.f;
  const float M = wave_max(mw);
  const float wl = lw > 0.f ? __expf(mw - M) : 0.f;
  const float L = wave_sum(lw * wl);
  float o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float ww = readlane_f(wl, w);
    o0 = fmaf(xo[w][h][2 * lane], ww, o0);
    o1 = fmaf(xo[w][h][2 * lane + 1], ww, o1);
  }
  if (p.max_splits == 1) {
    // one split: the merged result is final (attn.cu:433-438), no partials
    const float inv = 1.0f / L;
    uint32_t* dst = reinterpret_cast<uint32_t*>(p.out + ((size_t)b * kQHeads + g * kGQA + h) * kHeadDim);
    dst[lane] = pack_bf2(o0 * inv, o1 * inv);
    return;
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
  // (a host-side length: one sequence; the paged cache holds up to kMaxLongCtx positions)
  IE_REQUIRE(p.d_seq_len || (p.seq_len >= 1 && batch == 1 &&
                             p.seq_len <= (p.block_table ? kMaxLongCtx : kMaxCtx)),
             "attn_decode: seq_len %d out of range [1,%d]", p.seq_len,
             p.block_table ? kMaxLongCtx : kMaxCtx);
  IE_REQUIRE(p.max_splits >= 1 && p.max_splits <= kAttnSplits, "attn_decode: max_splits %d",
             p.max_splits);
  IE_REQUIRE(p.max_splits > 1 || (merge && p.out), "attn_decode: one split writes the output");
  // one workgroup per possible split: idle ones would still cost dispatch (at batch 16 and
  // 32 splits, 4096 mostly empty workgroups took 52 us)
  if (p.max_splits == 1)  // one workgroup per (sequence, kv head): 12 waves share its tiles
    hipLaunchKernelGGL((attn_decode_split_kernel<true, 12, 32>), dim3(1, kKVHeads, batch),
                       dim3(12 * 64), 0, st, p);
  else if (batch > 1)
    hipLaunchKernelGGL((attn_decode_split_kernel<true, kSplitWaves>),
                       dim3(p.max_splits, kKVHeads, batch), dim3(kSplitWaves * 64), 0, st, p);
  else
    hipLaunchKernelGGL((attn_decode_split_kernel<false, 8, 32>), dim3(p.max_splits, kKVHeads, batch),
                       dim3(8 * 64), 0, st, p);
  IE_CHECK_LAUNCH();
  if (merge && p.max_splits > 1) {
    IE_REQUIRE(p.out, "attn_decode: merge needs an output buffer");
    hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(kKVHeads, batch), dim3(256), 0, st, p);
    IE_CHECK_LAUNCH();
  }
  return IE_OK;
}

}  // namespace ie
