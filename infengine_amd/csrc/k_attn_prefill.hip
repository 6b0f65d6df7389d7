// Causal GQA prefill attention on MFMA (flash style: online softmax, no S x S
// scores in memory).
//
// Reference: attn (kernels/attn.cu:309-371) materialises QK^T for all 32 heads
// ([32, S, S] fp16, cublasGemmBatchedEx), runs a causal softmax kernel
// (softmax.cu:55-107), multiplies by V and permutes [h, s, d] -> [s, h, d].
//
// Here a workgroup owns 32 query rows of the 4 q heads of one kv head (GQA: q head h reads kv
// head h/4, attn.cu:51-53); wave w is q head 4g + w, so every K/V tile staged in LDS feeds the
// 4 heads.  Per 64-key tile and wave, with v_mfma_f32_16x16x32_bf16:
//   S^T[key][q] = K . Q^T      32 MFMAs (A = K rows from LDS, B = Q fragments in registers;
//                                the two 16-query column blocks share every K fragment)
//   online softmax per query column (scale 1/sqrt(128), causal mask key > q)
//   O^T[d][q] += V^T . P^T      32 MFMAs; B = P^T straight from the S^T accumulators: the 32
//                                contraction slots of one MFMA are mapped to keys {4G+r, 16+4G+r}
//                                of a 32-key half tile, the same permutation on both operands
// K and V tiles go global -> LDS with direct-to-LDS buffer loads, row-major [key][128] (chunk c
// of key r at slot c ^ (r & 15)), double-buffered so the next tile loads under this tile's
// MFMAs.  The A operand of O^T is V^T; gfx950's ds_read_b64_tr_b16 reads it from the row-major
// tile: in each 16-lane group, output lane j receives element j % 4 of the 8 bytes read by source
// lanes 4e + j / 4 (e = 0..3), so with source lane s reading V[key0 + s/4][d0 + 4 (s%4) ..+3],
// lane j gets V[key0 + e][d0 + j], e = 0..3: four consecutive keys of one dim.  Rows past the
// last key read as zero (buffer bounds), so the masked tail never multiplies garbage.
// Workgroups are issued longest causal extent first, paired so that the two a CU holds sum to
// about the mean.  Output rows are [s][h][d] (the attn_permute.cu:15-31 layout), bf16.
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) short4_t lds_short4;

constexpr int BQ = 32;                // query rows per workgroup at most (QI = 2 blocks of 16)
constexpr int BKEY = 64;              // keys per LDS tile
constexpr int TC = BKEY * 16;         // 16-byte chunks per K (or V) tile
constexpr int kRowBytes = kHeadDim * 2;
constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw 32-bit access)

__device__ __forceinline__ int kv_slot(int r, int c) { return r * 16 + (c ^ (r & 15)); }

// Loads of tile t into ring stage `stage`: this wave's 4 K and 4 V row groups (4 rows each).
// The tile offset goes into the vector offset, which the buffer range check covers.
// Paged KV: krs / vrs are the tile's page rows and toff is 0.
__device__ __forceinline__ void issue_tile(u32x4_t* lds, __amdgpu_buffer_rsrc_t krs,
                                           __amdgpu_buffer_rsrc_t vrs, const uint32_t* voff,
                                           int wv, uint32_t toff, int stage) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4_t* kd = &lds[stage * 2 * TC + (wv + 4 * j) * 64];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)kd, 16, voff[j] + toff, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(kd + TC), 16, voff[j] + toff, 0, 0, 0);
  }
}

// Online softmax of one tile's scores for the wave's 32 query columns (each spread over lanes fr,
// fr+16, fr+32, fr+48): s[qi][kb][r] = S[q = q0 + 16 qi][key = key0 + 16 kb + 4 G + r] (raw,
// unscaled).  p = exp((s - m) / sqrt(128)) as one fma and one exp2 per score (the measured
// alternative, rescaling o only when some lane's max grew by 2^8, was 8% slower: the wave-uniform
// branch costs more than the 64 multiplies it skips); MASK applies the causal and end-of-keys
// mask (key <= q, key < nkeys).  Rescales l and o by the max's change and
// packs P^T as the P.V MFMA's B operand: contraction slot 8 G + r <-> key 32 ks2 + 4 G + r, slot
// 8 G + 4 + r <-> key 32 ks2 + 16 + 4 G + r.
template <bool MASK, int QI>
__device__ __forceinline__ void softmax_tile(f32x4_t (&s)[QI][4], float (&m)[QI], float (&l)[QI],
                                             f32x4_t (&o)[QI][8], bf16x8_t (&pb)[QI][2], int key0,
                                             int q0, int nkeys, int G) {
  constexpr float c = 0.08838834764831845f * 1.4426950408889634f;  // 1/sqrt(128) (softmax.cu:79) * log2(e)
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) {
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (MASK) {
          const int key = key0 + 16 * kb + 4 * G + r;
          if (!(key <= q0 + 16 * qi && key < nkeys)) s[qi][kb][r] = -INFINITY;
        }
        mt = fmaxf(mt, s[qi][kb][r]);
      }
    mt = xor32_max(xor16_max(mt));
    // a query row whose keys in this tile are all masked keeps mn = m (finite after its first
    // tile, which always holds key 0)
    const float mn = fmaxf(m[qi], mt);
    const float nb = -mn * c;
    const float alpha = __builtin_amdgcn_exp2f(fmaf(m[qi], c, nb));  // m = -inf: 0
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[qi][kb][r], c, nb));
        s[qi][kb][r] = e;
        ls += e;
      }
    ls = xor32_sum(xor16_sum(ls));
    l[qi] = l[qi] * alpha + ls;
    m[qi] = mn;
#pragma unroll
    for (int db = 0; db < 8; ++db) o[qi][db] *= alpha;
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      const u32x4_t w = {pack_bf2(s[qi][2 * ks2][0], s[qi][2 * ks2][1]),
                         pack_bf2(s[qi][2 * ks2][2], s[qi][2 * ks2][3]),
                         pack_bf2(s[qi][2 * ks2 + 1][0], s[qi][2 * ks2 + 1][1]),
                         pack_bf2(s[qi][2 * ks2 + 1][2], s[qi][2 * ks2 + 1][3])};
      pb[qi][ks2] = __builtin_bit_cast(bf16x8_t, w);
    }
  }
}

// QI: 16-row query blocks per wave (2: 32 query rows per workgroup; 1: 16, twice the workgroups
// for short prompts).
template <bool PAGED, int QI>
__global__ __launch_bounds__(256, 2) void flash_prefill_kernel(AttnPrefillParams p) {
  __shared__ u32x4_t lds[2 * 2 * TC];  // [stage][K | V][key][16 chunks], 64 KiB
  constexpr int BQ = 16 * QI;

  const int nqb = (p.S + BQ - 1) / BQ;
  // workgroup b -> (query block, kv head): the first half of the grid takes the longest causal
  // extents in descending order, the second half the shortest in ascending order
  const int i = blockIdx.x / kKVHeads, g = blockIdx.x % kKVHeads;
  const int half = (nqb + 1) / 2;
  const int qb = i < half ? nqb - 1 - i : i - half;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int fr = lane & 15, G = lane >> 4;
  const int h = g * kGQA + wave;
  const int row0 = qb * BQ;
  const int rows = min(BQ, p.S - row0);
  const int nkeys = p.start_pos + row0 + rows;
  const int ntiles = (nkeys + BKEY - 1) / BKEY;

  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.k + (size_t)g * kKVPlane), 0, nkeys * kRowBytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.v + (size_t)g * kKVPlane), 0, nkeys * kRowBytes, kBufferFlags);
  // load j of this wave: tile rows 4 (wave + 4j) + lane/16; lane fills LDS slot lane%16 of its
  // row from global chunk (lane%16) ^ (row & 15)
  uint32_t voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * (wave + 4 * j) + (lane >> 4);
    voff[j] = (uint32_t)(r * kRowBytes + (((lane & 15) ^ (r & 15)) * 16));
  }

  // Q^T fragments: qf[qi][ks] = Q[row0 + 16 qi + fr][h][32 ks + 8 G .. +8]
  bf16x8_t qf[QI][4];
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) {
    const int qr = row0 + min(16 * qi + fr, rows - 1);
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(p.q + ((size_t)qr * kQHeads + h) * kHeadDim);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[qi][ks] = __builtin_bit_cast(bf16x8_t, qrow[4 * ks + G]);
  }

  f32x4_t o[QI][8];
#pragma unroll
  for (int qi = 0; qi < QI; ++qi)
#pragma unroll
    for (int db = 0; db < 8; ++db) o[qi][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // m: running max of the raw scores (the scale is applied inside the exponent)
  float m[QI], l[QI];
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) m[qi] = -INFINITY, l[qi] = 0.f;

  // Paged KV: tile t's buffers are its page's rows; the page id of tile t+1 is loaded (a vector
  // load, so the loop's vmcnt wait covers it) while tile t is multiplied.
  constexpr bool paged = PAGED;
  int pg_next = paged ? p.block_table[0] : 0;
  auto tile_rsrc = [&](int t, int page, __amdgpu_buffer_rsrc_t& tk, __amdgpu_buffer_rsrc_t& tv) {
    const bool ok = page >= 0 && page < p.n_pages;
    const size_t base = (size_t)(ok ? page : 0) * kPageElems + (size_t)g * kPageHead;
    const int bytes = ok ? min(BKEY, nkeys - t * BKEY) * kRowBytes : 0;
    tk = __builtin_amdgcn_make_buffer_rsrc((void*)(p.k + base), 0, bytes, kBufferFlags);
    tv = __builtin_amdgcn_make_buffer_rsrc((void*)(p.v + base), 0, bytes, kBufferFlags);
  };
  if constexpr (paged) {
    __amdgpu_buffer_rsrc_t tk, tv;
    tile_rsrc(0, __builtin_amdgcn_readfirstlane(pg_next), tk, tv);
    issue_tile(lds, tk, tv, voff, wv, 0, 0);
    pg_next = p.block_table[min(1, ntiles - 1)];
  } else {
    issue_tile(lds, krs, vrs, voff, wv, 0, 0);
  }
  for (int t = 0; t < ntiles; ++t) {
    // tile t has landed (the only loads in flight) and every wave is done with tile t-1
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (t + 1 < ntiles) {
      if constexpr (paged) {
        __amdgpu_buffer_rsrc_t tk, tv;
        tile_rsrc(t + 1, __builtin_amdgcn_readfirstlane(pg_next), tk, tv);
        issue_tile(lds, tk, tv, voff, wv, 0, (t + 1) & 1);
        pg_next = p.block_table[min(t + 2, ntiles - 1)];
      } else {
        issue_tile(lds, krs, vrs, voff, wv, (uint32_t)((t + 1) * BKEY * kRowBytes), (t + 1) & 1);
      }
    }
    const u32x4_t* kt = &lds[(t & 1) * 2 * TC];
    const u32x4_t* vt = kt + TC;
    const int key0 = t * BKEY;

    // ---- S^T blocks: s[qi][kb][r] = S[q = row0 + 16 qi + fr][key = key0 + 16 kb + 4 G + r]
    f32x4_t s[QI][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int qi = 0; qi < QI; ++qi) s[qi][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, kt[kv_slot(16 * kb + fr, 4 * ks + G)]);
#pragma unroll
        for (int qi = 0; qi < QI; ++qi)
          s[qi][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[qi][ks], s[qi][kb], 0, 0, 0);
      }
    }

    // ---- online softmax; causal masking only on the tiles that reach past the block's first query
    bf16x8_t pb[QI][2];
    if (key0 + BKEY - 1 <= p.start_pos + row0)
      softmax_tile<false, QI>(s, m, l, o, pb, key0, p.start_pos + row0 + fr, nkeys, G);
    else
      softmax_tile<true, QI>(s, m, l, o, pb, key0, p.start_pos + row0 + fr, nkeys, G);

    // ---- O^T[d][q] += V^T[d][keys] . P^T[keys][q]; the V^T fragment of dims 16 db .. +15 and
    //      the slot order above is two transposed 8-byte reads per lane
    const int kr = fr >> 2, dq = fr & 3;  // source-lane role in the transposed read
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int c = 2 * db + (dq >> 1), hb = (dq & 1) * 8;  // chunk and byte of dims 16db + 4dq
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        const int ka = 32 * ks2 + 4 * G + kr, kb2 = ka + 16;
        const char* va = reinterpret_cast<const char*>(&vt[kv_slot(ka, c)]) + hb;
        const char* vb = reinterpret_cast<const char*>(&vt[kv_slot(kb2, c)]) + hb;
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)va);
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)vb);
        const short4_t both[2] = {lo, hi};
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, both);
#pragma unroll
        for (int qi = 0; qi < QI; ++qi)
          o[qi][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[qi][ks2], o[qi][db], 0, 0, 0);
      }
    }
  }

  // ---- o[qi][db][r] = O[q = row0 + 16 qi + fr][d = 16 db + 4 G + r] (unnormalised)
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) {
    if (16 * qi + fr < rows) {
      const float inv = 1.0f / l[qi];
      uint16_t* dst = p.out + (size_t)(row0 + 16 * qi + fr) * kHidden + h * kHeadDim;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const u32x2_t w = {pack_bf2(o[qi][db][0] * inv, o[qi][db][1] * inv),
                           pack_bf2(o[qi][db][2] * inv, o[qi][db][3] * inv)};
        *reinterpret_cast<u32x2_t*>(dst + db * 16 + 4 * G) = w;
      }
    }
  }
}

}  // namespace

int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t st) {
  // the reference-layout planes hold kMaxCtx rows; pages reach kMaxLongCtx positions
  IE_REQUIRE(p.S >= 1 && p.start_pos >= 0 &&
                 p.start_pos + p.S <= (p.block_table ? kMaxLongCtx : kMaxCtx),
             "attn_prefill: rows [%d, %d) exceed the KV cache", p.start_pos, p.start_pos + p.S);
  // 32 query rows per workgroup from S = 1792 (448+ workgroups, two per CU), else 16: measured
  // at S = 1024 / 1280 / 1536 / 1792 / 2048, 16 rows 23.4 / 29.2 / 40.2 / 49.7 / 59.2 us against
  // 32 rows 29.7 / 38.0 / 43.4 / 49.1 / 54.7 us
  const bool wide = p.S >= 1792;
  const int nqb = wide ? (p.S + BQ - 1) / BQ : (p.S + 15) / 16;
  const dim3 grid(nqb * kKVHeads);
  if (p.block_table && wide)
    hipLaunchKernelGGL((flash_prefill_kernel<true, 2>), grid, dim3(256), 0, st, p);
  else if (p.block_table)
    hipLaunchKernelGGL((flash_prefill_kernel<true, 1>), grid, dim3(256), 0, st, p);
  else if (wide)
    hipLaunchKernelGGL((flash_prefill_kernel<false, 2>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((flash_prefill_kernel<false, 1>), grid, dim3(256), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
