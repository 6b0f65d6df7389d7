// Causal GQA prefill attention on MFMA (flash style: online softmax, no S x S
// scores in memory).
//
// Reference: attn (kernels/attn.cu:309-371) materialises QK^T for all 32 heads
// ([32, S, S] fp16, cublasGemmBatchedEx), runs a causal softmax kernel
// (softmax.cu:55-107), multiplies by V and permutes [h, s, d] -> [s, h, d].
//
// Here a wave owns 16 QI query rows of one q head, and the waves of a workgroup are the 4 q heads
// of one kv head (GQA: q head h reads kv head h/4, attn.cu:51-53) times SUB consecutive row
// blocks, so every K/V tile staged in LDS feeds 4 SUB waves.  Per 64-key tile and wave, with
// v_mfma_f32_16x16x32_bf16:
//   S^T[key][q] = K . Q^T      16 QI MFMAs (A = K rows from LDS, B = Q fragments in registers;
//                                the QI 16-query column blocks share every K fragment)
//   online softmax per query column (scale 1/sqrt(128), causal mask key > q)
//   O^T[d][q] += V^T . P^T      16 QI MFMAs; B = P^T straight from the S^T accumulators: the 32
//                                contraction slots of one MFMA are mapped to keys {4G+r, 16+4G+r}
//                                of a 32-key half tile, the same permutation on both operands
//   row sums l[q] += 1^T . P^T  2 QI MFMAs with an all-ones A operand (the sums of the bf16
//                                probabilities that P.V multiplies)
// K and V tiles go global -> LDS with direct-to-LDS buffer loads, row-major [key][128] (chunk c
// of key r at slot c ^ kv_swz(r)), double-buffered so the next tile loads under this tile's
// MFMAs.  The two ring stages are separate arrays and the next tile is issued on every step:
// then the compiler can see that the loads in flight never write the stage being read, and
// does not drain them before the reads.  The A operand of O^T is V^T; gfx950's
// ds_read_b64_tr_b16 reads it from the row-major tile: in each 16-lane group, output lane j
// receives element j % 4 of the 8 bytes read by source lanes 4e + j / 4 (e = 0..3), so with
// source lane s reading V[key0 + s/4][d0 + 4 (s%4) ..+3], lane j gets V[key0 + e][d0 + j],
// e = 0..3: four consecutive keys of one dim.  Rows past the last key read as zero (buffer
// bounds), so the masked tail never multiplies garbage.  Workgroups are issued longest causal
// extent first, paired so that the two a CU holds sum to about the mean.  Output rows are
// [s][h][d] (the attn_permute.cu:15-31 layout), bf16.
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) short4_t lds_short4;

constexpr int BKEY = 64;              // keys per LDS tile
constexpr int TC = BKEY * 16;         // 16-byte chunks per K (or V) tile
constexpr int kRowBytes = kHeadDim * 2;
constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw 32-bit access)

// Chunk swizzle of key row r, a bijection of r's low 4 bits b3 b2 b1 b0 -> (b2^b3) b1 b0 b2.
// Conflict-free (whether the LDS serves 128 or 256 bytes a clock) for both read patterns: the K
// fragment reads (16 consecutive rows of one chunk column: the low 3 bits, and all 4, are a
// bijection of the row) and the transposed V reads (rows 4G..4G+3, or 8j..8j+7, each with the
// chunk pair 2 db + {0, 1}: bits 1-2, and bits 1-3 with b3 fixed, are a bijection of the row).
// The plain r & 15 left the V reads 2-way conflicted (a third of all LDS cycles).
__device__ __forceinline__ int kv_swz(int r) {
  return ((((r >> 2) ^ (r >> 3)) & 1) << 3) | ((r & 3) << 1) | ((r >> 2) & 1);
}
__device__ __forceinline__ int kv_slot(int r, int c) { return r * 16 + (c ^ kv_swz(r)); }

// Loads of one tile into a stage (K at stage[0..TC), V at stage[TC..2TC)) by 4 waves: this
// wave's 4 K and 4 V row groups (4 rows each).  The tile offset goes into the vector offset,
// which the buffer range check covers.  Paged KV: krs / vrs are the tile's page rows, toff 0.
__device__ __forceinline__ void issue_tile4(u32x4_t* stage, __amdgpu_buffer_rsrc_t krs,
                                            __amdgpu_buffer_rsrc_t vrs, const uint32_t* voff,
                                            int wv, uint32_t toff) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4_t* kd = stage + (wv + 4 * j) * 64;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)kd, 16, voff[j] + toff, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(kd + TC), 16, voff[j] + toff, 0, 0, 0);
  }
}

// The same by 8 waves: this wave's 2 K and 2 V row groups.
__device__ __forceinline__ void issue_tile8(u32x4_t* stage, __amdgpu_buffer_rsrc_t krs,
                                            __amdgpu_buffer_rsrc_t vrs, const uint32_t* voff,
                                            int wv, uint32_t toff) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    u32x4_t* kd = stage + (wv + 8 * j) * 64;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)kd, 16, voff[j] + toff, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(kd + TC), 16, voff[j] + toff, 0, 0, 0);
  }
}

// Online softmax of one tile's scores for the wave's 16 QI query columns (each spread over lanes
// fr, fr+16, fr+32, fr+48): s[qi][kb][r] = S[q = q0 + 16 qi][key = key0 + 16 kb + 4 G + r] (raw,
// unscaled).  p = exp((s - m) / sqrt(128)) as one fma and one exp2 per score; MASK applies the
// causal and end-of-keys mask (key <= q, key < nkeys).  Rescales o by the max's change and
// returns that factor in alpha (the caller rescales the row sums), and packs P^T as the P.V
// MFMA's B operand: contraction slot 8 G + r <-> key 32 ks2 + 4 G + r, slot 8 G + 4 + r <->
// key 32 ks2 + 16 + 4 G + r.  (Measured and not kept: rescaling o only when some lane's max
// grew by 2^8, behind a wave-uniform branch -- no faster.)
template <bool MASK, int QI>
__device__ __forceinline__ void softmax_tile(f32x4_t (&s)[QI][4], float (&m)[QI],
                                             float (&alpha)[QI], f32x4_t (&o)[QI][8],
                                             bf16x8_t (&pb)[QI][2], int key0, int q0, int nkeys,
                                             int G) {
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
    alpha[qi] = __builtin_amdgcn_exp2f(fmaf(m[qi], c, nb));  // m = -inf: 0
    m[qi] = mn;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[qi][kb][r] = __builtin_amdgcn_exp2f(fmaf(s[qi][kb][r], c, nb));
#pragma unroll
    for (int db = 0; db < 8; ++db) o[qi][db] *= alpha[qi];
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

// QI: 16-row query blocks per wave (1 or 2); SUB: row blocks per workgroup (1: 4 waves, 2: 8
// waves, the two halves of the workgroup's rows).  A wave whose rows end before the
// workgroup's last tile skips that tile's work but still passes its barrier.
template <bool PAGED, int QI, int SUB>
__global__ __launch_bounds__(256 * SUB, (QI == 2 && SUB == 2) ? 1 : 2) void flash_prefill_kernel(
    AttnPrefillParams p) {
  __shared__ u32x4_t lds0[2 * TC];  // ring stage 0: [K | V][key][16 chunks], 32 KiB
  __shared__ u32x4_t lds1[2 * TC];  // ring stage 1
  constexpr int NW = 4 * SUB;       // waves
  constexpr int BW = 16 * QI;       // query rows per wave
  constexpr int BQ = BW * SUB;      // query rows per workgroup

  const int nqb = (p.S + BQ - 1) / BQ;
  // workgroup b -> (query block, kv head): the first half of the grid takes the longest causal
  // extents in descending order, the second half the shortest in ascending order
  const int i = blockIdx.x / kKVHeads, g = blockIdx.x % kKVHeads;
  const int half = (nqb + 1) / 2;
  const int qb = i < half ? nqb - 1 - i : i - half;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int fr = lane & 15, G = lane >> 4;
  const int h = g * kGQA + (wv & 3);
  const int row0 = qb * BQ;
  const int rows = min(BQ, p.S - row0);
  const int nkeys = p.start_pos + row0 + rows;
  const int ntiles = (nkeys + BKEY - 1) / BKEY;
  // this wave's rows (with SUB = 2 the second half may be empty in the last block)
  const int wrow0 = row0 + (wv >> 2) * BW;
  const int wrows = min(BW, p.S - wrow0);
  const int wtiles = wrows > 0 ? (p.start_pos + wrow0 + wrows + BKEY - 1) / BKEY : 0;

  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.k + (size_t)g * kKVPlane), 0, nkeys * kRowBytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.v + (size_t)g * kKVPlane), 0, nkeys * kRowBytes, kBufferFlags);
  // load j of this wave: tile rows 4 (wave + NW j) + lane/16; lane fills LDS slot lane%16 of its
  // row from global chunk (lane%16) ^ kv_swz(row)
  uint32_t voff[16 / NW];
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int r = 4 * (wave + NW * j) + (lane >> 4);
    voff[j] = (uint32_t)(r * kRowBytes + (((lane & 15) ^ kv_swz(r)) * 16));
  }

  // Q^T fragments: qf[qi][ks] = Q[wrow0 + 16 qi + fr][h][32 ks + 8 G .. +8]
  bf16x8_t qf[QI][4];
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) {
    const int qr = wrows > 0 ? wrow0 + min(16 * qi + fr, wrows - 1) : row0;
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(p.q + ((size_t)qr * kQHeads + h) * kHeadDim);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[qi][ks] = __builtin_bit_cast(bf16x8_t, qrow[4 * ks + G]);
  }

  f32x4_t o[QI][8];
#pragma unroll
  for (int qi = 0; qi < QI; ++qi)
#pragma unroll
    for (int db = 0; db < 8; ++db) o[qi][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // m: running max of the raw scores (the scale is applied inside the exponent); lsum[qi][0]:
  // running row sum (lanes of the ones-MFMA's other output rows are not rescaled and unused)
  float m[QI], alpha[QI];
  f32x4_t lsum[QI];
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) m[qi] = -INFINITY, lsum[qi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const u32x4_t ones_w = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_w);

  // byte offsets within a stage: K fragment ks of key row fr (+ 4096 per 16-key block), and the
  // transposed V read of dims 16 db + 4 (fr % 4) .. for keys 4 G + fr / 4 (+ 8192 per 32-key
  // half, + 4096 for keys + 16)
  const int kr = fr >> 2, dq = fr & 3;
  uint32_t koffs[4], voffs[8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koffs[ks] = (uint32_t)kv_slot(fr, 4 * ks + G) * 16;
#pragma unroll
  for (int db = 0; db < 8; ++db)
    voffs[db] = (uint32_t)(TC + kv_slot(4 * G + kr, 2 * db + (dq >> 1))) * 16 + (dq & 1) * 8;

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
  auto issue = [&](u32x4_t* dst, __amdgpu_buffer_rsrc_t tk, __amdgpu_buffer_rsrc_t tv,
                   uint32_t toff) {
    if constexpr (SUB == 1)
      issue_tile4(dst, tk, tv, voff, wv, toff);
    else
      issue_tile8(dst, tk, tv, voff, wv, toff);
  };
  if constexpr (paged) {
    __amdgpu_buffer_rsrc_t tk, tv;
    tile_rsrc(0, __builtin_amdgcn_readfirstlane(pg_next), tk, tv);
    issue(lds0, tk, tv, 0);
    pg_next = p.block_table[min(1, ntiles - 1)];
  } else {
    issue(lds0, krs, vrs, 0);
  }

  auto step = [&](int t, const u32x4_t* cur, u32x4_t* nxt) {
    // tile t has landed (the only loads in flight) and every wave is done with tile t-1
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // tile t+1 is issued unconditionally: past the last tile the buffer range is empty and the
    // loads return zeros into the idle stage
    if constexpr (paged) {
      __amdgpu_buffer_rsrc_t tk, tv;
      tile_rsrc(t + 1, t + 1 < ntiles ? __builtin_amdgcn_readfirstlane(pg_next) : -1, tk, tv);
      issue(nxt, tk, tv, 0);
      pg_next = p.block_table[min(t + 2, ntiles - 1)];
    } else {
      issue(nxt, krs, vrs, (uint32_t)((t + 1) * BKEY * kRowBytes));
    }
    if (t >= wtiles) return;  // this wave's rows end before tile t (wave-uniform)
    const char* kb8 = reinterpret_cast<const char*>(cur);
    const int key0 = t * BKEY;

    // ---- S^T blocks: s[qi][kb][r] = S[q = wrow0 + 16 qi + fr][key = key0 + 16 kb + 4 G + r]
    f32x4_t s[QI][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int qi = 0; qi < QI; ++qi) s[qi][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(kb8 + koffs[ks] + kb * 4096);
#pragma unroll
        for (int qi = 0; qi < QI; ++qi)
          s[qi][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[qi][ks], s[qi][kb], 0, 0, 0);
      }
    }

    // ---- online softmax; causal masking only on the tiles that reach past the wave's first query
    bf16x8_t pb[QI][2];
    if (key0 + BKEY - 1 <= p.start_pos + wrow0)
      softmax_tile<false, QI>(s, m, alpha, o, pb, key0, p.start_pos + wrow0 + fr, nkeys, G);
    else
      softmax_tile<true, QI>(s, m, alpha, o, pb, key0, p.start_pos + wrow0 + fr, nkeys, G);
#pragma unroll
    for (int qi = 0; qi < QI; ++qi) {
      lsum[qi][0] *= alpha[qi];
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
        lsum[qi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[qi][ks2], lsum[qi], 0, 0, 0);
    }

    // ---- O^T[d][q] += V^T[d][keys] . P^T[keys][q]; the V^T fragment of dims 16 db .. +15 is
    //      two transposed 8-byte reads per lane
#pragma unroll
    for (int db = 0; db < 8; ++db) {
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        const char* va = kb8 + voffs[db] + ks2 * 8192;
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)va);
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(va + 4096));
        const short4_t both[2] = {lo, hi};
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, both);
#pragma unroll
        for (int qi = 0; qi < QI; ++qi)
          o[qi][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[qi][ks2], o[qi][db], 0, 0, 0);
      }
    }
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, lds0, lds1);
    if (t + 1 < ntiles) step(t + 1, lds1, lds0);
  }

  // ---- o[qi][db][r] = O[q = wrow0 + 16 qi + fr][d = 16 db + 4 G + r] (unnormalised)
#pragma unroll
  for (int qi = 0; qi < QI; ++qi) {
    if (16 * qi + fr < wrows) {
      const float inv = 1.0f / lsum[qi][0];
      uint16_t* dst = p.out + (size_t)(wrow0 + 16 * qi + fr) * kHidden + h * kHeadDim;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const u32x2_t w = {pack_bf2(o[qi][db][0] * inv, o[qi][db][1] * inv),
                           pack_bf2(o[qi][db][2] * inv, o[qi][db][3] * inv)};
        *reinterpret_cast<u32x2_t*>(dst + db * 16 + 4 * G) = w;
      }
    }
  }
}

template <int QI, int SUB>
void launch_form(const AttnPrefillParams& p, hipStream_t st) {
  const int bq = 16 * QI * SUB;
  const dim3 grid(((p.S + bq - 1) / bq) * kKVHeads), block(256 * SUB);
  if (p.block_table)
    hipLaunchKernelGGL((flash_prefill_kernel<true, QI, SUB>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((flash_prefill_kernel<false, QI, SUB>), grid, block, 0, st, p);
}

}  // namespace

int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t st) {
  // the reference-layout planes hold kMaxCtx rows; pages reach kMaxLongCtx positions
  IE_REQUIRE(p.S >= 1 && p.start_pos >= 0 &&
                 p.start_pos + p.S <= (p.block_table ? kMaxLongCtx : kMaxCtx),
             "attn_prefill: rows [%d, %d) exceed the KV cache", p.start_pos, p.start_pos + p.S);
  // 16 rows per wave in 4-wave workgroups below 1280 query rows, 8-wave workgroups (two 16-row
  // blocks, 4 waves per SIMD) up to 2560, 32 rows per wave above (half the LDS reads per query
  // row): measured at S = 512 / 1024 / 1536 / 2048 / 2560 / 4096, 10.8 / 20.2 / 36.2 / 55.3 /
  // 81.6 / 179.6 us, 13.3 / 23.3 / 34.1 / 45.1 / 70.3 / 161.3 us and 15.2 / 26.0 / 38.0 / 48.2 /
  // 65.9 / 148.0 us
  if (p.S < 1280)
    launch_form<1, 1>(p, st);
  else if (p.S < 2560)
    launch_form<1, 2>(p, st);
  else
    launch_form<2, 1>(p, st);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace ie
