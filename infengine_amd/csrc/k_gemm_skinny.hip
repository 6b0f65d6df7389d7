// Skinny MFMA GEMM for batched decode (M <= 16 rows):
//   Y[M, N] = X[M, K] . W[N, K]^T      (fp32 accumulate)
//
// Reference: multiply_by_weight (kernels/ffn.cu:7-33) with m = batch rows.  At m <= 16 the
// product is HBM-bound on W exactly like the m = 1 GEMV, so the kernel is built for streaming:
// a workgroup owns 16 weight rows (output columns) and its 4 waves split K in quarters; each
// wave runs v_mfma_f32_16x16x32_bf16 with the 16 weight rows as A and the (up to) 16 X rows
// as B, and the quarters are summed through LDS.  Grid = N / 16 workgroups (256 for N = 4096,
// 8016 for the lm_head), enough to fill the chip where a 128-row tile GEMM had 32.  The SwiGLU
// and QKV projections (896 and 384 tiles: 3.5 and 1.5 per CU) run their last partial round of
// tiles as two workgroups each, one per K half, so that every CU streams the same share; the
// second half to finish adds the first's fp32 partials and stores the tile (no waiting).
//
// Load pattern: a step covers 128 k (256 bytes of each of the tile's 16 weight rows) as 4 MFMA
// k-chunks of 32.  The MFMA operand layout (lane l: row l % 16, 8 k at 8 (l / 16)) would make
// each load instruction read 64 bytes of 16 rows -- half a cache line per row, which measured
// 25-35% slower than whole rows -- so W is loaded as 4 rows x 256 contiguous bytes per
// instruction and transposed through a wave-private LDS tile (one 16-byte write and one
// 16-byte read per lane per instruction; the slot of row R's 16-byte chunk c is R*16 + (c ^ R),
// conflict-free both ways).  LDS operations of one wave run in order, so the tile needs no
// barrier.  X (L2-resident) takes the same path as one more 16-row tile.  D = W . X^T: lane l holds
// output row m = l % 16 and 4 consecutive output columns n = 4 (l / 16) + i.
//
// Epilogues as the MFMA GEMM: bf16, residual add, fp32, and SwiGLU (gate and up rows of the
// same 16 columns in one workgroup, lane-local silu(bf16(g)) * bf16(u)); and QKV + RoPE for
// batched decode: workgroup b owns RoPE pairs 8 (b % 8) .. +7 of head b / 8 (its 16 weight rows
// are those pairs' first halves, then their second halves), so lane l and lane l ^ 32 hold the
// two halves of the same 4 pairs and one cross-lane swap gives each both.
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSkRows = 16;   // weight rows (output columns) per workgroup
constexpr int kSkSplit = 4;   // waves per workgroup = K quarters
constexpr int kSkStep = 128;  // k per step
// Folded RMSNorm: each of a row's 16 summing threads takes kSsLoads float4 partials, the row's
// kNormParts partial sums of squares (one per producer workgroup, zeros where fewer produce).
constexpr int kSsLoads = 4;
static_assert(kNormParts == 16 * 4 * kSsLoads, "kNormParts partials per row");

constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw 32-bit access)

// Operand sources of one workgroup: buffer resources whose byte ranges end at the last row the
// tile may read (rows past a matrix end or past M read as zero; their outputs are not stored),
// and per-lane 32-bit byte offsets of row 4j + q, 16-byte chunk r, of each source.
struct SkSrc {
  __amdgpu_buffer_rsrc_t w[2];  // the W tiles: the weight rows, or gate and up rows
  __amdgpu_buffer_rsrc_t x;
  __amdgpu_buffer_rsrc_t nul;   // an empty range: loads through it read zeros and no memory
  uint32_t wo[4], xo[4];
};

// (the byte count is made provably uniform: a row count clamped with min/max can come out of a
// VALU instruction, and a descriptor in VGPRs turns every load into a readfirstlane loop)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const uint16_t* base, int rows, int K) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0,
                                           __builtin_amdgcn_readfirstlane(rows * K * 2),
                                           kBufferFlags);
}

// Loads of one step (k offset ks from each row start), 4 rows x 256 bytes per instruction: lane
// (r, q) loads 16-byte chunk r of row 4j + q of each W tile, or of the X rows.  The weights are
// read exactly once per launch: nontemporal loads (cache policy nt), as the GEMV's; measured 8-10%
// faster per projection than the default policy (the X rows, re-read by every workgroup, keep it).
// live = false reads through the empty range instead (a uniform select, not a branch: a load
// under a run-time condition makes the compiler wait for every load in flight where the paths
// join).
template <int NT>
__device__ __forceinline__ void sk_load_w(const SkSrc& src, int ks, u32x4_t (&w)[NT][4],
                                          bool live = true) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const __amdgpu_buffer_rsrc_t rs = live ? src.w[t] : src.nul;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[t][j] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, src.wo[j], 2 * ks, 2));
  }
}

__device__ __forceinline__ void sk_load_x(const SkSrc& src, int ks, u32x4_t (&xv)[4],
                                          bool live = true) {
  const __amdgpu_buffer_rsrc_t rs = live ? src.x : src.nul;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    xv[j] = __builtin_bit_cast(
        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, src.xo[j], 2 * ks, 0));
}

// One 16-row tile into a wave's LDS tile: row R's 16-byte chunk c goes to slot R*16 + (c ^ R).
__device__ __forceinline__ void sk_put(u32x4_t* t, const u32x4_t (&v)[4], int r, int q) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int R = 4 * j + q;
    t[R * 16 + (r ^ R)] = v[j];
  }
}

// rmsnorm.cu:61's two roundings on one packed pair of an X row: bf16(bf16(x * r) * w).
__device__ __forceinline__ uint32_t norm2(uint32_t x, uint32_t w, float r) {
  const uint32_t t = pack_bf2(bf_lo(x) * r, bf_hi(x) * r);
  return pack_bf2(bf_lo(t) * bf_lo(w), bf_hi(t) * bf_hi(w));
}

// RMSNorm of the X operand inside the projection: rr[j] = 1/rms of the lane's row 4j + q, nw =
// the norm weight's 8 values at the lane's chunk of the current step (refilled with the X rows).
struct SkNorm {
  const uint16_t* w;
  float rr[4];
  u32x4_t nw;
};

__device__ __forceinline__ u32x4_t sk_load_nw(const uint16_t* w, int ks, int r) {
  return *reinterpret_cast<const u32x4_t*>(w + ks + 8 * r);
}

__device__ __forceinline__ void sk_norm_x(u32x4_t (&xv)[4], const SkNorm& nm) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[j][i] = norm2(xv[j][i], nm.nw[i], nm.rr[j]);
}

// One step: the X rows (tr[1]) and each W tile in turn (tr[0]; the second W tile overwrites the
// first once its fragments are read -- one wave's LDS operations run in order) through the
// wave's LDS tiles into the operand layout, 4 MFMA k-chunks per W tile (the MFMA's 32-k
// contraction of chunk c is k = 32c .. 32c+31 of the step for both operands: chunk 4c + q of W
// row r and of X row r).  The X registers are refilled with step kx as soon as they are in LDS
// (X is L2-resident: one step of lookahead hides it), the W registers with step kw once the last
// W tile is in LDS.
template <int NT, bool NORM>
__device__ __forceinline__ void sk_step(u32x4_t (*tr)[256], const SkSrc& src, u32x4_t (&w)[NT][4],
                                        u32x4_t (&xv)[4], int r, int q, f32x4_t (&acc)[NT],
                                        bool lx, int kx, bool lw, int kw, SkNorm& nm,
                                        bool xlive = true, bool wlive = true) {
  sk_put(tr[0], w[0], r, q);
  if constexpr (NORM) sk_norm_x(xv, nm);
  sk_put(tr[1], xv, r, q);
  if (lx) {
    // (a step that is not live reads X through the empty range and re-reads the start of the
    // norm weight, a plain array)
    sk_load_x(src, kx, xv, xlive);
    if constexpr (NORM) nm.nw = sk_load_nw(nm.w, xlive ? kx : 0, r);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t > 0) sk_put(tr[0], w[t], r, q);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8_t, tr[0][r * 16 + ((4 * c + q) ^ r)]),
          __builtin_bit_cast(bf16x8_t, tr[1][r * 16 + ((4 * c + q) ^ r)]), acc[t], 0, 0, 0);
  }
  if (lw) sk_load_w<NT>(src, kw, w, wlive);
}

// Steps s and s+1 from the two W register buffers, each refilled with the step two ahead; X
// one step ahead.
// (loads are issued for the steps below `steps`, and read memory for those below `live`)
template <int NT, bool NORM>
__device__ __forceinline__ void sk_pair(u32x4_t (*tr)[256], const SkSrc& src, int kbase, int s,
                                        int steps, int r, int q, u32x4_t (&w0)[NT][4],
                                        u32x4_t (&w1)[NT][4], u32x4_t (&xv)[4],
                                        f32x4_t (&acc)[NT], SkNorm& nm, int live) {
  const int k1 = kbase + (s + 1) * kSkStep;
  sk_step<NT, NORM>(tr, src, w0, xv, r, q, acc, s + 1 < steps, k1, s + 2 < steps, k1 + kSkStep,
                    nm, s + 1 < live, s + 2 < live);
  __builtin_amdgcn_sched_barrier(0);
  sk_step<NT, NORM>(tr, src, w1, xv, r, q, acc, s + 2 < steps, k1 + kSkStep, s + 3 < steps,
                    k1 + 2 * kSkStep, nm, s + 2 < live, s + 3 < live);
  __builtin_amdgcn_sched_barrier(0);
}

// KC: K fixed at compile time (4096 or 14336; the step loop then unrolls fully), 0: at run time.
// At most 128 VGPRs (fixed K) and 32 KiB of LDS: 4 workgroups per CU, so the 896 workgroups of
// the gate/up projection are all resident at once (the same speed, measured, as 2 per CU).
// NORM: the X rows are the raw rows of an RMSNorm input, normalised on their way into LDS.
// The normalising SwiGLU instance gets the registers of 2 waves per SIMD (2 workgroups per CU;
// at 4 its 128-register cap slowed it by a quarter).
template <int EPI, int KC, bool NORM>
__global__ __launch_bounds__(kSkSplit * 64) __attribute__((
    amdgpu_waves_per_eu(KC > 0 ? (NORM && EPI == kGemmSwiglu ? 2 : 4) : 1)))
void gemm_skinny_kernel(GemmParams p) {
  constexpr bool SW = EPI == kGemmSwiglu;
  // The fp32 epilogue (the lm_head: 8016 16-row tiles) at a compile-time K takes 32-row tiles:
  // two 16-row W tiles against each X step, which halves the X re-reads per weight byte (as
  // many bytes as the weights for a 16-row tile); lm_head at M = 16 183.6 -> 163.5 us.  The
  // 4096-column projections keep 16-row tiles: at 32 rows their 128 tiles need K halves to fill
  // the chip, and the halves' hand-off (write-through stores, arrival counter, reads) ends these
  // short kernels ~2 us later (O 9.05 -> 10.34 us, down 22.69 -> 22.52 in the batched step).
  constexpr bool WIDE = KC > 0 && EPI == kGemmF32;
  constexpr int NT = (SW || WIDE) ? 2 : 1;  // 16-row W tiles: rows n0.. and n0+16.., or gate and up
  constexpr int TROWS = WIDE ? 2 * kSkRows : kSkRows;  // output columns per tile
  __shared__ u32x4_t tr[kSkSplit][2][256];  // per wave: a W tile and the X rows
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  // tiles 0 .. tfull-1 are one workgroup each; each of the p.sk_tail tiles after them is two,
  // K half 0 then K half 1 (the second to arrive sums the halves and runs the epilogue)
  constexpr bool TAIL = KC > 0 && (SW || WIDE || EPI == kGemmQkvRope);  // (the launcher checks sk_tail)
  const int tfull = gridDim.x - 2 * p.sk_tail;
  int tile = blockIdx.x, half = -1;
  if (TAIL && (int)blockIdx.x >= tfull) {
    tile = tfull + ((blockIdx.x - tfull) >> 1);
    half = (blockIdx.x - tfull) & 1;
  }
  const int n0 = tile * TROWS;
  const int K = KC > 0 ? KC : p.K;

  SkSrc src;
  // row offset of tile row 4j + q within the W source
  int wrow[4];
  if constexpr (EPI == kGemmQkvRope) {
    // head b / 8 of the [q|k|v] rows; the tile's rows are pairs 8 (b % 8) .. +7, first halves
    // (rows 0..7) then second halves (rows 8..15, 64 rows further on)
    const int head = tile >> 3, pr = (tile & 7) * 8;
    const uint16_t* base = head < kQHeads ? p.w0 + (size_t)head * kHeadDim * K
                           : head < kQHeads + kKVHeads
                               ? p.w1 + (size_t)(head - kQHeads) * kHeadDim * K
                               : p.w2 + (size_t)(head - kQHeads - kKVHeads) * kHeadDim * K;
    src.w[0] = sk_rsrc(base, kHeadDim, K);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int R = 4 * j + q;
      wrow[j] = pr + (R & 7) + 64 * (R >> 3);
    }
  } else {
    if constexpr (SW) {
      const int rows = min(kSkRows, p.N - n0);
      src.w[0] = sk_rsrc(p.w0 + (size_t)n0 * K, rows, K);  // gate
      src.w[1] = sk_rsrc(p.w1 + (size_t)n0 * K, rows, K);  // up
    } else {
      // the weight matrix holding the tile (the launch keeps tiles inside one matrix)
      const int e0 = min(p.n0, p.N), e1 = min(p.n0 + p.n1, p.N);
      const uint16_t* base;
      int end;
      if (n0 < e0) base = p.w0 + (size_t)n0 * K, end = e0;
      else if (n0 < e1) base = p.w1 + (size_t)(n0 - e0) * K, end = e1;
      else base = p.w2 + (size_t)(n0 - e1) * K, end = p.N;
      src.w[0] = sk_rsrc(base, min(kSkRows, end - n0), K);
      if constexpr (WIDE)
        src.w[1] = sk_rsrc(base + (size_t)kSkRows * K, max(0, min(kSkRows, end - n0 - kSkRows)), K);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) wrow[j] = 4 * j + q;
  }
  src.x = sk_rsrc(p.x, p.M, K);
  src.nul = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, 0, kBufferFlags);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    src.wo[j] = (uint32_t)(wrow[j] * K + 8 * r) * 2u;
    src.xo[j] = (uint32_t)((4 * j + q) * K + 8 * r) * 2u;
  }
  // kept as per-lane values: folding a row's uniform part into the scalar offset would take it
  // out of the buffer range check on the rows past the matrix end
  asm volatile("" : "+v"(src.wo[0]), "+v"(src.wo[1]), "+v"(src.wo[2]), "+v"(src.wo[3]));
  asm volatile("" : "+v"(src.xo[0]), "+v"(src.xo[1]), "+v"(src.xo[2]), "+v"(src.xo[3]));
  // wave w takes K quarter w (interleaving the waves' steps, so that the 4 waves read 1 KiB runs
  // of each row together, measured 4-6% slower)
  const int kq = half < 0 ? K / kSkSplit : K / (2 * kSkSplit);
  const int kbase = (half < 0 ? 0 : half * (K / 2)) + wave * kq;
  const int steps = kq / kSkStep;

  f32x4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // two W register buffers: step s is multiplied while step s+1 is in flight, then buffer s % 2
  // is refilled with step s+2; the X rows of step s+1 are loaded during step s, ahead of the W
  // rows of step s+2 (loads return in issue order)
  u32x4_t w0[NT][4], w1[NT][4], xv[4];
  // RMSNorm of the X rows: the rows' sums of squares from the producer's partials, [16][ss_parts]
  // (a multiple of 4).  Loaded before the first weight loads and summed after them: loads return
  // in issue order, so waiting for these does not wait for the weights.
  __shared__ float ssr[16];
  float4 ssv[kSsLoads];
  SkNorm nm;
  const int ss_row = threadIdx.x >> 4, ss_lane = threadIdx.x & 15;
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < kSsLoads; ++i) {
      const int b = 4 * (ss_lane + 16 * i);
      // (every row has kNormParts partials, so no load is conditional: a load under a
      // condition made the compiler wait for each one before the weight stream started)
      ssv[i] = *reinterpret_cast<const float4*>(p.ss_in + ss_row * kNormParts + b);
    }
  }
  // Epilogue operands, loaded ahead of the weight stream so that the epilogue does not end the
  // workgroup on load latencies: the residual columns, or the RoPE position (then its angles and
  // page below).  Every wave loads them (wave 0 stores the outputs): no load is conditional.
  const int em = min(r, max(p.M - 1, 0));
  int epos = 0;  // (the sequence length here; the position after the weight loads are issued)
  uint2 eold[NT];
  if constexpr (EPI == kGemmQkvRope) epos = p.d_seq_len[em];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    eold[t] = make_uint2(0u, 0u);
    const int en = min(n0 + kSkRows * t + 4 * q, max(p.N - 4, 0));
    if constexpr (EPI == kGemmResid) eold[t] = *reinterpret_cast<const uint2*>(p.y + (size_t)em * p.ldy + en);
  }
  __builtin_amdgcn_sched_barrier(0);
  sk_load_w<NT>(src, kbase, w0);
  sk_load_x(src, kbase, xv);
  if constexpr (NORM) {
    nm.w = p.x_norm_w;
    nm.nw = sk_load_nw(nm.w, kbase, r);
  }
  if (KC > 0 || steps > 1) sk_load_w<NT>(src, kbase + kSkStep, w1);
  float ecos[4], esin[4];
  int epage = 0;
  if constexpr (EPI == kGemmQkvRope) {
    epos -= 1;
    const int jp = (tile & 7) * 8 + 4 * (q & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ecos[i] = p.rope_cos[epos * 64 + jp + i];
      esin[i] = p.rope_sin[epos * 64 + jp + i];
    }
    // (a table entry of row 0 when the cache is not paged: the load stays unconditional)
    const int* bt = p.block_table ? p.block_table + (size_t)em * p.table_stride + epos / kPagePos
                                  : p.d_seq_len;
    epage = *bt;
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NORM) {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kSsLoads; ++i) sum += (ssv[i].x + ssv[i].y) + (ssv[i].z + ssv[i].w);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) sum += __shfl_xor(sum, o, 16);
    if (ss_lane == 0) ssr[ss_row] = sum;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) nm.rr[j] = rsqrtf(ssr[4 * j + q] / (float)K + kRmsEps);
  }
  int s = 0;
  if constexpr (KC > 0 && !TAIL) {
#pragma unroll
    for (; s + 1 < KC / kSkSplit / kSkStep; s += 2)
      sk_pair<NT, NORM>(tr[wave], src, kbase, s, steps, r, q, w0, w1, xv, acc, nm, steps);
  } else if constexpr (KC > 0) {
    // steps of a whole tile; a K half runs the first FS / 2 (the same code, its lookahead loads
    // past them switched off by the run-time step count)
    constexpr int FS = KC / kSkSplit / kSkStep;
    static_assert(FS % 4 == 0, "whole and half tiles run in step pairs");
#pragma unroll
    for (int s0 = 0; s0 < FS / 2; s0 += 2)
      sk_pair<NT, NORM>(tr[wave], src, kbase, s0, FS, r, q, w0, w1, xv, acc, nm, steps);
    s = FS / 2;
    if (half < 0) {
#pragma unroll
      for (int s0 = FS / 2; s0 < FS; s0 += 2)
        sk_pair<NT, NORM>(tr[wave], src, kbase, s0, FS, r, q, w0, w1, xv, acc, nm, FS);
      s = FS;
    }
  } else {
    for (; s + 1 < steps; s += 2)
      sk_pair<NT, NORM>(tr[wave], src, kbase, s, steps, r, q, w0, w1, xv, acc, nm, steps);
  }
  if (s < steps) sk_step<NT, NORM>(tr[wave], src, w0, xv, r, q, acc, false, 0, false, 0, nm);
  f32x4_t acc0 = acc[0], acc1 = acc[NT - 1];

  // sum the K quarters: waves 1..3 hand their tiles to wave 0 through their own W tile slots
  // (each wave's last reads of its slot precede these writes)
  tr[wave][0][lane] = __builtin_bit_cast(u32x4_t, acc0);
  if constexpr (NT == 2) tr[wave][0][64 + lane] = __builtin_bit_cast(u32x4_t, acc1);
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kSkSplit; ++w) {
    acc0 += __builtin_bit_cast(f32x4_t, tr[w][0][lane]);
    if constexpr (NT == 2) acc1 += __builtin_bit_cast(f32x4_t, tr[w][0][64 + lane]);
  }
  if constexpr (TAIL) {
    if (half >= 0) {
      // A K half: store this half's partials, then count the tile's arrivals; the second to
      // arrive adds the other half's (a + b: the same sum whichever half arrives last) and
      // stores the tile.  The halves may run on different XCDs, whose L2s are not coherent with
      // each other: device-scope stores and loads, and the stores performed (vmcnt) before the
      // count, which is a device-scope atomic.
      float* const part = p.sk_part + (size_t)(tile - tfull) * (4 * 64 * 4);
      float* const mine = part + half * (2 * 64 * 4) + 4 * lane;
      const float* const other = part + (half ^ 1) * (2 * 64 * 4) + 4 * lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __hip_atomic_store(mine + i, acc0[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (NT == 2)
          __hip_atomic_store(mine + 256 + i, acc1[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      unsigned int* const cnt = p.sk_cnt + (size_t)(tile - tfull) * kCntStride;
      unsigned int prev = 0;
      if (lane == 0) prev = atomicAdd(cnt, 1u);
      if (__builtin_amdgcn_readfirstlane(prev) == 0) return;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc0[i] += __hip_atomic_load(other + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (NT == 2)
          acc1[i] +=
              __hip_atomic_load(other + 256 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  const int m = r, n = n0 + 4 * q;
  if constexpr (EPI == kGemmResid) {
    if (p.ss_out) {
      // the new residual rows and each 16-column tile's share of each row's sum of squares (for
      // the next projection's RMSNorm: partial n / 16 of kNormParts; lanes q = 0..3 hold 4
      // columns each)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const f32x4_t a = t == 0 ? acc0 : acc1;
        const int nt = n + kSkRows * t;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (m < p.M && nt < p.N) {
          uint2* dst = reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + nt);
          const uint2 old = eold[t];
          v[0] = bf2f(f2bf(bf_lo(old.x) + bf2f(f2bf(a[0]))));
          v[1] = bf2f(f2bf(bf_hi(old.x) + bf2f(f2bf(a[1]))));
          v[2] = bf2f(f2bf(bf_lo(old.y) + bf2f(f2bf(a[2]))));
          v[3] = bf2f(f2bf(bf_hi(old.y) + bf2f(f2bf(a[3]))));
          *dst = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
        }
        float sq = fmaf(v[0], v[0], fmaf(v[1], v[1], fmaf(v[2], v[2], v[3] * v[3])));
        sq += __shfl_xor(sq, 16);
        sq += __shfl_xor(sq, 32);
        if (q == 0) p.ss_out[m * kNormParts + (n0 >> 4) + t] = sq;
      }
      return;
    }
  }
  if constexpr (EPI == kGemmQkvRope) {
    // lanes q < 2 hold the first halves of pairs jp .. jp+3, lanes q + 2 (= lane ^ 32) the second
    float a[4], b[4];
    const bool hi = q >= 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mine = bf2f(f2bf(acc0[i]));
      const float other = __shfl_xor(mine, 32);
      a[i] = hi ? other : mine;
      b[i] = hi ? mine : other;
    }
    if (m >= p.M) return;
    const int head = tile >> 3, jp = (tile & 7) * 8 + 4 * (q & 1);
    const int pos = epos;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (head < kQHeads + kKVHeads) {
        const float c = ecos[i], sn = esin[i];
        v[i] = hi ? rope_hi(a[i], b[i], c, sn) : rope_lo(a[i], b[i], c, sn);
      } else {
        v[i] = hi ? b[i] : a[i];
      }
    }
    uint16_t* dst;
    if (head < kQHeads) {
      dst = p.y + ((size_t)m * kQHeads + head) * kHeadDim;
    } else {
      const bool is_k = head < kQHeads + kKVHeads;
      const int kvh = head - kQHeads - (is_k ? 0 : kKVHeads);
      uint16_t* const plane = is_k ? p.k_cache : p.v_cache;
      if (p.block_table) {
        // paged: row pos % kPagePos of the page holding block pos / kPagePos
        const int page = epage;
        if (page < 0 || page >= p.n_pages) return;
        dst = plane + (size_t)page * kPageElems + ((size_t)kvh * kPagePos + pos % kPagePos) * kHeadDim;
      } else {
        dst = plane + (size_t)m * p.cache_stride + ((size_t)kvh * kMaxCtx + pos) * kHeadDim;
      }
    }
    *reinterpret_cast<uint2*>(dst + jp + (hi ? 64 : 0)) =
        make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
    return;
  }
  if (m >= p.M || n >= p.N) return;
  if constexpr (!SW) {
    // the plain epilogues, per 16-column tile (columns n0 + 16 t + 4 q ..)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const f32x4_t a = t == 0 ? acc0 : acc1;
      const int nt = n + kSkRows * t;
      if (nt >= p.N) break;
      if constexpr (EPI == kGemmF32) {
        *reinterpret_cast<float4*>(p.yf + (size_t)m * p.ldy + nt) = make_float4(a[0], a[1], a[2], a[3]);
      } else if constexpr (EPI == kGemmResid) {
        uint2* dst = reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + nt);
        const uint2 old = eold[t];
        *dst = make_uint2(
            pack_bf2(bf_lo(old.x) + bf2f(f2bf(a[0])), bf_hi(old.x) + bf2f(f2bf(a[1]))),
            pack_bf2(bf_lo(old.y) + bf2f(f2bf(a[2])), bf_hi(old.y) + bf2f(f2bf(a[3]))));
      } else {
        *reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + nt) =
            make_uint2(pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3]));
      }
    }
  } else {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float g = bf2f(f2bf(acc0[i])), u = bf2f(f2bf(acc1[i]));
      v[i] = g * (1.0f / (1.0f + expf(-g))) * u;
    }
    *reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n) =
        make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
  }
}

// X blocks of one step (rows 16 mb + 4 j + q, chunk r), for the 17-48-row kernel.
template <int MB>
__device__ __forceinline__ void mb_load_x(const __amdgpu_buffer_rsrc_t (&xr)[MB], const SkSrc& src,
                                          int ks, u32x4_t (&xv)[MB][4]) {
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xv[mb][j] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr[mb], src.wo[j], 2 * ks, 0));
}

// One step of the 17-48-row kernel: the X blocks into the wave's LDS slots 1..MB (then their
// registers refilled with step kx), each W tile into slot 0 in turn, 4 k-chunks x MB MFMAs per
// tile; the W registers refilled with step kw.
template <int NT, int MB>
__device__ __forceinline__ void mb_step(u32x4_t (*tr)[256], const SkSrc& src,
                                        const __amdgpu_buffer_rsrc_t (&xr)[MB], u32x4_t (&w)[NT][4],
                                        u32x4_t (&xv)[MB][4], f32x4_t (&acc)[NT][MB], int r, int q,
                                        bool lx, int kx, bool lw, int kw) {
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) sk_put(tr[1 + mb], xv[mb], r, q);
  if (lx) mb_load_x<MB>(xr, src, kx, xv);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    sk_put(tr[0], w[t], r, q);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8_t a = __builtin_bit_cast(bf16x8_t, tr[0][r * 16 + ((4 * c + q) ^ r)]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[t][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            a, __builtin_bit_cast(bf16x8_t, tr[1 + mb][r * 16 + ((4 * c + q) ^ r)]), acc[t][mb],
            0, 0, 0);
    }
  }
  if (lw) sk_load_w<NT>(src, kw, w);
}

// 17-48 rows (short prompts): the same streaming shape with the X rows as MB blocks of 16 (each
// with its own buffer range, rows past M read as zero), every W k-chunk multiplied against each
// block; bf16, residual and SwiGLU epilogues.  The weights stream once; the X blocks are re-read
// by every workgroup from L2.
template <int EPI, int KC, int MB>
__global__ __launch_bounds__(kSkSplit * 64) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_skinny_mb_kernel(GemmParams p) {
  constexpr bool SW = EPI == kGemmSwiglu;
  constexpr int NT = SW ? 2 : 1;
  __shared__ u32x4_t tr[kSkSplit][1 + MB][256];  // per wave: a W tile, then the MB X blocks
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * kSkRows;
  const int K = KC;

  SkSrc src;
  __amdgpu_buffer_rsrc_t xr[MB];
  if constexpr (SW) {
    const int rows = min(kSkRows, p.N - n0);
    src.w[0] = sk_rsrc(p.w0 + (size_t)n0 * K, rows, K);
    src.w[1] = sk_rsrc(p.w1 + (size_t)n0 * K, rows, K);
  } else {
    const int e0 = min(p.n0, p.N), e1 = min(p.n0 + p.n1, p.N);
    const uint16_t* base;
    int end;
    if (n0 < e0) base = p.w0 + (size_t)n0 * K, end = e0;
    else if (n0 < e1) base = p.w1 + (size_t)(n0 - e0) * K, end = e1;
    else base = p.w2 + (size_t)(n0 - e1) * K, end = p.N;
    src.w[0] = sk_rsrc(base, min(kSkRows, end - n0), K);
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    xr[mb] = sk_rsrc(p.x + (size_t)16 * mb * K, max(0, min(16, p.M - 16 * mb)), K);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    src.wo[j] = (uint32_t)((4 * j + q) * K + 8 * r) * 2u;
    src.xo[j] = src.wo[j];
  }
  asm volatile("" : "+v"(src.wo[0]), "+v"(src.wo[1]), "+v"(src.wo[2]), "+v"(src.wo[3]));
  const int kq = K / kSkSplit;
  const int kbase = wave * kq;
  constexpr int steps = KC / kSkSplit / kSkStep;

  f32x4_t acc[NT][MB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4_t w0[NT][4], w1[NT][4], xv[MB][4];
  sk_load_w<NT>(src, kbase, w0);
  mb_load_x<MB>(xr, src, kbase, xv);
  if (steps > 1) sk_load_w<NT>(src, kbase + kSkStep, w1);
#pragma unroll
  for (int s = 0; s < steps; s += 2) {
    const int k1 = kbase + (s + 1) * kSkStep;
    mb_step<NT, MB>(tr[wave], src, xr, w0, xv, acc, r, q, s + 1 < steps, k1, s + 2 < steps,
                    k1 + kSkStep);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < steps)
      mb_step<NT, MB>(tr[wave], src, xr, w1, xv, acc, r, q, s + 2 < steps, k1 + kSkStep,
                      s + 3 < steps, k1 + 2 * kSkStep);
    __builtin_amdgcn_sched_barrier(0);
  }

  // sum the K quarters through each wave's own LDS tiles (its last reads precede these writes):
  // NT * MB slots of 64 lanes, laid out flat over the wave's 1 + MB tiles
  static_assert(NT * MB * 64 <= (1 + MB) * 256, "K-quarter partials overflow the wave's tiles");
  u32x4_t* red = &tr[wave][0][0];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[(t * MB + mb) * 64 + lane] = __builtin_bit_cast(u32x4_t, acc[t][mb]);
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kSkSplit; ++w)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[t][mb] += __builtin_bit_cast(f32x4_t, (&tr[w][0][0])[(t * MB + mb) * 64 + lane]);

  const int n = n0 + 4 * q;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + r;
    if (m >= p.M || n >= p.N) continue;
    uint2* dst = reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n);
    const f32x4_t a0 = acc[0][mb];
    if constexpr (SW) {
      const f32x4_t a1 = acc[NT - 1][mb];
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = bf2f(f2bf(a0[i])), u = bf2f(f2bf(a1[i]));
        v[i] = g * (1.0f / (1.0f + expf(-g))) * u;
      }
      *dst = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
    } else if constexpr (EPI == kGemmResid) {
      const uint2 old = *dst;
      *dst = make_uint2(
          pack_bf2(bf_lo(old.x) + bf2f(f2bf(a0[0])), bf_hi(old.x) + bf2f(f2bf(a0[1]))),
          pack_bf2(bf_lo(old.y) + bf2f(f2bf(a0[2])), bf_hi(old.y) + bf2f(f2bf(a0[3]))));
    } else {
      *dst = make_uint2(pack_bf2(a0[0], a0[1]), pack_bf2(a0[2], a0[3]));
    }
  }
}

template <int EPI, int MB>
int launch_mb_k(const GemmParams& p, hipStream_t st) {
  const int blocks = (p.N + kSkRows - 1) / kSkRows;
  if (p.K == 4096)
    hipLaunchKernelGGL((gemm_skinny_mb_kernel<EPI, 4096, MB>), dim3(blocks), dim3(kSkSplit * 64), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_skinny_mb_kernel<EPI, 14336, MB>), dim3(blocks), dim3(kSkSplit * 64), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int EPI>
int launch_mb_e(const GemmParams& p, hipStream_t st) {
  if (p.M <= 32) return launch_mb_k<EPI, 2>(p, st);
  return launch_mb_k<EPI, 3>(p, st);
}

// Output columns per workgroup tile: 32 for the fp32 epilogue at a compile-time K (two 16-row
// W tiles), else 16.
int skinny_tile_rows(int epi, int K) {
  return epi == kGemmF32 && (K == 4096 || K == 14336) ? 2 * kSkRows : kSkRows;
}

template <int EPI, bool NORM>
int launch_sn(const GemmParams& p, hipStream_t st) {
  const int tr = skinny_tile_rows(EPI, p.K);
  const int blocks = (p.N + tr - 1) / tr + p.sk_tail;
  if constexpr (EPI == kGemmQkvRope) {
    IE_REQUIRE(p.K == kHidden && p.N == kQKVDim && p.n0 == kHidden && p.n1 == kKVDim && p.y &&
                   p.k_cache && p.v_cache && p.d_seq_len && p.rope_cos && p.rope_sin,
               "gemm_skinny: the QKV + RoPE epilogue is for the [q|k|v] projection");
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 4096, NORM>), dim3(blocks), dim3(kSkSplit * 64), 0,
                       st, p);
    IE_CHECK_LAUNCH();
    return IE_OK;
  }
  if constexpr (NORM) {
    // RMSNorm runs over the hidden size only
    IE_REQUIRE(p.K == kHidden, "gemm_skinny: RMSNorm of the X rows needs K = %d (K=%d)", kHidden,
               p.K);
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 4096, NORM>), dim3(blocks), dim3(kSkSplit * 64), 0,
                       st, p);
    IE_CHECK_LAUNCH();
    return IE_OK;
  }
  if (p.K == 4096)
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 4096, NORM>), dim3(blocks), dim3(kSkSplit * 64), 0,
                       st, p);
  else if (p.K == 14336)
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 14336, NORM>), dim3(blocks), dim3(kSkSplit * 64), 0,
                       st, p);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 0, NORM>), dim3(blocks), dim3(kSkSplit * 64), 0, st,
                       p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int EPI>
int launch_s(const GemmParams& p, hipStream_t st) {
  if constexpr (EPI == kGemmSwiglu || EPI == kGemmQkvRope) {
    if (p.ss_in) return launch_sn<EPI, true>(p, st);
  }
  return launch_sn<EPI, false>(p, st);
}


}  // namespace

int gemm_skinny_tail(int N) {
  // 256 CUs: the tiles past the last whole round of 256
  const int tiles = (N + kSkRows - 1) / kSkRows;
  return tiles > 256 ? std::min(tiles % 256, kSkTailMax) : 0;
}

int gemm_skinny_split(int epi, int N, int K) {
  if (epi == kGemmSwiglu || epi == kGemmQkvRope) return gemm_skinny_tail(N);
  const int tr = skinny_tile_rows(epi, K);
  if (tr == kSkRows) return 0;  // (the run-time-K instance has no K halves)
  // the last partial round of 32-row tiles (the lm_head: 168 of 4008)
  const int tiles = (N + tr - 1) / tr;
  return tiles > 256 ? std::min(tiles % 256, kSkTailMax) : 0;
}

bool gemm_skinny_fits(const GemmParams& p) {
  return p.M >= 1 && p.M <= kSkRows && p.K % (kSkSplit * kSkStep) == 0;
}

bool gemm_skinny_mb_fits(int epi, const GemmParams& p) {
  // (4 blocks, M = 64, measured 3% slower than split K: 80 KiB of LDS and ~250 VGPRs)
  return p.M > kSkRows && p.M <= 3 * kSkRows && (p.K == 4096 || p.K == 14336) &&
         (epi == kGemmBf16 || epi == kGemmResid || epi == kGemmSwiglu) && !p.ss_in && !p.ss_out &&
         p.N % 4 == 0;
}

int launch_gemm_skinny_mb(int epi, const GemmParams& p, hipStream_t st) {
  IE_REQUIRE(gemm_skinny_mb_fits(epi, p), "gemm_skinny_mb: needs 16 < M <= 48, K 4096 or 14336");
  const int e0 = std::min(p.n0, p.N), e1 = std::min(p.n0 + p.n1, p.N);
  IE_REQUIRE(epi == kGemmSwiglu ||
                 ((e0 == p.N || e0 % kSkRows == 0) && (e1 == p.N || e1 % kSkRows == 0)),
             "gemm_skinny_mb: weight matrix boundaries must fall on multiples of %d rows", kSkRows);
  if (epi == kGemmSwiglu) return launch_mb_e<kGemmSwiglu>(p, st);
  if (epi == kGemmResid) return launch_mb_e<kGemmResid>(p, st);
  return launch_mb_e<kGemmBf16>(p, st);
}

int launch_gemm_skinny(int epi, const GemmParams& p, hipStream_t st) {
  IE_REQUIRE(gemm_skinny_fits(p), "gemm_skinny: needs M <= %d and K %% %d == 0 (M=%d K=%d)",
             kSkRows, kSkSplit * kSkStep, p.M, p.K);
  IE_REQUIRE(!p.ss_in || (p.ss_parts == kNormParts &&
                          p.x_norm_w && (epi == kGemmSwiglu || epi == kGemmQkvRope)),
             "gemm_skinny: RMSNorm of the X rows (SwiGLU / QKV projections) needs the norm weight "
             "and %d partial sums per row",
             kNormParts);
  IE_REQUIRE(!p.ss_out || (epi == kGemmResid && p.N == 16 * kNormParts),
             "gemm_skinny: the sums-of-squares output is a residual-epilogue option for N = %d",
             16 * kNormParts);
  const int trows = skinny_tile_rows(epi, p.K);
  IE_REQUIRE(p.sk_tail == 0 ||
                 (p.sk_part && p.sk_cnt && p.sk_tail > 0 && p.sk_tail <= kSkTailMax &&
                  p.sk_tail <= (p.N + trows - 1) / trows &&
                  (p.ss_in || epi == kGemmQkvRope || p.K == 4096 || p.K == 14336)),
             "gemm_skinny: K-half tiles (sk_tail=%d) need K 4096 or 14336, at most %d tiles, "
             "partials and counters",
             p.sk_tail, kSkTailMax);
  switch (epi) {
    case kGemmSwiglu: return launch_s<kGemmSwiglu>(p, st);
    case kGemmQkvRope: return launch_s<kGemmQkvRope>(p, st);
    case kGemmBf16:
    case kGemmResid:
    case kGemmF32: break;
    default:
      set_error("gemm_skinny: bad epilogue %d", epi);
      return IE_ERR_INVALID_ARG;
  }
  // a workgroup's rows are read from one weight matrix
  const int e0 = std::min(p.n0, p.N), e1 = std::min(p.n0 + p.n1, p.N);
  IE_REQUIRE((e0 == p.N || e0 % trows == 0) && (e1 == p.N || e1 % trows == 0),
             "gemm_skinny: weight matrix boundaries must fall on multiples of %d rows (n0=%d n1=%d)",
             trows, p.n0, p.n1);
  if (epi == kGemmResid) return launch_s<kGemmResid>(p, st);
  if (epi == kGemmF32) return launch_s<kGemmF32>(p, st);
  return launch_s<kGemmBf16>(p, st);
}

}  // namespace ie
