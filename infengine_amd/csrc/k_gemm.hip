// MFMA bf16 GEMM for prefill (and any multi-row multiply_by_weight):
//   Y[M, N] = X[M, K] . W[N, K]^T      (X, W row-major, K contiguous; fp32 accumulate)
//
// Reference: every prefill matmul is cublasGemmEx / cublasGemmStridedBatchedEx
// with fp32 compute (kernels/ffn.cu:7-33, kernels/attn.cu:12-39, 265-293).
//
// Kernels of this file by the product's rows M (launch_gemm; M <= 16 goes to the skinny GEMM of
// k_gemm_skinny.hip):
//   17-128   gemm_mid_kernel: a workgroup streams 64 (or 128) weight rows, loaded nontemporal,
//            against all X rows; K split into fp32 partial planes summed by a split reduction
//            (RoPE + K/V write, residual + RMSNorm, SwiGLU or bf16), or unsplit with the
//            epilogue in the kernel.
//   to 1024  gemm_wide_kernel (128-row X tiles, direct-to-LDS rings) split over K, with the
//            same reductions, where the best tiling is one round that leaves half the chip idle.
//   beyond   launch_tiled: the ping-pong gemm_pp_kernel / gemm_pp_dual_kernel on 256 x 256,
//            256 x 128 and 192 x 256 tiles, chosen by rounds of 256 tiles; the 128 x 128
//            gemm_kernel described next takes what the larger tiles do not fit.
//
// Tile: 128 W-rows x 128 X-rows x 64 k per workgroup of 4 waves; each wave owns
// a 64 x 64 block as 4 x 4 v_mfma_f32_16x16x32_bf16 tiles.  The MFMA computes
// D = W_tile . X_tile^T, so a lane's 4 accumulator values are 4 consecutive
// output columns of one output row (one 8-byte store).  Both operands are
// K-contiguous in HBM, so every fragment is one 16-byte LDS read.
//
// LDS: two stages x (W tile + X tile) x 16 KiB = 64 KiB.  A 16-byte chunk c of
// tile row r is stored at chunk slot c ^ (r & 7), so the 16 rows a fragment read
// touches land in distinct bank groups.  Global loads for stage k+1 are issued
// into registers before the MFMAs of stage k and written to the other LDS stage
// afterwards: one barrier per k-step.
//
// Workgroup -> tile mapping is XCD-aware: workgroups are dealt round-robin to
// the 8 XCDs, so workgroup b is given logical tile (b % 8) * (nb / 8) + b / 8,
// which hands each XCD a contiguous run of tiles that share W rows (column-major
// sweep over M inside one W tile) and keeps those rows in that XCD's L2.
//
// Epilogues: bf16 store, fp32 store, residual add (Y = bf16(Y + bf16(acc)),
// residual_add.cu:17-19), and SwiGLU over a gate/up pair of weights in which the
// 128 W rows of a tile are [32 gate | 32 up | 32 gate | 32 up] for 64 output
// columns, so each lane holds gate and up for the same output element.
#include <algorithm>

#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128;  // X rows per tile
constexpr int BN = 128;  // W rows per tile
constexpr int BK = 64;
constexpr int kWideMinRows = 128;  // smallest M the wide-tile kernels are considered for

template <int EPI>
__device__ __forceinline__ const uint16_t* w_row(const GemmParams& p, int ntile, int r) {
  if constexpr (EPI == kGemmSwiglu) {
    // local row r -> [32 gate | 32 up] x 2; output columns ntile*64 + (r/64)*32 + (r%32)
    const int half = r >> 6, within = r & 63;
    const int col = ntile * 64 + half * 32 + (within & 31);
    const int c = col < p.N ? col : p.N - 1;
    return (within < 32 ? p.w0 : p.w1) + (size_t)c * p.K;
  } else {
    int R = ntile * BN + r;
    if (R >= p.N) R = p.N - 1;
    if (R < p.n0) return p.w0 + (size_t)R * p.K;
    if (R < p.n0 + p.n1) return p.w1 + (size_t)(R - p.n0) * p.K;
    return p.w2 + (size_t)(R - p.n0 - p.n1) * p.K;
  }
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p, int m_tiles) {
  __shared__ u32x4_t smem[2][2][BN * (BK / 8)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1;
  const int nb = gridDim.x, b = blockIdx.x;
  const int t = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
  const int mtile = t % m_tiles, ntile = t / m_tiles;
  const int m0 = mtile * BM;

  // each thread moves 4 chunks of W and 4 chunks of X per k-step
  const uint16_t* wsrc[4];
  const uint16_t* xsrc[4];
  int slot[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + i * 256, r = idx >> 3, c = idx & 7;
    wsrc[i] = w_row<EPI>(p, ntile, r) + c * 8;
    const int xr = min(m0 + r, p.M - 1);
    xsrc[i] = p.x + (size_t)xr * p.K + c * 8;
    slot[i] = r * 8 + (c ^ (r & 7));
  }

  u32x4_t rw[4], rx[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rw[i] = *reinterpret_cast<const u32x4_t*>(wsrc[i]);
    rx[i] = *reinterpret_cast<const u32x4_t*>(xsrc[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    smem[0][0][slot[i]] = rw[i];
    smem[0][1][slot[i]] = rx[i];
  }
  __syncthreads();

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int KT = p.K / BK;
  const int fr = lane & 15, fq = lane >> 4, sw = lane & 7;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      const int ko = (kt + 1) * BK;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw[i] = *reinterpret_cast<const u32x4_t*>(wsrc[i] + ko);
        rx[i] = *reinterpret_cast<const u32x4_t*>(xsrc[i] + ko);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = (ks * 4 + fq) ^ sw;
      bf16x8_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wn * 64 + i * 16 + fr;
        af[i] = __builtin_bit_cast(bf16x8_t, smem[cur][0][row * 8 + ch]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = wm * 64 + j * 16 + fr;
        bf[j] = __builtin_bit_cast(bf16x8_t, smem[cur][1][row * 8 + ch]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        smem[cur ^ 1][0][slot[i]] = rw[i];
        smem[cur ^ 1][1][slot[i]] = rx[i];
      }
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds rows m = m0 + wm*64 + j*16 + fr, cols n = base + i*16 + 4*fq + q
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wm * 64 + j * 16 + fr;
    if (m >= p.M) continue;
    if constexpr (EPI == kGemmSwiglu) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int n = ntile * 64 + wn * 32 + i * 16 + 4 * fq;
        if (n >= p.N) continue;
        uint32_t o[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float v[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float g = bf2f(f2bf(acc[i][j][2 * q + e]));
            const float u = bf2f(f2bf(acc[i + 2][j][2 * q + e]));
            v[e] = g * (1.0f / (1.0f + expf(-g))) * u;
          }
          o[q] = pack_bf2(v[0], v[1]);
        }
        *reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n) = make_uint2(o[0], o[1]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = ntile * BN + wn * 64 + i * 16 + 4 * fq;
        if (n >= p.N) continue;
        const f32x4_t a = acc[i][j];
        if constexpr (EPI == kGemmF32) {
          *reinterpret_cast<float4*>(p.yf + (size_t)m * p.ldy + n) =
              make_float4(a[0], a[1], a[2], a[3]);
        } else if constexpr (EPI == kGemmResid) {
          uint2* dst = reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n);
          const uint2 old = *dst;
          *dst = make_uint2(pack_bf2(bf_lo(old.x) + bf2f(f2bf(a[0])), bf_hi(old.x) + bf2f(f2bf(a[1]))),
                            pack_bf2(bf_lo(old.y) + bf2f(f2bf(a[2])), bf_hi(old.y) + bf2f(f2bf(a[3]))));
        } else {
          *reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n) =
              make_uint2(pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3]));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wide-tile kernel for M >= 128 (prefill): 256 (or 192) W rows x 128 (or 256) X rows x 64 k
// per workgroup; each wave owns 128 (96) W rows x 64 X rows as 4 (3) x 2 tiles of
// v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators per lane).  The 256 x 128 tile runs 8 waves
// as two k-groups (each takes two of a k-step's four k16 sub-steps for the whole tile, and the
// groups' sums are added through LDS at the end): two waves per SIMD where one tile's worth
// of 128 x 64 blocks would leave one.
//
// Operands reach LDS by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds:
// lane i of a wave writes 16 bytes at LDS base + 16 i), through a 3-stage ring
// of 48 KiB stages, so the loads for k-step kt+2 are in flight while k-step kt
// is multiplied.  Each load covers 8 tile rows through its own buffer descriptor
// (base = the group's first row, size = the rows left in its matrix), so rows
// past the end of a matrix read as zero, and the k offset is a scalar operand.
// (The buffer form, not global_load_lds: a FLAT-encoded LDS load makes the
// compiler treat every later LDS wait as unordered, i.e. lgkmcnt(0).)  The LDS destination of a load is fixed by the lane index, so
// the bank swizzle is applied on the global side: LDS chunk slot s of tile row r
// holds global chunk s ^ swz(r).  swz(r) = ((r >> 1) & 7) ^ ((r >> 4) & 1) makes
// the 16 (or 32) rows that one ds_read_b128 phase touches land in distinct
// 16-byte bank groups for both a 64-bank and a 128-bank LDS.
//
// The loads are counted by vmcnt; the compiler does not track them, so every
// k-step starts with an explicit "s_waitcnt vmcnt(N); s_barrier": N = the loads
// of the one younger stage still allowed in flight (12 per wave), 0 on the last
// step.  No other vector-memory instruction is issued inside the loop.
namespace wide {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw 32-bit access)

// Tile geometry: BN (256 or 192) W rows x BM (128 or 256) X rows x BK (32 or 64) k, in a
// ring of STAGES LDS stages.  Every wave owns BN / 2 W rows x 64 X rows (NI = BN / 64 blocks
// of 32 W rows), so a workgroup has NW = 2 * BM / 64 waves (4 or 8).
template <int BM_, int BK_, int STAGES_, int BN_ = 256, int KG_ = 1>
struct Cfg {
  static constexpr int BN = BN_;
  static constexpr int WTN = BN / 2;                 // W rows per wave
  static constexpr int NI = WTN / 32;                // 32-row MFMA blocks per wave
  static constexpr int NT = 2 * NI;                  // MFMAs per k16 sub-step
  static constexpr int BM = BM_;
  static constexpr int BK = BK_;
  static constexpr int STAGES = STAGES_;
  static constexpr int WM = BM / 64;                 // waves along X
  static constexpr int NW = 2 * WM;                  // waves per k-group (one tile's worth)
  static constexpr int KG = KG_;                     // k-groups: waves splitting each k-step
  static constexpr int NWT = NW * KG;                // waves per workgroup
  static constexpr int THREADS = 64 * NWT;
  static constexpr int CPR = BK / 8;                 // 16-byte chunks per tile row
  static constexpr int RPL = 64 / CPR;               // tile rows per wave-wide load
  static constexpr int W_CHUNKS = BN * CPR;
  static constexpr int X_CHUNKS = BM * CPR;
  static constexpr int STAGE = W_CHUNKS + X_CHUNKS;  // chunks per stage
  static constexpr int W_LOADS = W_CHUNKS / THREADS; // loads per thread per stage
  static constexpr int X_LOADS = X_CHUNKS / THREADS;
  static constexpr int LOADS = W_LOADS + X_LOADS;
  static constexpr int KSUB = BK / 16;               // MFMA k16 sub-steps per stage
  static constexpr int KSUBW = KSUB / KG;            // sub-steps per wave per k-step
  // With a ring of 3 or more stages a stage's loads are spread over a wave's KSUBW sub-steps (the
  // last of k-step kt and the first KSUBW-1 of k-step kt+1) instead of all issued in one.
  static constexpr bool SPREAD = STAGES >= 3;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(BN == 256 || BN == 192, "BN");
  static_assert(KSUBW % 2 == 0, "fragment double buffer alternates within a k-step");
  static_assert(W_CHUNKS % THREADS == 0 && X_CHUNKS % THREADS == 0, "loads per thread");
  static_assert(STAGES * STAGE * 16 <= 160 * 1024, "LDS");
  // Chunk slot s of row r holds global chunk s ^ swz(r): the 16 (or 32) consecutive rows one
  // ds_read_b128 phase touches fall in distinct 16-byte bank groups (64- or 128-bank LDS).
  static __device__ __forceinline__ int swz(int r) {
    if constexpr (CPR == 8) return ((r >> 1) & 7) ^ ((r >> 4) & 1);
    else return ((r >> 2) & 3) ^ ((r >> 4) & 1);
  }
};

// Buffer descriptor for the `rows` W rows starting at tile-local row r (all in one matrix).
template <int EPI, int BN>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t w_group(const GemmParams& p, int ntile, int r,
                                                          int k0 = 0) {
  const uint16_t* base;
  long long rows;
  if constexpr (EPI == kGemmSwiglu) {
    // local row r -> [32 gate | 32 up] x (BN / 64); output column ntile*BN/2 + (r/64)*32 + r%32
    const int col = ntile * (BN / 2) + (r >> 6) * 32 + (r & 31);
    base = ((r & 63) < 32 ? p.w0 : p.w1) + (size_t)col * p.K;
    rows = p.N - col;
  } else {
    int R = ntile * BN + r;
    if constexpr (EPI == kGemmQkvRope) {
      // tile rows 0..95: the first halves (dims 0..63) of RoPE pairs P = 96 ntile + r, rows
      // 96..191 the second halves (dims 64..127) of the same pairs; pair P is dim P % 64 of head
      // P / 64 of [q|k|v] (a group of 8 rows stays within one half-head: consecutive rows)
      static_assert(BN == 192, "QKV + RoPE tiles hold 96 pairs");
      const int half = r >= 96 ? 1 : 0, P = ntile * 96 + r - 96 * half;
      R = (P >> 6) * kHeadDim + 64 * half + (P & 63);
    }
    const int e0 = min(p.n0, p.N), e1 = min(p.n0 + p.n1, p.N);
    if (R < e0) {
      base = p.w0 + (size_t)R * p.K;
      rows = e0 - R;
    } else if (R < e1) {
      base = p.w1 + (size_t)(R - e0) * p.K;
      rows = e1 - R;
    } else if (R < p.N) {
      base = p.w2 + (size_t)(R - e1) * p.K;
      rows = p.N - R;
    } else {
      base = p.w0;
      rows = 0;
    }
  }
  // (split K: the buffer starts at column k0 of its first row and ends where the rows end)
  const long long bytes = rows > 0 ? rows * p.K * 2 - 2LL * k0 : 0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base + k0), 0, (int)min(bytes, 0x7fffffffLL),
                                           kBufferFlags);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_group(const GemmParams& p, int m0, int r,
                                                          int k0 = 0) {
  const int R = m0 + r;
  const long long rows = p.M - R;
  const long long bytes = rows > 0 ? rows * p.K * 2 - 2LL * k0 : 0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)(p.x + (size_t)min(R, p.M - 1) * p.K + k0), 0,
                                           (int)min(bytes, 0x7fffffffLL), kBufferFlags);
}

// Direct-to-LDS loads of k-step kt into ring slot `stage`.  (Plain device functions, not
// lambdas: a lambda around the amdgcn builtin inside a kernel template stops the host pass
// from emitting the kernel's launch stub.)
template <class C>
__device__ __forceinline__ void issue_load(u32x4_t* lds, const __amdgpu_buffer_rsrc_t* rsrc,
                                           const uint32_t* voff, int wv, int kt, int stage, int j) {
  const bool is_w = j < C::W_LOADS;
  const int g = wv + C::NWT * (is_w ? j : j - C::W_LOADS);
  u32x4_t* dst = &lds[stage * C::STAGE + (is_w ? 0 : C::W_CHUNKS) + g * 64];
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc[j], (lds_void*)dst, 16, voff[j],
                                           (uint32_t)(kt * C::BK * 2), 0, 0);
}

template <class C>
__device__ __forceinline__ void issue_stage(u32x4_t* lds, const __amdgpu_buffer_rsrc_t* rsrc,
                                            const uint32_t* voff, int wv, int kt, int stage) {
#pragma unroll
  for (int j = 0; j < C::LOADS; ++j) issue_load<C>(lds, rsrc, voff, wv, kt, stage, j);
}

// Operand fragment n (0..NI+1) of a k16 sub-step, in the order the sub-step's MFMAs first use
// them: X0 W0 X1 W1 W2 (W3).  Lane l supplies tile row base + l%32 at k chunk ch (2*kk + l/32,
// swizzled).
template <class C>
__device__ __forceinline__ void read_frag(const u32x4_t* src, int a_row, int b_row, int ch, int n,
                                          bf16x8_t* af, bf16x8_t* bfr) {
  if (n == 0 || n == 2) {
    bfr[n / 2] = __builtin_bit_cast(bf16x8_t, src[b_row + (n / 2) * 32 * C::CPR + ch]);
  } else {
    const int i = n == 1 ? 0 : n - 2;
    af[i] = __builtin_bit_cast(bf16x8_t, src[a_row + i * 32 * C::CPR + ch]);
  }
}

// 8 bf16 at dst (8-byte aligned; 16-byte aligned when a16)
__device__ __forceinline__ void store16(uint16_t* dst, uint2 lo, uint2 hi, bool a16) {
  if (a16) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(lo.x, lo.y, hi.x, hi.y);
  } else {
    reinterpret_cast<uint2*>(dst)[0] = lo;
    reinterpret_cast<uint2*>(dst)[1] = hi;
  }
}

// Wait until at most n stages of loads (n * loads per stage) are in flight and this wave's
// LDS reads have returned, then barrier: after it the stage is visible to every wave and no
// wave still reads the ring slot the next loads overwrite.
template <int LOADS, int N>
__device__ __forceinline__ void wait_stage_n(int n) {
  if constexpr (N < 0) {
    return;
  } else {
    if (n == N) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N * LOADS) : "memory");
      return;
    }
    wait_stage_n<LOADS, N - 1>(n);
  }
}

// Logical tile of workgroup b.  Workgroups are dealt round-robin to the 8 XCDs, so each XCD
// is handed a contiguous range of W tiles (n_tiles / 8); inside it the range is swept in
// groups of MAPG W tiles x all X tiles, X-tile-major within a group, so the 32 tiles an XCD
// runs at once share W rows and X rows in its L2.
template <int MAPG>
__device__ __forceinline__ void tile_of(int b, int nb, int m_tiles, int& mtile, int& ntile) {
  const int n_tiles = nb / m_tiles;
  if (nb % 8 == 0 && n_tiles % (8 * MAPG) == 0) {
    const int x = b % 8, local = b / 8;
    const int grp = local / (MAPG * m_tiles), within = local % (MAPG * m_tiles);
    ntile = x * (n_tiles / 8) + grp * MAPG + within % MAPG;
    mtile = within / MAPG;
  } else {
    const int t = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    mtile = t % m_tiles;
    ntile = t / m_tiles;
  }
}

// One k-step on ring slot kt % STAGES, as 4 (BK 64) or 2 (BK 32) MFMA sub-steps of k16 (with
// KG = 2 k-groups a wave runs the KSUBW = KSUB / 2 sub-steps from kk0 = its group's half).  The
// fragments of the next sub-step are read one after each MFMA of the current one, so that their
// issue hides under the MFMAs (the scheduling fences keep this order: left alone the scheduler
// groups the reads and moves each just before its use).  The last sub-step waits for stage
// kt+1 and reads its first fragments, so no k-step starts on an LDS latency.
// Loads: with NEW the last sub-step refills slot kt % STAGES (free once every wave has passed
// that sub-step's barrier) with stage kt+STAGES -- all of it, or with SPREAD its first share;
// with REST (SPREAD) sub-step kk < KSUBW-1 issues share kk+1 of stage kt-1+STAGES.  Loads are
// issued in stage order either way, so the wait for stage kt+1 allows exactly the younger
// stages issued so far: min(STAGES-2, KT-2-kt) of them.
template <class C, bool NEW, bool REST>
__device__ __forceinline__ void k_step(f32x16_t (&acc)[C::NI][2], bf16x8_t (&af)[2][C::NI],
                                       bf16x8_t (&bfr)[2][2], u32x4_t* lds,
                                       const __amdgpu_buffer_rsrc_t* rsrc, const uint32_t* voff,
                                       int wv, int a_row, int b_row, int fh, int fs, int kk0,
                                       int kt, int KT) {
  const u32x4_t* st = &lds[(kt % C::STAGES) * C::STAGE];
  const u32x4_t* nst = &lds[((kt + 1) % C::STAGES) * C::STAGE];
#pragma unroll
  for (int kk = 0; kk < C::KSUBW; ++kk) {
    const int cur = kk & 1;
    const bool last = kk + 1 == C::KSUBW;
    const bool rd = !last || kt + 1 < KT;
    // stage kt+1 must have landed; the younger stages issued so far may stay in flight
    if (last && rd)
      wait_stage_n<C::LOADS, C::STAGES - 2>(NEW ? C::STAGES - 2 : min(C::STAGES - 2, KT - 2 - kt));
    const u32x4_t* src = last ? nst : st;
    const int ch = (2 * (kk0 + (last ? 0 : kk + 1)) + fh) ^ fs;
    // loads of this sub-step: share `sh` of stage `ls` into ring slot `slot`
    const bool issue = last ? NEW : (C::SPREAD && REST);
    const int sh = !C::SPREAD ? 0 : last ? 0 : kk + 1;
    const int ls = last ? kt + C::STAGES : kt - 1 + C::STAGES;
    const int slot = ls % C::STAGES;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
      acc[t / 2][t % 2] =
          __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[cur][t / 2], bfr[cur][t % 2], acc[t / 2][t % 2], 0, 0, 0);
      if (rd && t < C::NI + 2) read_frag<C>(src, a_row, b_row, ch, t, af[cur ^ 1], bfr[cur ^ 1]);
      if (issue) {
        constexpr int SHARES = C::SPREAD ? C::KSUBW : 1;
        constexpr int PER = (C::LOADS + SHARES - 1) / SHARES;  // loads per share (last may be short)
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int j = sh * PER + i;
          if (j < C::LOADS && i * C::NT / PER == t) issue_load<C>(lds, rsrc, voff, wv, ls, slot, j);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Output-tile swizzle: 8-byte unit u of row r (of `upr` units) sits at slot swz_out(u, r).  The
// 32 rows one write instruction touches land in distinct 8-byte bank pairs: within a 32-unit
// group u ^ (r % 32) is a permutation of the rows; in the 16-unit tail of a 48-unit row the rows'
// alternating 16-unit offset (48 r mod 32) supplies the fifth bit.
template <int UPR>
__device__ __forceinline__ int swz_out(int u, int r) {
  if constexpr (UPR == 48) {
    if (u >= 32) return 32 + ((u - 32) ^ ((r & 14) | ((r >> 4) & 1)));
  }
  return u ^ (r & 31);
}

// The epilogue of a 256- or 192-row W tile: wave (wn, wm) of k-group kg holds accumulator element
// 4*g + q of tile (i, j) = W row wn*WTN + 32*i + 8*g + 4*(lane/32) + q, X row m0 + wm*64 + 32*j +
// lane%32 (k-group 0 holds the sums).  fp32 results go straight to global memory; bf16 ones are
// staged through the LDS ring as a [BM][OUTN] tile and stored as whole row segments.
// Copy-out of a bf16 output tile staged in LDS as [BM][UPR] 8-byte units (unit u of row r at
// swz(u, r)): 16 bytes (8 columns) per thread, consecutive threads along a row; the residual
// epilogue adds the tile to y.
template <int THREADS, int BM, int UPR, int EPI, class SW>
__device__ __forceinline__ void tile_copy_out(const GemmParams& p, const uint2* ot, uint16_t* y,
                                              int m0, int n_base, int tid, SW swz) {
  const bool ld16 = (p.ldy & 7) == 0;  // rows 16-byte aligned: one 16-byte store per thread
#pragma unroll 4
  for (int P = tid; P < BM * UPR / 2; P += THREADS) {
    const int r = P / (UPR / 2), c2 = P % (UPR / 2);
    const int m = m0 + r, n = n_base + 8 * c2;
    if (m >= p.M || n >= p.N) continue;
    const uint2 lo = ot[r * UPR + swz(2 * c2, r)], hi = ot[r * UPR + swz(2 * c2 + 1, r)];
    uint16_t* dst = y + (size_t)m * p.ldy + n;
    if constexpr (EPI == kGemmResid) {
      // y = bf16(y + bf16(acc)) (residual_add.cu:17-19); the LDS tile holds bf16(acc)
      const uint2 a = *reinterpret_cast<const uint2*>(dst);
      const uint2 o0 = make_uint2(pack_bf2(bf_lo(a.x) + bf_lo(lo.x), bf_hi(a.x) + bf_hi(lo.x)),
                                  pack_bf2(bf_lo(a.y) + bf_lo(lo.y), bf_hi(a.y) + bf_hi(lo.y)));
      if (n + 8 <= p.N) {
        const uint2 b = *reinterpret_cast<const uint2*>(dst + 4);
        const uint2 o1 = make_uint2(pack_bf2(bf_lo(b.x) + bf_lo(hi.x), bf_hi(b.x) + bf_hi(hi.x)),
                                    pack_bf2(bf_lo(b.y) + bf_lo(hi.y), bf_hi(b.y) + bf_hi(hi.y)));
        store16(dst, o0, o1, ld16);
      } else {
        *reinterpret_cast<uint2*>(dst) = o0;
      }
    } else {
      if (n + 8 <= p.N) store16(dst, lo, hi, ld16);
      else *reinterpret_cast<uint2*>(dst) = lo;
    }
  }
}

// Copy-out of the prefill QKV + RoPE tile staged in LDS as [256][48] 8-byte units: unit u < 24
// holds the first halves of pairs 96 ntile + 4u .. +3 (pair P: head P / 64, dims P % 64 and
// P % 64 + 64), unit 24 + u their second halves.  Each thread takes 4 pairs of one row: RoPE at
// position start_pos + m on q and k (the scatter kernel's pairing and roundings, on the same
// bf16 values), q to y [M][32][128], k and v to this layer's cache planes (or pages).
template <int THREADS, class SW>
__device__ __forceinline__ void rope_copy_out(const GemmParams& p, const uint2* ot, int m0,
                                              int ntile, int tid, SW swz) {
  constexpr int UPR = 48, QUADS = 24;
#pragma unroll 4
  for (int it = tid; it < 256 * QUADS; it += THREADS) {
    const int r = it / QUADS, u = it % QUADS;
    const int m = m0 + r;
    if (m >= p.M) continue;
    const uint2 lo = ot[r * UPR + swz(u, r)], hi = ot[r * UPR + swz(QUADS + u, r)];
    const int P = ntile * 96 + 4 * u;
    const int head = P >> 6, j = P & 63;
    const int pos = p.start_pos + m;
    uint2 o0 = lo, o1 = hi;
    if (head < kQHeads + kKVHeads) {
      const float4 c = *reinterpret_cast<const float4*>(p.rope_cos + (size_t)pos * 64 + j);
      const float4 sn = *reinterpret_cast<const float4*>(p.rope_sin + (size_t)pos * 64 + j);
      const float a[4] = {bf_lo(lo.x), bf_hi(lo.x), bf_lo(lo.y), bf_hi(lo.y)};
      const float b[4] = {bf_lo(hi.x), bf_hi(hi.x), bf_lo(hi.y), bf_hi(hi.y)};
      const float cc[4] = {c.x, c.y, c.z, c.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
      float va[4], vb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        va[e] = rope_lo(a[e], b[e], cc[e], ss[e]);
        vb[e] = rope_hi(a[e], b[e], cc[e], ss[e]);
      }
      o0 = make_uint2(pack_bf2(va[0], va[1]), pack_bf2(va[2], va[3]));
      o1 = make_uint2(pack_bf2(vb[0], vb[1]), pack_bf2(vb[2], vb[3]));
    }
    uint16_t* dst;
    if (head < kQHeads) {
      dst = p.y + ((size_t)m * kQHeads + head) * kHeadDim;
    } else {
      const bool is_k = head < kQHeads + kKVHeads;
      const int kvh = head - kQHeads - (is_k ? 0 : kKVHeads);
      uint16_t* const plane = is_k ? p.k_cache : p.v_cache;
      if (p.block_table) {  // paged: row pos % kPagePos of the page holding block pos / kPagePos
        const int page = p.block_table[pos / kPagePos];
        if (page < 0 || page >= p.n_pages) continue;
        dst = plane + (size_t)page * kPageElems + ((size_t)kvh * kPagePos + pos % kPagePos) * kHeadDim;
      } else {
        dst = plane + ((size_t)kvh * kMaxCtx + pos) * kHeadDim;
      }
    }
    *reinterpret_cast<uint2*>(dst + j) = o0;
    *reinterpret_cast<uint2*>(dst + j + 64) = o1;
  }
}

template <int UPR>
struct WideOutSwz {
  __device__ __forceinline__ int operator()(int u, int r) const { return swz_out<UPR>(u, r); }
};

template <class C, int EPI>
__device__ __forceinline__ void wide_epilogue(const GemmParams& p, f32x16_t (&acc)[C::NI][2],
                                              u32x4_t* lds, uint16_t* y, float* yf, int m0,
                                              int ntile, int kg, int wn, int wm, int lane,
                                              int tid) {
  constexpr int BM = C::BM, BN = C::BN, STAGES = C::STAGES;
  const int fr = lane & 31, fh = lane >> 5;
  if constexpr (EPI == kGemmF32) {
    if (kg != 0) return;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = m0 + wm * 64 + j * 32 + fr;
      if (m >= p.M) continue;
#pragma unroll
      for (int i = 0; i < C::NI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = ntile * BN + wn * C::WTN + i * 32 + 8 * g + 4 * fh;
          if (n < p.N)
            *reinterpret_cast<float4*>(yf + (size_t)m * p.ldy + n) =
                make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
        }
    }
  } else {
    // bf16 results go through LDS so that the global stores are whole, coalesced row segments
    // (a lane's accumulators are 4 columns of 32 different rows; storing them directly writes
    // every 128-byte line in eight 16-byte pieces).  The tile is [BM][OUTN] bf16 held as
    // 8-byte units; unit u of row r sits at swz_out(u, r), which spreads the 32 rows one
    // write instruction touches over distinct banks without padding.
    constexpr int OUTN = (EPI == kGemmSwiglu) ? 128 : BN;  // output columns per tile
    constexpr int UPR = OUTN / 4;                            // 8-byte units per row
    static_assert(BM * OUTN * 2 <= STAGES * C::STAGE * 16, "output tile must fit the LDS ring");
    uint2* ot = reinterpret_cast<uint2*>(lds);
    __syncthreads();  // every wave is done reading the ring
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (kg != 0) break;
      const int r = wm * 64 + j * 32 + fr;
      if constexpr (EPI == kGemmSwiglu) {
#pragma unroll
        for (int i = 0; i < 4; i += 2)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            uint32_t o[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              float v[2];
#pragma unroll
              for (int e = 0; e < 2; ++e) {
                const float gt = bf2f(f2bf(acc[i][j][4 * g + 2 * q + e]));
                const float up = bf2f(f2bf(acc[i + 1][j][4 * g + 2 * q + e]));
                v[e] = gt * (1.0f / (1.0f + expf(-gt))) * up;
              }
              o[q] = pack_bf2(v[0], v[1]);
            }
            const int u = (2 * wn + i / 2) * 8 + 2 * g + fh;
            ot[r * UPR + swz_out<UPR>(u, r)] = make_uint2(o[0], o[1]);
          }
      } else {
#pragma unroll
        for (int i = 0; i < C::NI; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int u = wn * (C::WTN / 4) + i * 8 + 2 * g + fh;
            ot[r * UPR + swz_out<UPR>(u, r)] = make_uint2(pack_bf2(acc[i][j][4 * g], acc[i][j][4 * g + 1]),
                                                pack_bf2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]));
          }
      }
    }
    __syncthreads();
    tile_copy_out<C::THREADS, BM, UPR, EPI>(p, ot, y, m0, ntile * OUTN, tid, WideOutSwz<UPR>{});
  }
}

template <int EPI, int BM, int BK, int STAGES, int MAPG, int BN, int KG>
__global__ __launch_bounds__(2 * BM * KG) __attribute__((amdgpu_waves_per_eu(BM * KG / 128, BM * KG / 128)))
void gemm_wide_kernel(GemmParams p, int m_tiles) {
  using C = Cfg<BM, BK, STAGES, BN, KG>;
  static_assert(C::THREADS == 2 * BM * KG, "launch bounds");
  static_assert(EPI != kGemmSwiglu || BN == 256, "SwiGLU tiles are 256 W rows");
  __shared__ u32x4_t lds[STAGES * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // wave = kg * NW + wt: k-group kg runs sub-steps kk0 .. kk0+KSUBW-1 of every k-step for the
  // 128 x 64 block wt of the tile; with KG = 2 the groups' sums are added at the end
  const int kg = wave / C::NW, wt = wave % C::NW;
  const int wn = wt / C::WM, wm = wt % C::WM;
  const int kk0 = __builtin_amdgcn_readfirstlane(kg * C::KSUBW);
  // split K: workgroup b takes k-steps [split * KT, (split + 1) * KT) of tile b % tiles and
  // writes its fp32 partial product to partial plane `split` of yf
  const int nsplit = max(1, p.k_splits);
  const int nb = gridDim.x / nsplit, split = blockIdx.x / nb;
  int mtile, ntile;
  tile_of<MAPG>(blockIdx.x - split * nb, nb, m_tiles, mtile, ntile);
  const int m0 = mtile * BM;
  const int KT = p.K / BK / nsplit;
  const int k0 = split * KT * BK;

  // load j of this wave covers tile rows RPL*g .. RPL*g+RPL-1 with g = wave + NWT*j;
  // lane i fills LDS slot (row RPL*g + i/CPR, chunk i%CPR) from global chunk (i%CPR) ^ swz(row)
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  __amdgpu_buffer_rsrc_t rsrc[C::LOADS];
  uint32_t voff[C::LOADS];
#pragma unroll
  for (int j = 0; j < C::LOADS; ++j) {
    const bool is_w = j < C::W_LOADS;
    const int g = wv + C::NWT * (is_w ? j : j - C::W_LOADS);
    rsrc[j] = is_w ? w_group<EPI, C::BN>(p, ntile, g * C::RPL, k0) : x_group(p, m0, g * C::RPL, k0);
    const int rl = lane / C::CPR, c = (lane % C::CPR) ^ C::swz(g * C::RPL + rl);
    voff[j] = (uint32_t)((rl * p.K + c * 8) * 2);
  }
  f32x16_t acc[C::NI][2];
#pragma unroll
  for (int i = 0; i < C::NI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // fragment addressing: operand lane l supplies tile row base + l%32, k chunk 2*kk + l/32
  const int fr = lane & 31, fh = lane >> 5, fs = C::swz(fr);
  const int a_row = (wn * C::WTN + fr) * C::CPR;
  const int b_row = C::W_CHUNKS + (wm * 64 + fr) * C::CPR;

  // The epilogue's kernel arguments are pulled into SGPRs here: a scalar load still in
  // flight inside the loop would force every LDS wait there to lgkmcnt(0).
  uint16_t* const y = p.y;
  float* const yf = p.yf + (size_t)split * p.M * p.ldy;
  asm volatile("" ::"s"(y), "s"(yf), "s"(p.ldy), "s"(p.M), "s"(p.N));

#pragma unroll
  for (int s0 = 0; s0 < STAGES - 1; ++s0)
    if (s0 < KT) issue_stage<C>(lds, rsrc, voff, wv, s0, s0);
  // stage 0 landed; stage STAGES-1 goes to the last ring slot, which no wave reads yet
  wait_stage_n<C::LOADS, STAGES - 2>(min(STAGES - 2, KT - 1));
  if (STAGES - 1 < KT) issue_stage<C>(lds, rsrc, voff, wv, STAGES - 1, STAGES - 1);
  bf16x8_t af[2][C::NI], bfr[2][2];
#pragma unroll
  for (int n = 0; n < C::NI + 2; ++n) read_frag<C>(lds, a_row, b_row, (2 * kk0 + fh) ^ fs, n, af[0], bfr[0]);
  int kt = 0;
  // stage STAGES-1 was issued whole above, so k-step 0 issues no remaining shares
  if (STAGES < KT) {
    k_step<C, true, false>(acc, af, bfr, lds, rsrc, voff, wv, a_row, b_row, fh, fs, kk0, kt, KT);
    ++kt;
  }
  for (; kt + STAGES < KT; ++kt)
    k_step<C, true, true>(acc, af, bfr, lds, rsrc, voff, wv, a_row, b_row, fh, fs, kk0, kt, KT);
  if (C::SPREAD && kt >= 1 && kt < KT) {  // the shares of stage KT-1 still to issue
    k_step<C, false, true>(acc, af, bfr, lds, rsrc, voff, wv, a_row, b_row, fh, fs, kk0, kt, KT);
    ++kt;
  }
  for (; kt < KT; ++kt)
    k_step<C, false, false>(acc, af, bfr, lds, rsrc, voff, wv, a_row, b_row, fh, fs, kk0, kt, KT);

  if constexpr (C::KG == 2) {
    // k-group 1 hands its sums to k-group 0 through the ring: block wt's 128 fp32 per lane,
    // lane-contiguous (conflict-free)
    static_assert(C::NW * C::NI * 2 * 16 * 64 * 4 <= STAGES * C::STAGE * 16, "reduction fits the ring");
    float* red = reinterpret_cast<float*>(lds) + (size_t)wt * (C::NI * 2 * 16 * 64) + lane;
    __syncthreads();  // every wave is done reading the ring
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < C::NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) red[((i * 2 + j) * 16 + e) * 64] = acc[i][j][e];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int i = 0; i < C::NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += red[((i * 2 + j) * 16 + e) * 64];
    }
  }

  wide_epilogue<C, EPI>(p, acc, lds, y, yf, m0, ntile, kg, wn, wm, lane, tid);
}

// ---------------------------------------------------------------------------
// Ping-pong kernel for the 256 x 256 (or 192 W x 256 X) tile on v_mfma_f32_16x16x32_bf16.
//
// The part runs these GEMMs power-limited: the same kernels on all-zero operands run 25-35%
// faster, and on random data a stream of 32x32x16 MFMAs alone (no LDS reads, loads or
// barriers) reached 0.58-0.61 of the nominal peak where the same flops as 16x16x32 MFMAs
// reached 0.61-0.66 (a 16x16x32 MFMA reads and writes a quarter of the accumulators for half
// the flops).  So this kernel runs 16x16x32 MFMAs, and keeps every SIMD's matrix core fed from
// registers:
//
// The two waves that share a SIMD (wave w and w + 4) alternate between a compute phase -- one
// k-step (64 k) of MFMAs from fragments already in registers, 64 (48) back to back -- and a
// memory phase -- the 24 (20) ds_read_b128 of their next k-step's fragments plus their share
// of the direct-to-LDS loads of a later stage.  Group 0 (waves 0-3) owns W rows 0 .. WTN-1 of
// the tile and loads the W half of every stage; group 1 (waves 4-7) owns W rows WTN .. and
// loads the X half; wave 4 g + q owns X rows 64 q .. +63.  Group 1 runs one phase behind group
// 0, and every phase ends at a workgroup barrier:
//   phase 2k+1: group 0 multiplies k-step k; group 1 reads k-step k's fragments (ring slot k%2);
//               every wave waits for its loads of stage k+1 (issued in phase 2k) first
//   phase 2k+2: group 0 reads k-step k+1's fragments (slot (k+1)%2), then issues the W half of
//               stage k+2 into slot k%2; group 1 issues the X half of stage k+2 into slot k%2
//               between its first MFMAs of k-step k
// Slot k%2 is free in phase 2k+2: its last readers (group 1, phase 2k+1) waited for their reads
// before the barrier that ended that phase; a memory phase reads a stage every wave waited for
// before the barrier that started the phase.  Each group runs a loop of its own (s_barrier
// syncs the workgroup wherever each wave executes it), so each role's registers are allocated
// on their own.
//
// MFMA operands: A = 16 W rows, B = 16 X rows, k 32: lane l supplies row l % 16 at k chunk
// 4 ks + l / 16 of the 64-k stage (ks = 0, 1), so D[w][x] puts output row x = l % 16 and output
// columns w = 4 (l / 16) .. +3 in a lane: an 8-byte unit.  LDS chunk slot s of row r holds
// global chunk s ^ swz(r), swz(r) = (r >> 1) & 7: the 16 rows of one chunk a fragment read
// touches fall in 16 distinct 16-byte bank groups (and, with the next chunk's 16, in 32 of a
// 512-byte LDS line).  swz does not depend on a fragment's 16-row block, so a lane's fragment
// offsets are base ^ (ks << 6) plus immediates of 2048 bytes per block.
namespace pp {

// Tile: BN W rows x BM X rows x 64 k per stage.  BM = 256 (KG = 1): the two wave groups split the
// W rows.  BM = 128 (KG = 2): each group owns the whole tile and multiplies one k32 half of every
// stage, and group 1's sums are added to group 0's through LDS at the end.
template <int BN_, int BM_, int NW_ = 3>
struct PC {
  static constexpr int BN = BN_, BM = BM_, BK = 64;
  static constexpr int KG = BM == 256 ? 1 : 2;
  static constexpr int KS = 2 / KG;            // k32 sub-steps a wave multiplies per stage
  static constexpr int WTN = BN / 2;           // W rows per wave
  static constexpr int NA = WTN / 16;          // 16-row W blocks per wave (8 or 6)
  static constexpr int NB = 4;                 // 16-row X blocks per wave (64 X rows)
  static constexpr int CPR = 8;                // 16-byte chunks per tile row
  static constexpr int W_CHUNKS = BN * CPR;    // one stage's W half
  static constexpr int X_CHUNKS = BM * CPR;    // one stage's X half
  static constexpr int WL = W_CHUNKS / 64 / 4; // W loads per group-0 wave per stage
  static constexpr int XL = X_CHUNKS / 64 / 4; // X loads per group-1 wave per stage
  static constexpr int PL = WL > XL ? WL : XL;
  // The W and X halves have rings of their own: NW W slots (the W rows come from HBM; stage
  // k + NW is issued 2 NW - 2 phases before it is read), and 3 X slots where they fit beside
  // them in the 160 KiB of LDS, else 2.  X slots follow the W slots.
  static constexpr int NW = NW_;
  static constexpr int NX = (NW * W_CHUNKS + 3 * X_CHUNKS) * 16 <= 160 * 1024 ? 3 : 2;
  static constexpr int X_BASE = NW * W_CHUNKS;  // chunk offset of X slot 0
  static constexpr int TOTAL = NW * W_CHUNKS + NX * X_CHUNKS;
  static_assert(BM == 256 || (BM == 128 && BN == 256), "tile shapes");
  static_assert(NW == 3 || NW == 4, "W ring depth");
  static_assert(TOTAL * 16 <= 160 * 1024, "LDS");
  static __device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
};

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Load j of a wave's stage share (8 tile rows) into LDS chunk base + 256 j (base: the ring slot's
// first chunk plus the wave's first 8-row group).
template <int NL>
__device__ __forceinline__ void issue(u32x4_t* lds, const __amdgpu_buffer_rsrc_t* rs,
                                      const uint32_t* vo, int base, int kt) {
#pragma unroll
  for (int j = 0; j < NL; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs[j], (lds_void*)&lds[base + 256 * j], 16, vo[j],
                                             (uint32_t)(kt * 128), 0, 0);
}

// All fragments of one k-step: the W half at LDS byte offset sa, the X half at sb.
template <class C>
__device__ __forceinline__ void read(const u32x4_t* lds, uint32_t sa, uint32_t sb, uint32_t aA,
                                     uint32_t aB, bf16x8_t (&fa)[C::KS][C::NA],
                                     bf16x8_t (&fb)[C::KS][C::NB]) {
  const char* base = reinterpret_cast<const char*>(lds);
  uint32_t a0 = sa + aA, b0 = sb + aB;
  // (computed here, at the reads: hoisted out of the k loop the offsets of both ring slots
  // would stay live through the MFMAs)
  asm volatile("" : "+v"(a0), "+v"(b0));
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    const char* pa = base + (a0 ^ (uint32_t)(ks << 6));
    const char* pb = base + (b0 ^ (uint32_t)(ks << 6));
#pragma unroll
    for (int i = 0; i < C::NA; ++i) fa[ks][i] = *reinterpret_cast<const bf16x8_t*>(pa + i * 2048);
#pragma unroll
    for (int j = 0; j < C::NB; ++j) fb[ks][j] = *reinterpret_cast<const bf16x8_t*>(pb + j * 2048);
  }
}

// One k-step of MFMAs at raised wave priority; with DMA this wave's loads of stage kt into
// `slot` go out one after each of the first NL MFMAs.
template <class C, int NL, bool DMA>
__device__ __forceinline__ void compute(f32x4_t (&acc)[C::NA][C::NB], const bf16x8_t (&fa)[C::KS][C::NA],
                                        const bf16x8_t (&fb)[C::KS][C::NB], u32x4_t* lds,
                                        const __amdgpu_buffer_rsrc_t* rs, const uint32_t* vo,
                                        int base, int kt) {
  asm volatile("s_setprio 2" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks)
#pragma unroll
    for (int i = 0; i < C::NA; ++i)
#pragma unroll
      for (int j = 0; j < C::NB; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[ks][i], fb[ks][j], acc[i][j], 0, 0, 0);
        const int n = (ks * C::NA + i) * C::NB + j;
        if (DMA && n < NL)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs[n], (lds_void*)&lds[base + 256 * n], 16, vo[n],
                                                   (uint32_t)(kt * 128), 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
  asm volatile("s_setprio 0" ::: "memory");
}

// Output staging swizzle (a bijection of a row's units): 8-byte unit u of row r at
// u ^ ((r & 15) << 2) (64 units a row), u ^ ((r & 7) << 2) (32), u ^ ((r & 3) << 2) (16), and for
// 48 the 32-unit form within the first 32 units and the 16-unit form in the last 16; a write
// instruction covers 16 rows x 4 consecutive units.
template <int UPR>
struct OutSwz {
  static_assert(UPR == 64 || UPR == 48 || UPR == 32 || UPR == 16, "units per row");
  __device__ __forceinline__ int operator()(int u, int r) const {
    if constexpr (UPR == 64) return u ^ ((r & 15) << 2);
    else if constexpr (UPR == 32) return u ^ ((r & 7) << 2);
    else if constexpr (UPR == 16) return u ^ ((r & 3) << 2);
    else return u < 32 ? u ^ ((r & 7) << 2) : u ^ ((r & 3) << 2);
  }
};

// Tile b of the nb tiles of p (the LDS ring: at least PC<BN, BM, NWR>::TOTAL chunks).
template <int EPI, int BN, int BM, int NWR>
__device__ __forceinline__ void pp_tile(const GemmParams& p, int m_tiles, int b, int nb,
                                        u32x4_t* lds) {
  using C = PC<BN, BM, NWR>;
  constexpr int NA = C::NA, NB = C::NB, WL = C::WL, XL = C::XL, PL = C::PL, KS = C::KS;
  static_assert(EPI == kGemmBf16 || EPI == kGemmResid || EPI == kGemmSwiglu || EPI == kGemmQkvRope,
                "bf16 epilogues");
  static_assert(EPI != kGemmSwiglu || BN == 256, "SwiGLU tiles are 256 W rows");
  static_assert(EPI != kGemmQkvRope || (BN == 192 && BM == 256), "QKV + RoPE: 192 x 256 tiles");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wv >> 2, gw = wv & 3;
  // the wave's output block: W rows wn * WTN .., X rows wm * 64 ..; with KG = 2 its k32 half grp
  const int wn = C::KG == 1 ? grp : gw >> 1, wm = C::KG == 1 ? gw : gw & 1;
  int mtile, ntile;
  tile_of<1>(b, nb, m_tiles, mtile, ntile);
  const int m0 = mtile * BM;
  const int KT = p.K / 64;

  // this wave's share of a stage: 8-row groups gw + 4 j of its half (W or X); lane i fills LDS
  // slot (row 8 g + i / 8, chunk i % 8) from global chunk (i % 8) ^ swz(row)
  __amdgpu_buffer_rsrc_t rs[PL];
  uint32_t vo[PL];
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int g = gw + 4 * j;
    rs[j] = grp == 0 ? w_group<EPI, BN>(p, ntile, min(g, BN / 8 - 1) * 8) : x_group(p, m0, g * 8);
    const int rl = lane / 8, c = (lane % 8) ^ C::swz(g * 8 + rl);
    vo[j] = (uint32_t)((rl * p.K + c * 8) * 2);
  }
  const int dst0 = (grp == 0 ? 0 : C::X_BASE) + gw * 64;  // the wave's first row group, slot 0
  const int slot_chunks = grp == 0 ? C::W_CHUNKS : C::X_CHUNKS;

  f32x4_t acc[NA][NB];
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // fragment byte offsets within a stage (ks = 0, block 0): lane l reads row base + l % 16 at
  // chunk (l / 16) ^ swz(row)
  const int fr = lane & 15, fq = lane >> 4;
  const uint32_t chunk0 = (uint32_t)((fq ^ C::swz(fr)) * 16) ^ (C::KG == 2 ? (uint32_t)(grp << 6) : 0u);
  const uint32_t aA = (uint32_t)((wn * C::WTN + fr) * C::CPR * 16) + chunk0;
  const uint32_t aB = (uint32_t)((wm * 64 + fr) * C::CPR * 16) + chunk0;
  bf16x8_t fa[KS][NA], fb[KS][NB];

  uint16_t* const y = p.y;
  asm volatile("" ::"s"(y), "s"(p.ldy), "s"(p.M), "s"(p.N));

  // stage k's W half lives in W slot k % NW, its X half in X slot k % NX.  The wait that ends
  // phase 2k+1 leaves in flight only this wave's loads of stages issued after k+1.
  constexpr int NW = C::NW, NX = C::NX;
  constexpr uint32_t WSB = C::W_CHUNKS * 16, XSB = C::X_CHUNKS * 16, XB0 = C::X_BASE * 16;
  if (grp == 0) {
#pragma unroll
    for (int t = 0; t < NW; ++t)
      if (t < KT) issue<WL>(lds, rs, vo, dst0 + t * C::W_CHUNKS, t);
    if (KT >= NW) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NW - 1) * WL) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // phase 0: fragments of k-step 0
    read<C>(lds, 0, XB0, aA, aB, fa, fb);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    int sw = 0, sx = 0;  // W and X slots of stage k
#pragma unroll 1
    for (int k = 0; k < KT; ++k) {
      const int swn = sw + 1 == NW ? 0 : sw + 1, sxn = sx + 1 == NX ? 0 : sx + 1;
      // phase 2k+1: multiply k-step k
      compute<C, WL, false>(acc, fa, fb, lds, rs, vo, 0, 0);
      // stage k+1 must have landed; stages k+2 .. min(k+NW-1, KT-1) may stay in flight
      if (NW == 4 && k + 3 < KT) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * WL) : "memory");
      else if (k + 2 < KT) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(WL) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      // phase 2k+2: fragments of k-step k+1, then the W half of stage k+NW into W slot sw
      if (k + 1 < KT) read<C>(lds, swn * WSB, XB0 + sxn * XSB, aA, aB, fa, fb);
      if (k + NW < KT) issue<WL>(lds, rs, vo, dst0 + sw * C::W_CHUNKS, k + NW);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      sw = swn;
      sx = sxn;
    }
  } else {
#pragma unroll
    for (int t = 0; t < NX; ++t)
      if (t < KT) issue<XL>(lds, rs, vo, dst0 + t * C::X_CHUNKS, t);
    if (KT >= NX) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NX - 1) * XL) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    int k = 0, sw = 0, sx = 0;
#pragma unroll 1
    for (; k + NX < KT; ++k) {
      // phase 2k+1: fragments of k-step k
      read<C>(lds, sw * WSB, XB0 + sx * XSB, aA, aB, fa, fb);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NX - 2) * XL) : "memory");
      // phase 2k+2: the X half of stage k+NX into X slot sx while multiplying k-step k
      compute<C, XL, true>(acc, fa, fb, lds, rs, vo, dst0 + sx * C::X_CHUNKS, k + NX);
      asm volatile("s_barrier" ::: "memory");
      sw = sw + 1 == NW ? 0 : sw + 1;
      sx = sx + 1 == NX ? 0 : sx + 1;
    }
#pragma unroll 1
    for (; k < KT; ++k) {
      read<C>(lds, sw * WSB, XB0 + sx * XSB, aA, aB, fa, fb);
      if (k + 2 < KT)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NX - 2) * XL) : "memory");
      else
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      compute<C, XL, false>(acc, fa, fb, lds, rs, vo, 0, 0);
      asm volatile("s_barrier" ::: "memory");
      sw = sw + 1 == NW ? 0 : sw + 1;
      sx = sx + 1 == NX ? 0 : sx + 1;
    }
  }
  (void)slot_chunks;

  // ---- epilogue: acc[i][j][r] = D[W row wn*WTN + 16 i + 4 (lane/16) + r][X row wm*64 + 16 j +
  //      lane%16]; staged in the ring as [256][OUTN] bf16 (8-byte units), then stored as rows
  if constexpr (C::KG == 2) {
    // group 1 hands its sums to group 0 through the ring, half the W blocks at a time (a lane's
    // 16-byte accumulators lane-contiguous: conflict-free)
    constexpr int HALF = NA / 2 * NB;
    static_assert(4 * HALF * 64 * 16 <= C::TOTAL * 16, "reduction fits the ring");
    f32x4_t* red = reinterpret_cast<f32x4_t*>(lds) + (size_t)gw * HALF * 64 + lane;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __syncthreads();  // the ring (or the previous half) is free
      if (grp == 1) {
#pragma unroll
        for (int i = 0; i < NA / 2; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j) red[(i * NB + j) * 64] = acc[h * NA / 2 + i][j];
      }
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int i = 0; i < NA / 2; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[h * NA / 2 + i][j] += red[(i * NB + j) * 64];
      }
    }
  }
  constexpr int OUTN = (EPI == kGemmSwiglu) ? BN / 2 : BN;
  constexpr int UPR = OUTN / 4;
  static_assert(BM * OUTN * 2 <= C::TOTAL * 16, "output tile must fit the LDS ring");
  const OutSwz<UPR> swz;
  uint2* ot = reinterpret_cast<uint2*>(lds);
  __syncthreads();  // every wave is done reading the ring
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (C::KG == 2 && grp != 0) break;
    const int r = wm * 64 + 16 * j + fr;
    if constexpr (EPI == kGemmSwiglu) {
      // W rows of the wave: [32 gate | 32 up] x 2, so block i (gate) pairs with i + 2 (up)
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        if ((i & 2) != 0) continue;
        uint32_t o[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float v[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float gt = bf2f(f2bf(acc[i][j][2 * q + e]));
            const float up = bf2f(f2bf(acc[i + 2][j][2 * q + e]));
            v[e] = gt * (1.0f / (1.0f + expf(-gt))) * up;
          }
          o[q] = pack_bf2(v[0], v[1]);
        }
        const int u = (wn * (C::WTN / 64) + i / 4) * 8 + (i & 1) * 4 + fq;
        ot[r * UPR + swz(u, r)] = make_uint2(o[0], o[1]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int u = wn * (C::WTN / 4) + 4 * i + fq;
        ot[r * UPR + swz(u, r)] = make_uint2(pack_bf2(acc[i][j][0], acc[i][j][1]),
                                             pack_bf2(acc[i][j][2], acc[i][j][3]));
      }
    }
  }
  __syncthreads();
  if constexpr (EPI == kGemmQkvRope) rope_copy_out<512>(p, ot, m0, ntile, tid, swz);
  else tile_copy_out<512, BM, UPR, EPI>(p, ot, y, m0, ntile * OUTN, tid, swz);
}

template <int EPI, int BN, int BM, int NWR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_pp_kernel(GemmParams p, int m_tiles) {
  __shared__ u32x4_t lds[PC<BN, BM, NWR>::TOTAL];
  pp_tile<EPI, BN, BM, NWR>(p, m_tiles, blockIdx.x, gridDim.x, lds);
}

// Two column ranges of one product in one launch: workgroups 0 .. nb1-1 take the BM1-row X
// tiles of p1, the rest the BM2-row tiles of p2 (gate/up at S = 2048: three rounds of 256 x 256
// tiles, then the last 2048 columns as 256 x 128 tiles, each starting on a CU as soon as the CU's
// third big tile ends instead of after a kernel boundary).
template <int EPI, int BN, int BM1, int BM2>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_pp_dual_kernel(GemmParams p1, int m_tiles1, int nb1, GemmParams p2, int m_tiles2) {
  constexpr int T1 = PC<BN, BM1, 3>::TOTAL, T2 = PC<BN, BM2, 3>::TOTAL;
  __shared__ u32x4_t lds[T1 > T2 ? T1 : T2];
  if ((int)blockIdx.x < nb1)
    pp_tile<EPI, BN, BM1, 3>(p1, m_tiles1, blockIdx.x, nb1, lds);
  else
    pp_tile<EPI, BN, BM2, 3>(p2, m_tiles2, blockIdx.x - nb1, gridDim.x - nb1, lds);
}

}  // namespace pp

// ---------------------------------------------------------------------------
// Medium-M kernel (17-128 rows: prompts of a few dozen tokens), where a product is bound by its
// weight stream: 64 W rows x XR X rows (XR = 64 or 128) a workgroup, 4 waves each owning 16 W
// rows and all XR X rows (XR / 16 MFMA blocks, v_mfma_f32_16x16x32_bf16), over a K range of
// K / k_splits.  64-k stages (128-byte rows, 8-row direct-to-LDS loads: whole lines) in a ring
// of S slots (4 at XR = 64: 64 KiB, two workgroups a CU; 3 at 128): stage k + S - 1 is issued at
// k-step k, so S - 1 stages are in flight per workgroup.  The weight rows are read once per
// launch and loaded nontemporal (cache policy nt, as the GEMV's); measured 3-5% faster per
// 17-64-token prefill (1-1.5% at 100-128) than the default policy, which the X rows, re-read by
// every tile, keep.
// One barrier per k-step: after it, every wave's loads of stage k have landed and every wave is
// done with slot (k - 1) % S, which takes stage k + S - 1.
// Epilogues: fp32 partial planes (split K, reduced by the split reductions), bf16, residual,
// and SwiGLU over [32 gate | 32 up] W rows (output columns 32 t ..), through an fp32 LDS tile.
// The X rows are re-read by every W tile from L2 (one K range: XR x K / k_splits x 2 bytes).
namespace mid {

using pp::f32x4_t;

template <int XR_, int WR_>
struct MC {
  static constexpr int XR = XR_, WR = WR_;
  static constexpr int NWV = WR / 16;                // waves, 16 W rows each
  static constexpr int NB = XR / 16;                 // X blocks per wave
  static constexpr int W_CHUNKS = WR * 8, X_CHUNKS = XR * 8;
  static constexpr int STAGE = W_CHUNKS + X_CHUNKS;  // 16-byte chunks per stage
  static constexpr int S = XR == 64 ? 4 : 3;         // ring slots
  static constexpr int WL = WR / 8 / NWV, XL = XR / 8 / NWV;  // 8-row loads per wave per stage
  static constexpr int L = WL + XL;
  static constexpr int U = WR / 4;                   // 16-byte units of an fp32 output row
  static_assert(XR == 64 || XR == 128, "X rows per tile");
  static_assert(WR == 64 || WR == 128, "W rows per tile");
  static_assert(S * STAGE * 16 <= 160 * 1024, "LDS");
};

// This wave's loads of stage kt into ring slot `slot`: W groups wv + NWV j, then X groups.
template <class C>
__device__ __forceinline__ void mid_issue(u32x4_t* lds, const __amdgpu_buffer_rsrc_t* rs,
                                          uint32_t vo, int wv, int slot, int kt) {
  const uint32_t koff = (uint32_t)(kt * 128);
#pragma unroll
  for (int j = 0; j < C::WL; ++j) {  // weight rows: nontemporal (aux 2 = nt)
    const int dst = slot * C::STAGE + (wv + C::NWV * j) * 64;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs[j], (lds_void*)&lds[dst], 16, vo, koff, 0, 2);
  }
#pragma unroll
  for (int j = C::WL; j < C::L; ++j) {  // X rows: default policy
    const int dst = slot * C::STAGE + C::W_CHUNKS + (wv + C::NWV * (j - C::WL)) * 64;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs[j], (lds_void*)&lds[dst], 16, vo, koff, 0, 0);
  }
}

// s_waitcnt vmcnt(n * L): n younger stages may stay in flight (n <= 6).
template <int L>
__device__ __forceinline__ void mid_wait(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * L) : "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * L) : "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * L) : "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * L) : "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * L) : "memory"); break;
  }
}

template <int EPI, int XR, int WR>
__global__ __launch_bounds__(WR * 4) void gemm_mid_kernel(GemmParams p, int n_tiles) {
  using C = MC<XR, WR>;
  constexpr int U = C::U;
  constexpr int NB = C::NB, S = C::S;
  static_assert(EPI == kGemmF32 || EPI == kGemmBf16 || EPI == kGemmResid || EPI == kGemmSwiglu,
                "epilogues");
  __shared__ u32x4_t lds[S * C::STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nsplit = max(1, p.k_splits);
  const int split = blockIdx.x / n_tiles, ntile = blockIdx.x - split * n_tiles;
  const int KT = p.K / 64 / nsplit;
  const int k0 = split * KT * 64;

  // loads: W groups g = wv + NWV j of 8 rows, X groups likewise; row 8 g + r has
  // swz = (4 (g & 1) + r / 2) & 7 with g & 1 = wv & 1, so one lane offset serves every group
  __amdgpu_buffer_rsrc_t rs[C::L];
#pragma unroll
  for (int j = 0; j < C::WL; ++j) rs[j] = w_group<EPI, WR>(p, ntile, (wv + C::NWV * j) * 8, k0);
#pragma unroll
  for (int j = 0; j < C::XL; ++j) rs[C::WL + j] = x_group(p, 0, (wv + C::NWV * j) * 8, k0);
  const int rl = lane >> 3;
  const uint32_t vo =
      (uint32_t)((rl * p.K + (((lane & 7) ^ ((4 * (wv & 1) + (rl >> 1)) & 7)) * 8)) * 2);

  // fragments: lane l reads row l % 16 of its block at chunk (l / 16 + 4 ks) ^ ((row >> 1) & 7)
  const int fr = lane & 15, fq = lane >> 4;
  const uint32_t sw0 = (uint32_t)((fq ^ ((fr >> 1) & 7)) * 16);
  const uint32_t aA = (uint32_t)((wv * 16 + fr) * 128) + sw0;
  const uint32_t aB = (uint32_t)(C::W_CHUNKS * 16 + fr * 128) + sw0;

  f32x4_t acc[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < S - 1; ++t)
    if (t < KT) mid_issue<C>(lds, rs, vo, wv, t, t);
  const char* base = reinterpret_cast<const char*>(lds);
  int slot = 0;
#pragma unroll 1
  for (int k = 0; k < KT; ++k) {
    // stage k has landed (stages k+1 .. min(k+S-2, KT-1) may stay in flight) for every wave
    mid_wait<C::L>(min(S - 2, KT - 1 - k));
    asm volatile("s_barrier" ::: "memory");
    if (k + S - 1 < KT) mid_issue<C>(lds, rs, vo, wv, slot == 0 ? S - 1 : slot - 1, k + S - 1);
    uint32_t ra = (uint32_t)(slot * C::STAGE * 16) + aA, rb = (uint32_t)(slot * C::STAGE * 16) + aB;
    asm volatile("" : "+v"(ra), "+v"(rb));
    bf16x8_t fa[2], fb[2][NB];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      fa[ks] = *reinterpret_cast<const bf16x8_t*>(base + (ra ^ (uint32_t)(ks << 6)));
#pragma unroll
      for (int j = 0; j < NB; ++j)
        fb[ks][j] = *reinterpret_cast<const bf16x8_t*>(base + (rb ^ (uint32_t)(ks << 6)) + j * 2048);
    }
    // all of the step's reads issued before its first MFMA (left alone, the scheduler puts each
    // read just before its use: one LDS round trip per MFMA)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[ks], fb[ks][j], acc[j], 0, 0, 0);
    slot = slot == S - 1 ? 0 : slot + 1;
  }

  // epilogue: acc[j][r] = D[W col 16 wv + 4 (lane / 16) + r][X row 16 j + lane % 16], staged as
  // an fp32 [XR][WR] tile (row m at WR m floats, 16-byte unit u at u ^ (m % U))
  float4* ot = reinterpret_cast<float4*>(lds);
  constexpr int T = 64 * C::NWV;
  const auto at = [&](int m, int u) -> float4& { return ot[m * U + (u ^ (m & (U - 1)))]; };
  __syncthreads();  // every wave is done with the ring (its last wait was vmcnt(0))
#pragma unroll
  for (int j = 0; j < NB; ++j)
    at(16 * j + fr, 4 * wv + fq) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
  __syncthreads();
  if constexpr (EPI == kGemmF32) {
    float* const yf = p.yf + (size_t)split * p.M * p.ldy;
    for (int it = tid; it < XR * U; it += T) {
      const int m = it / U, u = it % U, n = ntile * WR + 4 * u;
      if (m < p.M && n < p.N) *reinterpret_cast<float4*>(yf + (size_t)m * p.ldy + n) = at(m, u);
    }
  } else if constexpr (EPI == kGemmSwiglu) {
    // W rows [32 gate | 32 up] x (WR / 64): tile columns 64 b .. 64 b + 31 are the gate of output
    // columns ntile WR / 2 + 32 b + c, 64 b + 32 .. the up of the same
    constexpr int CPR = WR / 16;  // 8-column output groups per row
    for (int it = tid; it < XR * CPR; it += T) {
      const int m = it / CPR, c = it % CPR, b = c >> 2, c8 = c & 3;
      const int n = ntile * (WR / 2) + 32 * b + 8 * c8;
      if (m >= p.M || n >= p.N) continue;
      uint32_t o[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 g = at(m, 16 * b + 2 * c8 + h);
        const float4 up = at(m, 16 * b + 8 + 2 * c8 + h);
        const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {up.x, up.y, up.z, up.w};
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gt = bf2f(f2bf(gv[e])), ut = bf2f(f2bf(uv[e]));
          v[e] = gt * (1.0f / (1.0f + expf(-gt))) * ut;
        }
        o[2 * h] = pack_bf2(v[0], v[1]);
        o[2 * h + 1] = pack_bf2(v[2], v[3]);
      }
      *reinterpret_cast<uint4*>(p.y + (size_t)m * p.ldy + n) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    constexpr int CPR = WR / 8;  // 8-column groups per row
    for (int it = tid; it < XR * CPR; it += T) {
      const int m = it / CPR, c8 = it % CPR, n = ntile * WR + 8 * c8;
      if (m >= p.M || n >= p.N) continue;
      const float4 a = at(m, 2 * c8), b = at(m, 2 * c8 + 1);
      uint4 o = make_uint4(pack_bf2(a.x, a.y), pack_bf2(a.z, a.w), pack_bf2(b.x, b.y), pack_bf2(b.z, b.w));
      uint16_t* dst = p.y + (size_t)m * p.ldy + n;
      if constexpr (EPI == kGemmResid) {
        // y = bf16(y + bf16(acc)) (residual_add.cu:17-19)
        const uint4 r = *reinterpret_cast<const uint4*>(dst);
        o = make_uint4(pack_bf2(bf_lo(r.x) + bf_lo(o.x), bf_hi(r.x) + bf_hi(o.x)),
                       pack_bf2(bf_lo(r.y) + bf_lo(o.y), bf_hi(r.y) + bf_hi(o.y)),
                       pack_bf2(bf_lo(r.z) + bf_lo(o.z), bf_hi(r.z) + bf_hi(o.z)),
                       pack_bf2(bf_lo(r.w) + bf_lo(o.w), bf_hi(r.w) + bf_hi(o.w)));
      }
      *reinterpret_cast<uint4*>(dst) = o;
    }
  }
}

}  // namespace mid

}  // namespace wide

template <int EPI, int BM = 128, int BK = 64, int STAGES = 3, int MAPG = 1, int WBN = 256, int KG = 1>
int launch_wide(const GemmParams& p, hipStream_t st) {
  const int m_tiles = (p.M + BM - 1) / BM;
  const int n_tiles = (EPI == kGemmSwiglu) ? (p.N + 127) / 128 : (p.N + WBN - 1) / WBN;
  const long long blocks = (long long)m_tiles * n_tiles * std::max(1, p.k_splits);
  IE_REQUIRE(blocks <= 0x7fffffff, "gemm: too many tiles");
  hipLaunchKernelGGL((wide::gemm_wide_kernel<EPI, BM, BK, STAGES, MAPG, WBN, KG>), dim3((unsigned)blocks),
                     dim3(wide::Cfg<BM, BK, STAGES, WBN, KG>::THREADS), 0, st, p, m_tiles);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int EPI, int WBN, int XBM = 256, int NW = 3>
int launch_pp(const GemmParams& p, hipStream_t st) {
  const int m_tiles = (p.M + XBM - 1) / XBM;
  const int n_tiles = (EPI == kGemmSwiglu) ? (p.N + WBN / 2 - 1) / (WBN / 2) : (p.N + WBN - 1) / WBN;
  const long long blocks = (long long)m_tiles * n_tiles;
  IE_REQUIRE(blocks <= 0x7fffffff && p.k_splits <= 1, "gemm: ping-pong tiles");
  hipLaunchKernelGGL((wide::pp::gemm_pp_kernel<EPI, WBN, XBM, NW>), dim3((unsigned)blocks), dim3(512), 0,
                     st, p, m_tiles);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int EPI>
int launch_pp_dual(const GemmParams& head, const GemmParams& tail, hipStream_t st) {
  const int m1 = (head.M + 255) / 256, m2 = (tail.M + 127) / 128;
  const int n1 = (EPI == kGemmSwiglu) ? (head.N + 127) / 128 : (head.N + 255) / 256;
  const int n2 = (EPI == kGemmSwiglu) ? (tail.N + 127) / 128 : (tail.N + 255) / 256;
  const long long b1 = (long long)m1 * n1, b2 = (long long)m2 * n2;
  IE_REQUIRE(b1 + b2 <= 0x7fffffff && head.k_splits <= 1 && tail.k_splits <= 1,
             "gemm: ping-pong tiles");
  hipLaunchKernelGGL((wide::pp::gemm_pp_dual_kernel<EPI, 256, 256, 128>), dim3((unsigned)(b1 + b2)),
                     dim3(512), 0, st, head, m1, (int)b1, tail, m2);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

template <int EPI>
int launch_e(const GemmParams& p, hipStream_t st) {
  const int m_tiles = (p.M + BM - 1) / BM;
  const int n_tiles = (EPI == kGemmSwiglu) ? (p.N + 63) / 64 : (p.N + BN - 1) / BN;
  const long long blocks = (long long)m_tiles * n_tiles;
  IE_REQUIRE(blocks <= 0x7fffffff, "gemm: too many tiles");
  hipLaunchKernelGGL((gemm_kernel<EPI>), dim3((unsigned)blocks), dim3(256), 0, st, p, m_tiles);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

// ---------------------------------------------------------------------------
// Tile shape by a cost model: time = rounds of workgroups over the 256 CUs x the time of one
// tile at the measured per-CU rate of that shape (256x256 and 192x256: 1085, 256x128: 900,
// 128x128: 750 TFLOP/s over the chip at full occupancy).  Big tiles win when they fill the
// chip; at small S the 128 x 128 tile keeps more CUs busy.  192 W rows x 256 X rows gives
// exactly 256 tiles for the QKV projection at S = 2048 (N = 6144).
enum { kTileSmall, kTileWide, kTileBig, kTileBig192, kTileKinds };

// Kernel of the bf16 wide tiles: 0 = the DMA-ring wide kernels; 1 = the ping-pong kernel for
// the 256-row X tiles; 2 (default) = the ping-pong kernel for those and for the 128-row X tiles;
// 3 = as 2 with 4 W ring slots (2 X slots) on the 256 x 128 and 192 x 256 tiles.
// Outputs are bit-identical across all (same per-accumulator MFMA order).
int g_gemm_schedule = 2;

struct TileKind {
  int tm, tn, tn_swiglu;  // X rows, output columns (plain / SwiGLU) per tile
  double unit;            // relative time of one tile
};
constexpr TileKind kTiles[kTileKinds] = {
    {128, 128, 64, 128.0 * 128 / 750.0},
    {128, 256, 128, 256.0 * 128 / 900.0},
    {256, 256, 128, 256.0 * 256 / 1085.0},
    {256, 192, 0, 192.0 * 256 / 1085.0},
};

bool tile_ok(int kind, int epi, const GemmParams& p) {
  if (kind == kTileSmall) return true;
  if (p.M < kWideMinRows) return false;
  if (kind == kTileWide) return true;
  if (epi == kGemmF32) return false;
  return kind == kTileBig || epi != kGemmSwiglu;
}

long long tile_count(int kind, int epi, int M, int N) {
  const TileKind& t = kTiles[kind];
  const int tn = epi == kGemmSwiglu ? t.tn_swiglu : t.tn;
  return (long long)((M + t.tm - 1) / t.tm) * ((N + tn - 1) / tn);
}

double tile_cost(int kind, int epi, int M, int N) {
  return (double)((tile_count(kind, epi, M, N) + 255) / 256) * kTiles[kind].unit;
}

int launch_kind(int kind, int epi, const GemmParams& p, hipStream_t st) {
  if (g_gemm_schedule == 3 && kind == kTileWide && epi != kGemmF32) {
    switch (epi) {
      case kGemmBf16: return launch_pp<kGemmBf16, 256, 128, 4>(p, st);
      case kGemmResid: return launch_pp<kGemmResid, 256, 128, 4>(p, st);
      case kGemmSwiglu: return launch_pp<kGemmSwiglu, 256, 128, 4>(p, st);
    }
  }
  if (g_gemm_schedule == 3 && kind == kTileBig192) {
    switch (epi) {
      case kGemmBf16: return launch_pp<kGemmBf16, 192, 256, 4>(p, st);
      case kGemmResid: return launch_pp<kGemmResid, 192, 256, 4>(p, st);
    }
  }
  if (g_gemm_schedule >= 2 && kind == kTileWide && epi != kGemmF32) {
    switch (epi) {
      case kGemmBf16: return launch_pp<kGemmBf16, 256, 128>(p, st);
      case kGemmResid: return launch_pp<kGemmResid, 256, 128>(p, st);
      case kGemmSwiglu: return launch_pp<kGemmSwiglu, 256, 128>(p, st);
    }
  }
  switch (kind * 4 + epi) {
    case kTileSmall * 4 + kGemmBf16: return launch_e<kGemmBf16>(p, st);
    case kTileSmall * 4 + kGemmResid: return launch_e<kGemmResid>(p, st);
    case kTileSmall * 4 + kGemmF32: return launch_e<kGemmF32>(p, st);
    case kTileSmall * 4 + kGemmSwiglu: return launch_e<kGemmSwiglu>(p, st);
    case kTileWide * 4 + kGemmBf16: return launch_wide<kGemmBf16, 128, 64, 3, 1, 256, 2>(p, st);
    case kTileWide * 4 + kGemmResid: return launch_wide<kGemmResid, 128, 64, 3, 1, 256, 2>(p, st);
    case kTileWide * 4 + kGemmF32: return launch_wide<kGemmF32, 128, 64, 3, 1, 256, 2>(p, st);
    case kTileWide * 4 + kGemmSwiglu: return launch_wide<kGemmSwiglu, 128, 64, 3, 1, 256, 2>(p, st);
  }
  if (g_gemm_schedule >= 1) {
    switch (kind * 4 + epi) {
      case kTileBig * 4 + kGemmBf16: return launch_pp<kGemmBf16, 256>(p, st);
      case kTileBig * 4 + kGemmResid: return launch_pp<kGemmResid, 256>(p, st);
      case kTileBig * 4 + kGemmSwiglu: return launch_pp<kGemmSwiglu, 256>(p, st);
      case kTileBig192 * 4 + kGemmBf16: return launch_pp<kGemmBf16, 192>(p, st);
      case kTileBig192 * 4 + kGemmResid: return launch_pp<kGemmResid, 192>(p, st);
    }
  }
  switch (kind * 4 + epi) {
    case kTileBig * 4 + kGemmBf16: return launch_wide<kGemmBf16, 256, 64, 2>(p, st);
    case kTileBig * 4 + kGemmResid: return launch_wide<kGemmResid, 256, 64, 2>(p, st);
    case kTileBig * 4 + kGemmSwiglu: return launch_wide<kGemmSwiglu, 256, 64, 2>(p, st);
    case kTileBig192 * 4 + kGemmBf16: return launch_wide<kGemmBf16, 256, 64, 2, 1, 192>(p, st);
    case kTileBig192 * 4 + kGemmResid: return launch_wide<kGemmResid, 256, 64, 2, 1, 192>(p, st);
  }
  set_error("gemm: bad epilogue %d", epi);
  return IE_ERR_INVALID_ARG;
}

// Output columns [c, N) of p as a GEMM of its own (c a multiple of 64, and of 16 past a
// weight split point).
GemmParams column_tail(int epi, const GemmParams& p, int c) {
  GemmParams q = p;
  const size_t off = (size_t)c * p.K;
  q.N = p.N - c;
  if (p.y) q.y = p.y + c;
  if (p.yf) q.yf = p.yf + c;
  if (epi == kGemmSwiglu) {
    q.w0 = p.w0 + off;
    q.w1 = p.w1 + off;
    return q;
  }
  const int e0 = std::min(p.n0, p.N), e1 = std::min(p.n0 + p.n1, p.N);
  if (c < e0) {
    q.w0 = p.w0 + off;
    q.n0 = e0 - c;
  } else if (c < e1) {
    q.w0 = p.w1 + (size_t)(c - e0) * p.K;
    q.n0 = e1 - c;
    q.w1 = p.w2;
    q.n1 = q.N - q.n0;
  } else {
    q.w0 = p.w2 + (size_t)(c - e1) * p.K;
    q.n0 = q.N;
    q.n1 = 0;
  }
  return q;
}

// Cheapest tile shape; with `split`, a partial last round of that shape may instead be run as
// a second launch over the remaining output columns with the shape that fills the chip for
// them (gate/up at S = 2048: 3 rounds of 256 x 256 tiles, then the last 2048 columns as one
// round of 256 x 128 tiles, in place of a half-empty fourth round).
// Cheapest tile shape for p.
int best_kind(int epi, const GemmParams& p) {
  int best = kTileSmall;
  double best_cost = tile_cost(kTileSmall, epi, p.M, p.N);
  for (int k = kTileWide; k < kTileKinds; ++k) {
    if (!tile_ok(k, epi, p)) continue;
    const double c = tile_cost(k, epi, p.M, p.N);
    if (c < best_cost) best = k, best_cost = c;
  }
  return best;
}

int launch_tiled(int epi, const GemmParams& p, hipStream_t st, bool split) {
  const int best = best_kind(epi, p);
  const double best_cost = tile_cost(best, epi, p.M, p.N);
  if (split) {
    const TileKind& t = kTiles[best];
    const int tn = epi == kGemmSwiglu ? t.tn_swiglu : t.tn;
    const int m_tiles = (p.M + t.tm - 1) / t.tm;
    const long long tiles = tile_count(best, epi, p.M, p.N);
    if (tiles > 256 && tiles % 256 != 0 && 256 % m_tiles == 0) {
      const int c = (int)(tiles / 256 * 256 / m_tiles) * tn;  // columns of the full rounds
      const GemmParams tail = column_tail(epi, p, c);
      double tail_cost = 1e30;
      for (int k = kTileSmall; k < kTileKinds; ++k)
        if (tile_ok(k, epi, tail)) tail_cost = std::min(tail_cost, tile_cost(k, epi, tail.M, tail.N));
      if ((double)(tiles / 256) * t.unit + tail_cost < best_cost) {
        GemmParams head = p;
        head.N = c;
        // 256 x 256 then 256 x 128 ping-pong tiles: one launch
        if (g_gemm_schedule >= 2 && best == kTileBig && best_kind(epi, tail) == kTileWide) {
          switch (epi) {
            case kGemmBf16: return launch_pp_dual<kGemmBf16>(head, tail, st);
            case kGemmResid: return launch_pp_dual<kGemmResid>(head, tail, st);
            case kGemmSwiglu: return launch_pp_dual<kGemmSwiglu>(head, tail, st);
          }
        }
        const int rc = launch_kind(best, epi, head, st);
        if (rc != IE_OK) return rc;
        return launch_tiled(epi, tail, st, false);
      }
    }
  }
  return launch_kind(best, epi, p, st);
}

// Sum of the split planes of 8 consecutive partials.
__device__ __forceinline__ void split_sum8(const float* src, size_t plane, int splits, float4& a,
                                           float4& b) {
  a = *reinterpret_cast<const float4*>(src);
  b = *reinterpret_cast<const float4*>(src + 4);
  for (int s = 1; s < splits; ++s) {
    const float4 c = *reinterpret_cast<const float4*>(src + s * plane);
    const float4 d = *reinterpret_cast<const float4*>(src + s * plane + 4);
    a.x += c.x, a.y += c.y, a.z += c.z, a.w += c.w;
    b.x += d.x, b.y += d.y, b.z += d.z, b.w += d.w;
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  g = bf2f(f2bf(g));
  return g * (1.0f / (1.0f + expf(-g))) * bf2f(f2bf(u));
}

// Split K's reduction: y = epilogue(sum of the fp32 partial planes), 8 columns per thread.
// bf16: bf16(sum); residual: bf16(y + bf16(sum)); SwiGLU (planes of 2N columns, gate then up):
// bf16(silu(bf16(g)) * bf16(u)) -- the unsplit epilogues' roundings.
template <int EPI>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* part, int splits, int M,
                                                           int N, uint16_t* y, int ldy) {
  constexpr int W = EPI == kGemmSwiglu ? 2 : 1;  // plane width in output columns
  const int per_row = N / 8;
  const size_t total = (size_t)M * per_row, plane = (size_t)M * N * W;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int m = (int)(i / per_row), n = (int)(i % per_row) * 8;
    const float* src = part + (size_t)m * N * W + n;
    float4 a, b;
    split_sum8(src, plane, splits, a, b);
    if constexpr (EPI == kGemmSwiglu) {
      float4 c, d;
      split_sum8(src + N, plane, splits, c, d);
      a = make_float4(silu_mul(a.x, c.x), silu_mul(a.y, c.y), silu_mul(a.z, c.z), silu_mul(a.w, c.w));
      b = make_float4(silu_mul(b.x, d.x), silu_mul(b.y, d.y), silu_mul(b.z, d.z), silu_mul(b.w, d.w));
    }
    uint4 o = make_uint4(pack_bf2(a.x, a.y), pack_bf2(a.z, a.w), pack_bf2(b.x, b.y), pack_bf2(b.z, b.w));
    uint16_t* dst = y + (size_t)m * ldy + n;
    if constexpr (EPI == kGemmResid) {
      const uint4 r = *reinterpret_cast<const uint4*>(dst);
      o = make_uint4(pack_bf2(bf_lo(r.x) + bf_lo(o.x), bf_hi(r.x) + bf_hi(o.x)),
                     pack_bf2(bf_lo(r.y) + bf_lo(o.y), bf_hi(r.y) + bf_hi(o.y)),
                     pack_bf2(bf_lo(r.z) + bf_lo(o.z), bf_hi(r.z) + bf_hi(o.z)),
                     pack_bf2(bf_lo(r.w) + bf_lo(o.w), bf_hi(r.w) + bf_hi(o.w)));
    }
    *reinterpret_cast<uint4*>(dst) = o;
  }
}

// The residual reduction followed by the RMSNorm of the same rows (N = 4096, one 256-thread
// workgroup per row): y = bf16(y + bf16(sum)), then rn_out = bf16(bf16(y * r) * w) with r from
// the fp32 sum of squares of the new y -- each thread owns 16-byte chunks t and t + 256 of the
// row and sums their squares in the same order as rmsnorm_kernel, so both outputs equal the
// reduction followed by that kernel bit for bit, without writing and re-reading y between them.
__global__ __launch_bounds__(256) void split_reduce_norm_kernel(const float* part, int splits,
                                                                int M, uint16_t* y, int ldy,
                                                                const uint16_t* w,
                                                                uint16_t* out) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t plane = (size_t)M * kHidden;
  uint4 v[2], wv[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int n = (tid + 256 * k) * 8;
    float4 a, b;
    split_sum8(part + (size_t)m * kHidden + n, plane, splits, a, b);
    const uint4 o = make_uint4(pack_bf2(a.x, a.y), pack_bf2(a.z, a.w), pack_bf2(b.x, b.y),
                               pack_bf2(b.z, b.w));
    uint16_t* dst = y + (size_t)m * ldy + n;
    const uint4 r = *reinterpret_cast<const uint4*>(dst);
    v[k] = make_uint4(pack_bf2(bf_lo(r.x) + bf_lo(o.x), bf_hi(r.x) + bf_hi(o.x)),
                      pack_bf2(bf_lo(r.y) + bf_lo(o.y), bf_hi(r.y) + bf_hi(o.y)),
                      pack_bf2(bf_lo(r.z) + bf_lo(o.z), bf_hi(r.z) + bf_hi(o.z)),
                      pack_bf2(bf_lo(r.w) + bf_lo(o.w), bf_hi(r.w) + bf_hi(o.w)));
    *reinterpret_cast<uint4*>(dst) = v[k];
    wv[k] = reinterpret_cast<const uint4*>(w)[tid + 256 * k];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ss = fmaf(bf_lo(e[q]), bf_lo(e[q]), ss);
      ss = fmaf(bf_hi(e[q]), bf_hi(e[q]), ss);
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float rr = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)kHidden + kRmsEps);
  uint4* o4 = reinterpret_cast<uint4*>(out + (size_t)m * kHidden);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
    const uint32_t f[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = bf2f(f2bf(bf_lo(e[q]) * rr)) * bf_lo(f[q]);
      const float hi = bf2f(f2bf(bf_hi(e[q]) * rr)) * bf_hi(f[q]);
      o[q] = pack_bf2(lo, hi);
    }
    o4[tid + 256 * k] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// The QKV reduction with RoPE and the K/V scatter (prefill, kGemmQkvRope): each thread sums 4
// RoPE pairs of one row (dims j..j+3 and j+64..j+67 of one head of [q|k|v]) over the split
// planes in plane order, rounds to bf16 (the bf16 reduction's values), rotates q and k with the
// scatter kernel's arithmetic at position start_pos + m, and stores q to y [M][32][128], k and v
// to the cache (or its pages).
__global__ __launch_bounds__(256) void split_reduce_rope_kernel(const float* part, int splits,
                                                                GemmParams p) {
  constexpr int kQuads = (kQHeads + 2 * kKVHeads) * 16;  // 4-pair groups per row
  const size_t plane = (size_t)p.M * kQKVDim;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < (size_t)p.M * kQuads;
       i += (size_t)gridDim.x * blockDim.x) {
    const int m = (int)(i / kQuads), qd = (int)(i % kQuads);
    const int head = qd >> 4, j = (qd & 15) * 4;
    const float* src = part + (size_t)m * kQKVDim + head * kHeadDim + j;
    float4 a = *reinterpret_cast<const float4*>(src);
    float4 b = *reinterpret_cast<const float4*>(src + 64);
    for (int sp = 1; sp < splits; ++sp) {
      const float4 c = *reinterpret_cast<const float4*>(src + sp * plane);
      const float4 d = *reinterpret_cast<const float4*>(src + sp * plane + 64);
      a.x += c.x, a.y += c.y, a.z += c.z, a.w += c.w;
      b.x += d.x, b.y += d.y, b.z += d.z, b.w += d.w;
    }
    const float av[4] = {bf2f(f2bf(a.x)), bf2f(f2bf(a.y)), bf2f(f2bf(a.z)), bf2f(f2bf(a.w))};
    const float bv[4] = {bf2f(f2bf(b.x)), bf2f(f2bf(b.y)), bf2f(f2bf(b.z)), bf2f(f2bf(b.w))};
    const int pos = p.start_pos + m;
    float lo[4], hi[4];
    if (head < kQHeads + kKVHeads) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float c = p.rope_cos[(size_t)pos * 64 + j + e], sn = p.rope_sin[(size_t)pos * 64 + j + e];
        lo[e] = rope_lo(av[e], bv[e], c, sn);
        hi[e] = rope_hi(av[e], bv[e], c, sn);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) lo[e] = av[e], hi[e] = bv[e];
    }
    uint16_t* dst;
    if (head < kQHeads) {
      dst = p.y + ((size_t)m * kQHeads + head) * kHeadDim;
    } else {
      const bool is_k = head < kQHeads + kKVHeads;
      const int kvh = head - kQHeads - (is_k ? 0 : kKVHeads);
      uint16_t* const plane_kv = is_k ? p.k_cache : p.v_cache;
      if (p.block_table) {  // paged: row pos % kPagePos of the page holding block pos / kPagePos
        const int page = p.block_table[pos / kPagePos];
        if (page < 0 || page >= p.n_pages) continue;
        dst = plane_kv + (size_t)page * kPageElems + ((size_t)kvh * kPagePos + pos % kPagePos) * kHeadDim;
      } else {
        dst = plane_kv + ((size_t)kvh * kMaxCtx + pos) * kHeadDim;
      }
    }
    *reinterpret_cast<uint2*>(dst + j) = make_uint2(pack_bf2(lo[0], lo[1]), pack_bf2(lo[2], lo[3]));
    *reinterpret_cast<uint2*>(dst + j + 64) = make_uint2(pack_bf2(hi[0], hi[1]), pack_bf2(hi[2], hi[3]));
  }
}

// Split K when the best tiling is a single round that leaves at least half the chip idle, or
// one of 128 x 128 tiles: the wide kernel's tiles times the largest K split that divides the
// k-steps, fits one round of 256 workgroups and whose partials fit p.split_ws (at least 2),
// fp32 partials into p.split_ws, then the reduction.  Returns
// IE_OK after launching, 1 when split K does not apply.
// The reduction of a split product: p.split_ws holds `splits` fp32 planes of M x NP (NP = 2N
// for SwiGLU: gate then up), y = epilogue(sum) -- RoPE and the K/V scatter, residual + RMSNorm
// (p.rn_out), residual, SwiGLU or bf16.
int launch_split_reduce(int epi, const GemmParams& p, int splits, hipStream_t st) {
  const bool sw = epi == kGemmSwiglu, rope = epi == kGemmQkvRope;
  const size_t total = (size_t)p.M * p.N / 8;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 2048);
  if (sw) {
    hipLaunchKernelGGL(split_reduce_kernel<kGemmSwiglu>, dim3(blocks), dim3(256), 0, st,
                       p.split_ws, splits, p.M, p.N, p.y, p.ldy);
  } else if (rope) {
    const size_t items = (size_t)p.M * (kQHeads + 2 * kKVHeads) * 16;
    hipLaunchKernelGGL(split_reduce_rope_kernel, dim3((unsigned)std::min<size_t>((items + 255) / 256, 2048)),
                       dim3(256), 0, st, p.split_ws, splits, p);
  } else if (epi == kGemmResid && p.rn_out) {
    hipLaunchKernelGGL(split_reduce_norm_kernel, dim3(p.M), dim3(256), 0, st, p.split_ws, splits,
                       p.M, p.y, p.ldy, p.rn_w, p.rn_out);
    if (p.rn_done) *p.rn_done = 1;
  } else if (epi == kGemmResid) {
    hipLaunchKernelGGL(split_reduce_kernel<kGemmResid>, dim3(blocks), dim3(256), 0, st,
                       p.split_ws, splits, p.M, p.N, p.y, p.ldy);
  } else {
    hipLaunchKernelGGL(split_reduce_kernel<kGemmBf16>, dim3(blocks), dim3(256), 0, st,
                       p.split_ws, splits, p.M, p.N, p.y, p.ldy);
  }
  IE_CHECK_LAUNCH();
  return IE_OK;
}

int launch_split(int epi, const GemmParams& p, hipStream_t st) {
  // (below kWideMinRows too: a 128-row tile half empty still beats a few 128 x 128 tiles)
  if (!p.split_ws || epi == kGemmF32 || p.M > kSplitMaxRows || p.N % 8 != 0 || p.ldy % 8 != 0)
    return 1;
  const bool sw = epi == kGemmSwiglu;
  const bool rope = epi == kGemmQkvRope;
  const int te = rope ? kGemmBf16 : epi;  // the tiling of the plain product
  if (sw && p.N % 16 != 0) return 1;
  int best = kTileSmall;
  for (int k = kTileWide; k < kTileKinds; ++k)
    if (tile_ok(k, te, p) && tile_cost(k, te, p.M, p.N) < tile_cost(best, te, p.M, p.N)) best = k;
  // a single round that leaves half the chip idle, or one of 128 x 128 tiles (the older,
  // slower kernel)
  const long long best_tiles = tile_count(best, te, p.M, p.N);
  if (best_tiles > 256 || (best_tiles > 128 && best != kTileSmall)) return 1;
  // SwiGLU: one fp32 product over the gate rows then the up rows (2N columns)
  const int NP = sw ? 2 * p.N : p.N;
  const long long tiles = tile_count(kTileWide, kGemmF32, p.M, NP);
  const int kt = p.K / 64;
  const size_t plane = (size_t)p.M * NP * sizeof(float);
  int splits = 1;
  for (int s = 2; s <= 16; ++s)
    if (kt % s == 0 && tiles * s <= 256 && (size_t)s * plane <= (size_t)p.split_ws_bytes) splits = s;
  if (splits < 2) return 1;
  GemmParams q = p;
  q.yf = p.split_ws;
  q.ldy = NP;
  q.k_splits = splits;
  if (sw) {
    q.N = NP;
    q.n0 = p.N;  // rows [0, N) of w0 (gate), then [N, 2N) of w1 (up)
    q.n1 = p.N;
    q.w2 = p.w1;
  }
  const int rc = launch_wide<kGemmF32, 128, 64, 3, 1, 256, 2>(q, st);
  if (rc != IE_OK) return rc;
  return launch_split_reduce(epi, p, splits, st);
}

// Medium M (16 < M <= 128, K a multiple of 64): the 64-W-row streaming kernel, with its fp32
// partials reduced by the split reductions, or (gate/up and products of many tiles) unsplit
// with the epilogue in the kernel.  1: not applicable.
int launch_mid(int epi, const GemmParams& p, hipStream_t st) {
  if (g_gemm_schedule < 2 || p.M <= 16 || p.M > 128 || p.K % 64 != 0 || p.K < 64 ||
      p.N % 8 != 0 || p.ldy % 8 != 0 || epi == kGemmF32)
    return 1;
  const bool sw = epi == kGemmSwiglu, rope = epi == kGemmQkvRope;
  const int kt = p.K / 64;
  const bool x128 = p.M > 64;
  // 65-128 rows: SwiGLU over 64-column tiles (128 W rows, 8 waves: each tile re-reads the X
  // rows from L2 for twice the weight rows), when they alone fill most of the chip (in situ at
  // 100 and 128 rows 2.6% and 3.7% faster per prefill than 32-column tiles; at 64 rows and
  // fewer, level or slower)
  if (sw && x128 && p.N % 64 == 0 && p.N / 64 >= 192) {
    const int n_tiles = p.N / 64;
    GemmParams q = p;
    q.k_splits = 1;
    hipLaunchKernelGGL((wide::mid::gemm_mid_kernel<kGemmSwiglu, 128, 128>), dim3(n_tiles), dim3(512), 0,
                       st, q, n_tiles);
    IE_CHECK_LAUNCH();
    return IE_OK;
  }
  // unsplit: SwiGLU over 32-column tiles, bf16 / residual over 64-column tiles, once the tiles
  // alone fill most of the chip
  if (!rope && !p.rn_out && (sw ? p.N / 32 : (p.N + 63) / 64) >= 192 && (!sw || p.N % 32 == 0)) {
    const int n_tiles = sw ? p.N / 32 : (p.N + 63) / 64;
    GemmParams q = p;
    q.k_splits = 1;
#define IE_MID(E, XR, G) \
  hipLaunchKernelGGL((wide::mid::gemm_mid_kernel<E, XR, 64>), dim3(G), dim3(256), 0, st, q, n_tiles)
    switch (epi) {
      case kGemmSwiglu: if (x128) IE_MID(kGemmSwiglu, 128, n_tiles); else IE_MID(kGemmSwiglu, 64, n_tiles); break;
      case kGemmResid: if (x128) IE_MID(kGemmResid, 128, n_tiles); else IE_MID(kGemmResid, 64, n_tiles); break;
      default: if (x128) IE_MID(kGemmBf16, 128, n_tiles); else IE_MID(kGemmBf16, 64, n_tiles); break;
    }
    IE_CHECK_LAUNCH();
    return IE_OK;
  }
  if (!p.split_ws) return 1;
  // split K over fp32 planes of NP columns (SwiGLU: gate rows then up rows)
  const int NP = sw ? 2 * p.N : p.N;
  const int n_tiles = (NP + 63) / 64;
  const size_t plane = (size_t)p.M * NP * sizeof(float);
  int splits = 1;
  for (int sp = 2; sp <= 16; ++sp)
    if (kt % sp == 0 && (long long)n_tiles * sp <= 256 && (size_t)sp * plane <= (size_t)p.split_ws_bytes)
      splits = sp;
  if (splits < 2 && n_tiles < 128) return 1;
  GemmParams q = p;
  q.yf = p.split_ws;
  q.ldy = NP;
  q.k_splits = splits;
  if (sw) {
    q.N = NP;
    q.n0 = p.N;  // rows [0, N) of w0 (gate), then [N, 2N) of w1 (up)
    q.n1 = p.N;
    q.w2 = p.w1;
  }
  const unsigned blocks = (unsigned)(n_tiles * splits);
  if (x128) IE_MID(kGemmF32, 128, blocks);
  else IE_MID(kGemmF32, 64, blocks);
#undef IE_MID
  IE_CHECK_LAUNCH();
  return launch_split_reduce(epi, p, splits, st);
}

}  // namespace

int launch_gemm(int epi, const GemmParams& p, hipStream_t st) {
  IE_REQUIRE(p.M >= 1 && p.N >= 1 && p.K >= BK, "gemm: bad shape M=%d N=%d K=%d", p.M, p.N, p.K);
  IE_REQUIRE(p.K % BK == 0, "gemm: K=%d must be a multiple of %d", p.K, BK);
  IE_REQUIRE(p.N % 4 == 0, "gemm: N=%d must be a multiple of 4", p.N);
  IE_REQUIRE(p.ldy >= p.N, "gemm: ldy=%d < N=%d", p.ldy, p.N);
  // a 16-row load group must not straddle two weight matrices
  IE_REQUIRE(epi == kGemmSwiglu || ((p.n0 >= p.N || p.n0 % 16 == 0) &&
                                    (p.n0 + p.n1 >= p.N || (p.n0 + p.n1) % 16 == 0)),
             "gemm: weight split points n0=%d n0+n1=%d inside N=%d must be multiples of 16", p.n0,
             p.n0 + p.n1, p.N);
  if (gemm_skinny_fits(p)) return launch_gemm_skinny(epi, p, st);
  if (epi >= kGemmBf16 && epi <= kGemmSwiglu && !p.ss_in && !p.ss_out && p.k_splits <= 1) {
    const int rc = launch_mid(epi, p, st);
    if (rc != 1) return rc;
  }
  if (gemm_skinny_mb_fits(epi, p)) return launch_gemm_skinny_mb(epi, p, st);
  IE_REQUIRE(epi >= kGemmBf16 && epi <= kGemmSwiglu, "gemm: epilogue %d needs M <= 16", epi);
  IE_REQUIRE(!p.ss_in && !p.ss_out, "gemm: the folded RMSNorm needs M <= 16");
  IE_REQUIRE(p.k_splits <= 1, "gemm: k_splits is the launcher's");
  IE_REQUIRE(!p.rn_out || (epi == kGemmResid && p.N == kHidden && p.rn_w),
             "gemm: the fused RMSNorm output follows a residual product of %d columns", kHidden);
  const int rc = launch_split(epi, p, st);
  if (rc != 1) return rc;
  return launch_tiled(epi, p, st, true);
}

}  // namespace ie

namespace ie {

int launch_qkv_rope_prefill(const GemmParams& p, hipStream_t st) {
  IE_REQUIRE(p.N == kQKVDim && p.K == kHidden && p.n0 == kHidden && p.n1 == kKVDim && p.y &&
                 p.k_cache && p.v_cache && p.rope_cos && p.rope_sin && !p.d_seq_len &&
                 p.start_pos >= 0,
             "qkv_rope_prefill: the [q|k|v] projection of one sequence");
  if (g_gemm_schedule < 1 || gemm_skinny_fits(p)) return 1;
  {
    const int rc = launch_mid(kGemmQkvRope, p, st);
    if (rc != 1) return rc;
  }
  if (gemm_skinny_mb_fits(kGemmBf16, p)) return 1;
  // up to kSplitMaxRows rows: K split with the RoPE / scatter reduction where the bf16 product
  // would split
  if (p.M <= kSplitMaxRows) return launch_split(kGemmQkvRope, p, st);
  // above: the bf16 product's own choice (launch_gemm): the 192 x 256 tile in whole rounds
  int best = kTileSmall;
  for (int k = kTileWide; k < kTileKinds; ++k)
    if (tile_ok(k, kGemmBf16, p) &&
        tile_cost(k, kGemmBf16, p.M, p.N) < tile_cost(best, kGemmBf16, p.M, p.N))
      best = k;
  const long long tiles = tile_count(kTileBig192, kGemmBf16, p.M, p.N);
  if (best != kTileBig192 || (tiles > 256 && tiles % 256 != 0)) return 1;
  if (g_gemm_schedule == 3) return launch_pp<kGemmQkvRope, 192, 256, 4>(p, st);
  return launch_pp<kGemmQkvRope, 192, 256>(p, st);
}

}  // namespace ie

extern "C" int ie_tune_gemm_schedule(int schedule) {
  IE_REQUIRE(schedule >= 0 && schedule <= 3, "tune_gemm_schedule: %d not in [0, 3]", schedule);
  ie::g_gemm_schedule = schedule;
  return IE_OK;
}
