// MFMA bf16 GEMM for prefill (and any multi-row multiply_by_weight):
//   Y[M, N] = X[M, K] . W[N, K]^T      (X, W row-major, K contiguous; fp32 accumulate)
//
// Reference: every prefill matmul is cublasGemmEx / cublasGemmStridedBatchedEx
// with fp32 compute (kernels/ffn.cu:7-33, kernels/attn.cu:12-39, 265-293).
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
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128;  // X rows per tile
constexpr int BN = 128;  // W rows per tile
constexpr int BK = 64;

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

}  // namespace

int launch_gemm(int epi, const GemmParams& p, hipStream_t st) {
  IE_REQUIRE(p.M >= 1 && p.N >= 1 && p.K >= BK, "gemm: bad shape M=%d N=%d K=%d", p.M, p.N, p.K);
  IE_REQUIRE(p.K % BK == 0, "gemm: K=%d must be a multiple of %d", p.K, BK);
  IE_REQUIRE(p.N % 4 == 0, "gemm: N=%d must be a multiple of 4", p.N);
  IE_REQUIRE(p.ldy >= p.N, "gemm: ldy=%d < N=%d", p.ldy, p.N);
  switch (epi) {
    case kGemmBf16: return launch_e<kGemmBf16>(p, st);
    case kGemmResid: return launch_e<kGemmResid>(p, st);
    case kGemmF32: return launch_e<kGemmF32>(p, st);
    case kGemmSwiglu: return launch_e<kGemmSwiglu>(p, st);
  }
  set_error("gemm: bad epilogue %d", epi);
  return IE_ERR_INVALID_ARG;
}

}  // namespace ie
