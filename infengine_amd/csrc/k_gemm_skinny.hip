// Skinny MFMA GEMM for batched decode (M <= 16 rows):
//   Y[M, N] = X[M, K] . W[N, K]^T      (fp32 accumulate)
//
// Reference: multiply_by_weight (kernels/ffn.cu:7-33) with m = batch rows.  At m <= 16 the
// product is HBM-bound on W exactly like the m = 1 GEMV, so the kernel is built for streaming:
// a workgroup owns 16 weight rows (output columns) and its 4 waves split K in quarters; each
// wave runs v_mfma_f32_16x16x32_bf16 with the 16 weight rows as A and the (up to) 16 X rows
// as B, and the quarters are summed through LDS.  Grid = N / 16 workgroups (256 for N = 4096,
// 8016 for the lm_head), enough to fill the chip where a 128-row tile GEMM had 32.
//
// Load pattern: a step covers 128 k as 4 MFMA k-chunks of 32; for chunk c lane l (row l % 16,
// group q = l / 16) loads the 16 bytes at k = 32c + 8q of its W row and of its X row (the
// MFMA operand layout), so each load instruction reads 64 contiguous bytes of 16 rows and a
// step streams 256 contiguous bytes of every weight row.  D = W . X^T: lane l holds output
// row m = l % 16 and 4 consecutive output columns n = 4 (l / 16) + i.
//
// Epilogues as the MFMA GEMM: bf16, residual add, fp32, and SwiGLU (gate and up rows of the
// same 16 columns in one workgroup, lane-local silu(bf16(g)) * bf16(u)).
#include "ie_kernels.h"

namespace ie {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSkRows = 16;   // weight rows (output columns) per workgroup
constexpr int kSkSplit = 4;   // waves per workgroup = K quarters
constexpr int kSkStep = 128;  // k per step

__device__ __forceinline__ const uint16_t* skinny_w_row(const GemmParams& p, int R) {
  if (R >= p.N) R = p.N - 1;
  const int e0 = min(p.n0, p.N), e1 = min(p.n0 + p.n1, p.N);
  if (R < e0) return p.w0 + (size_t)R * p.K;
  if (R < e1) return p.w1 + (size_t)(R - e0) * p.K;
  return p.w2 + (size_t)(R - e1) * p.K;
}

// the 4 chunks of one step: 16 bytes every 64 bytes from src (= row + k0 + 8q)
__device__ __forceinline__ void load_step(const uint16_t* src, u32x4_t (&v)[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) v[c] = *reinterpret_cast<const u32x4_t*>(src + 32 * c);
}

template <int EPI>
__global__ __launch_bounds__(kSkSplit * 64) void gemm_skinny_kernel(GemmParams p) {
  constexpr bool SW = EPI == kGemmSwiglu;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * kSkRows;

  const uint16_t *wa, *wb = nullptr;
  if constexpr (SW) {
    const int col = min(n0 + r, p.N - 1);
    wa = p.w0 + (size_t)col * p.K;  // gate
    wb = p.w1 + (size_t)col * p.K;  // up
  } else {
    wa = skinny_w_row(p, n0 + r);
  }
  const uint16_t* xr = p.x + (size_t)min(r, p.M - 1) * p.K;
  const int kq = p.K / kSkSplit;
  const int kbase = wave * kq + 8 * q;
  const int steps = kq / kSkStep;

  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  u32x4_t ca[4], cb[4], cx[4], na[4], nb[4], nx[4];
  load_step(wa + kbase, ca);
  if constexpr (SW) load_step(wb + kbase, cb);
  load_step(xr + kbase, cx);
  for (int s = 0; s < steps; ++s) {
    if (s + 1 < steps) {
      const int k = kbase + (s + 1) * kSkStep;
      load_step(wa + k, na);
      if constexpr (SW) load_step(wb + k, nb);
      load_step(xr + k, nx);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8_t xb = __builtin_bit_cast(bf16x8_t, cx[c]);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ca[c]), xb, acc0,
                                                     0, 0, 0);
      if constexpr (SW)
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, cb[c]), xb,
                                                       acc1, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ca[c] = na[c];
      cx[c] = nx[c];
      if constexpr (SW) cb[c] = nb[c];
    }
  }

  // sum the K quarters: waves 1..3 hand their tiles to wave 0
  __shared__ f32x4_t red[kSkSplit][SW ? 2 : 1][64];
  red[wave][0][lane] = acc0;
  if constexpr (SW) red[wave][SW ? 1 : 0][lane] = acc1;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kSkSplit; ++w) {
    acc0 += red[w][0][lane];
    if constexpr (SW) acc1 += red[w][SW ? 1 : 0][lane];
  }

  const int m = r, n = n0 + 4 * q;
  if (m >= p.M || n >= p.N) return;
  if constexpr (EPI == kGemmF32) {
    *reinterpret_cast<float4*>(p.yf + (size_t)m * p.ldy + n) =
        make_float4(acc0[0], acc0[1], acc0[2], acc0[3]);
  } else if constexpr (EPI == kGemmResid) {
    uint2* dst = reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n);
    const uint2 old = *dst;
    *dst = make_uint2(
        pack_bf2(bf_lo(old.x) + bf2f(f2bf(acc0[0])), bf_hi(old.x) + bf2f(f2bf(acc0[1]))),
        pack_bf2(bf_lo(old.y) + bf2f(f2bf(acc0[2])), bf_hi(old.y) + bf2f(f2bf(acc0[3]))));
  } else if constexpr (SW) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float g = bf2f(f2bf(acc0[i])), u = bf2f(f2bf(acc1[i]));
      v[i] = g * (1.0f / (1.0f + expf(-g))) * u;
    }
    *reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n) =
        make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
  } else {
    *reinterpret_cast<uint2*>(p.y + (size_t)m * p.ldy + n) =
        make_uint2(pack_bf2(acc0[0], acc0[1]), pack_bf2(acc0[2], acc0[3]));
  }
}

template <int EPI>
int launch_s(const GemmParams& p, hipStream_t st) {
  const int blocks = (p.N + kSkRows - 1) / kSkRows;
  hipLaunchKernelGGL((gemm_skinny_kernel<EPI>), dim3(blocks), dim3(kSkSplit * 64), 0, st, p);
  IE_CHECK_LAUNCH();
  return IE_OK;
}

}  // namespace

bool gemm_skinny_fits(const GemmParams& p) {
  return p.M >= 1 && p.M <= kSkRows && p.K % (kSkSplit * kSkStep) == 0;
}

int launch_gemm_skinny(int epi, const GemmParams& p, hipStream_t st) {
  IE_REQUIRE(gemm_skinny_fits(p), "gemm_skinny: needs M <= %d and K %% %d == 0 (M=%d K=%d)",
             kSkRows, kSkSplit * kSkStep, p.M, p.K);
  switch (epi) {
    case kGemmBf16: return launch_s<kGemmBf16>(p, st);
    case kGemmResid: return launch_s<kGemmResid>(p, st);
    case kGemmF32: return launch_s<kGemmF32>(p, st);
    case kGemmSwiglu: return launch_s<kGemmSwiglu>(p, st);
  }
  set_error("gemm_skinny: bad epilogue %d", epi);
  return IE_ERR_INVALID_ARG;
}

}  // namespace ie
