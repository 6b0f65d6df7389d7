// CPU ORACLE — TEST INFRASTRUCTURE ONLY.
//
// A plain C++ (OpenMP) restatement of the reference's per-token Llama-3.1-8B
// math, used only by tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg as the checker.  The product path (infengine_amd) never
// links, loads or calls anything here.
//
// Storage is bf16 (uint16_t bit patterns), accumulation fp32, logits fp32.
// Rounding points are the reference's (each kernel rounds its output to the
// storage type); the build keeps bf16 where the reference converted to fp16
// (model_weights.cu:61-78).  Every function names the reference code it follows.
// Compiled with -ffp-contract=off so no a*b+c is fused behind the code's back.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <numbers>
#include <vector>

namespace {

constexpr int kHidden = 4096, kFFN = 14336, kQHeads = 32, kKVHeads = 8, kHeadDim = 128;
constexpr int kMaxCtx = 8192, kGQA = kQHeads / kKVHeads;
constexpr float kEps = 1e-5f;  // rmsnorm.cu:5

inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint16_t f2bf(float f) {  // round to nearest even; NaN stays (quiet) NaN
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

inline uint64_t synth_base(uint64_t seed, uint64_t tensor_id) {
  return splitmix64(splitmix64(seed) ^ (tensor_id * 0xD1B54A32D192ED03ull));
}

constexpr double kSynthStd = 37837.22627754049;  // sqrt(4 * (65536^2 - 1) / 12)

// Summation order of every fp32 dot product: 0 = ascending k, 1 = descending k.
// Both are valid fp32 accumulations; running the oracle both ways measures the
// rounding-noise floor that any fp32-accumulating implementation sits inside.
int g_sum_reverse = 0;

// Rounding point of the attention probabilities before P.V (orc_set_prob_round):
//   0  fp32 throughout: out = bf16(sum_t p_t v_t), p = softmax in fp32 (the exact math);
//   1  the reference's point: the softmax kernel stores the normalised probabilities in the
//      storage type (softmax.cu:105,158) and the A.V GEMM multiplies those
//      (attn.cu:167-204): p_t = bf16(exp(s_t - max) / sum), out = bf16(sum_t p_t v_t);
//   2  the flash form: keys in 64-key tiles from key 0, a running max m of the raw scores,
//      p_t = bf16(exp2((s_t - m) c)) with c = log2(e)/sqrt(128), o and the row sum l of the
//      rounded p rescaled by exp2((m_old - m_new) c) when m grows, out = bf16(o * (1 / l)):
//      the rounding the MFMA prefill attention applies (its P.V operand is bf16).
int g_prob_round = 0;

// fp32 dot product of two bf16 vectors, 8 running partial sums.
inline float dot_bf16(const uint16_t* a, const uint16_t* b, int k) {
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float t;
  if (!g_sum_reverse) {
    int i = 0;
    for (; i + 8 <= k; i += 8)
      for (int j = 0; j < 8; ++j) s[j] += bf2f(a[i + j]) * bf2f(b[i + j]);
    t = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    for (; i < k; ++i) t += bf2f(a[i]) * bf2f(b[i]);
  } else {
    int i = k;
    for (; i - 8 >= 0; i -= 8)
      for (int j = 0; j < 8; ++j) s[j] += bf2f(a[i - 1 - j]) * bf2f(b[i - 1 - j]);
    t = ((s[7] + s[6]) + (s[5] + s[4])) + ((s[3] + s[2]) + (s[1] + s[0]));
    for (; i > 0; --i) t += bf2f(a[i - 1]) * bf2f(b[i - 1]);
  }
  return t;
}

inline float silu_mul(float g, float u) {  // swiglu.cu:24-29
  return g * (1.0f / (1.0f + std::exp(-g))) * u;
}

}  // namespace

extern "C" {

void orc_set_sum_order(int reverse) { g_sum_reverse = reverse ? 1 : 0; }
void orc_set_prob_round(int mode) { g_prob_round = mode < 0 || mode > 2 ? 0 : mode; }

// ---------------------------------------------------------------- synthetic data
// Deterministic approximate normal keyed by (seed, tensor_id, index): centred
// sum of the four 16-bit fields of splitmix64(base + index) (Irwin-Hall n=4),
// scaled with one correctly-rounded fma and rounded to bf16.  Integer-exact up to
// that fma, so the GPU generator reproduces it bit for bit.
void orc_fill_synthetic(uint16_t* out, size_t n, uint64_t seed, uint64_t tensor_id, float mean,
                        float std) {
  const uint64_t base = synth_base(seed, tensor_id);
  const float scale = (float)((double)std / kSynthStd);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) {
    const uint64_t h = splitmix64(base + i);
    const int s = (int)(h & 0xFFFF) + (int)((h >> 16) & 0xFFFF) + (int)((h >> 32) & 0xFFFF) +
                  (int)(h >> 48);
    out[i] = f2bf(std::fma((float)(s - 131070), scale, mean));
  }
}

// Tensor ids of the synthetic model: emb 1, final_norm 2, lm_head 3,
// layer l field f -> 16 + 16 l + f with f = 0 input_layernorm, 1 w_q, 2 w_k,
// 3 w_v, 4 w_o, 5 post_attention_layernorm, 6 w_gate, 7 w_up, 8 w_down.
uint64_t orc_tensor_id(int layer, int field) { return 16 + (uint64_t)layer * 16 + field; }

// ---------------------------------------------------------------- rope tables
// rope.cu:68-96 (init_rope_buffer): Llama-3 scaled inverse frequencies (theta
// 500000, factor 8, low 1, high 4, original context 8192; orc_rope_freqs) and fp32
// cos/sin of pos * freq for pos < n_pos, i < 64 (the reference stops at 8192; the same
// formula continues for long contexts).  Same arithmetic types as the reference.
void orc_rope_freqs(float* freqs) {
  const float theta = 500000.0f;
  const int factor = 8, low_ff = 1, high_ff = 4, orig = 8192;
  const int low_wl = orig / low_ff, high_wl = orig / high_ff;
  for (int i = 0; i < 64; ++i) {
    const float freq = 1 / std::pow(theta, 2.0 * i / kHeadDim);
    const float wavelength = 2 * std::numbers::pi / freq;
    if (wavelength > low_wl) {
      freqs[i] = freq / factor;
    } else if (wavelength < high_wl) {
      freqs[i] = freq;
    } else {
      const float smooth = (orig / wavelength - low_ff) / (high_ff - low_ff);
      freqs[i] = (1 - smooth) * (freq / factor) + smooth * freq;
    }
  }
}

void orc_rope_tables(int n_pos, float* cos_t, float* sin_t) {
  float freqs[64];
  orc_rope_freqs(freqs);
#pragma omp parallel for schedule(static)
  for (int pos = 0; pos < n_pos; ++pos)
    for (int i = 0; i < 64; ++i) {
      const float angle = pos * freqs[i];
      cos_t[(size_t)pos * 64 + i] = std::cos(angle);
      sin_t[(size_t)pos * 64 + i] = std::sin(angle);
    }
}

// ---------------------------------------------------------------- elementwise
// emblookup.cu:19-24: out[t] = E[ids[t]]  (bit-exact copy)
void orc_emblookup(int rows, const int* ids, const uint16_t* table, uint16_t* out) {
  for (int t = 0; t < rows; ++t)
    std::memcpy(out + (size_t)t * kHidden, table + (size_t)ids[t] * kHidden, kHidden * 2);
}

// rmsnorm.cu:44-61: fp32 sum of squares over the row, r = 1/sqrt(mean + 1e-5),
// out = bf16(bf16(x * r) * w)  (the half-precision multiply by w at :61).
void orc_rmsnorm(int rows, int cols, const uint16_t* x, const uint16_t* w, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + (size_t)r * cols;
    float ss = 0.f;
    for (int i = 0; i < cols; ++i) ss += bf2f(xr[i]) * bf2f(xr[i]);
    const float inv = 1.0f / std::sqrt(ss / (float)cols + kEps);
    uint16_t* o = out + (size_t)r * cols;
    for (int i = 0; i < cols; ++i) o[i] = f2bf(bf2f(f2bf(bf2f(xr[i]) * inv)) * bf2f(w[i]));
  }
}

// residual_add.cu:17-19: x += delta, rounded to the storage type
void orc_residual_add(size_t n, uint16_t* x, const uint16_t* d) {
  for (size_t i = 0; i < n; ++i) x[i] = f2bf(bf2f(x[i]) + bf2f(d[i]));
}

// swiglu.cu:24-29: out = g * sigmoid(g) * u in fp32, rounded
void orc_swiglu(size_t n, const uint16_t* g, const uint16_t* u, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = f2bf(silu_mul(bf2f(g[i]), bf2f(u[i])));
}

// ---------------------------------------------------------------- matmul
// ffn.cu:7-33 (multiply_by_weight): Y[m, n] = X[m, k] . W[n, k]^T, fp32
// accumulation, output rounded to the storage type (bf16) or kept fp32.
void orc_matmul_bf16(int m, int k, int n, const uint16_t* x, const uint16_t* w, uint16_t* y) {
#pragma omp parallel for schedule(static) collapse(2)
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j)
      y[(size_t)i * n + j] = f2bf(dot_bf16(x + (size_t)i * k, w + (size_t)j * k, k));
}

void orc_matmul_f32(int m, int k, int n, const uint16_t* x, const uint16_t* w, float* y) {
#pragma omp parallel for schedule(static) collapse(2)
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) y[(size_t)i * n + j] = dot_bf16(x + (size_t)i * k, w + (size_t)j * k, k);
}

// ---------------------------------------------------------------- rope
// rope.cu:30-66 (apply_rope_kern): for each head and token, rotate the pair
// (x_j, x_{j+64}) by angle table[start_pos + t][j] in fp32 (rotate-half pairing
// of rope.cu:59-64, i.e. HF apply_rotary_pos_emb), round to the storage type.
// Heads are head_rows rows apart (seq_len for activations, 8192 for the cache).
void orc_apply_rope(int start_pos, int heads, int seq_len, int head_rows, const float* cos_t,
                    const float* sin_t, const uint16_t* in, uint16_t* out) {
  for (int h = 0; h < heads; ++h)
    for (int t = 0; t < seq_len; ++t) {
      const size_t off = ((size_t)h * head_rows + t) * kHeadDim;
      const int pos = start_pos + t;
      for (int j = 0; j < 64; ++j) {
        const float c = cos_t[(size_t)pos * 64 + j], s = sin_t[(size_t)pos * 64 + j];
        const float a = bf2f(in[off + j]), b = bf2f(in[off + j + 64]);
        // one rounding over the second product, as nvcc contracts rope.cu:63-64 by default
        out[off + j] = f2bf(std::fma(a, c, -(b * s)));
        out[off + j + 64] = f2bf(std::fma(a, s, b * c));
      }
    }
}

// ---------------------------------------------------------------- softmax
// softmax.cu:55-160: softmax(x / sqrt(128)) over each row of length `len`; with
// `causal`, row r of each [len, len] head block keeps entries 0..r (the others
// are written as 0).  fp32 math (the reference keeps max and exp in half; its
// golden generator, generate_test_data.py:58-76, uses fp32).
void orc_softmax_scaled(int rows, int len, int causal, const uint16_t* in, uint16_t* out) {
  const float scale = 0.08838834764831845f;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const int valid = causal ? (r % len) + 1 : len;
    const uint16_t* x = in + (size_t)r * len;
    uint16_t* y = out + (size_t)r * len;
    float mx = -INFINITY;
    for (int i = 0; i < valid; ++i) mx = std::max(mx, bf2f(x[i]) * scale);
    float sum = 0.f;
    for (int i = 0; i < valid; ++i) sum += std::exp(bf2f(x[i]) * scale - mx);
    for (int i = 0; i < len; ++i)
      y[i] = i < valid ? f2bf(std::exp(bf2f(x[i]) * scale - mx) / sum) : (uint16_t)0;
  }
}

// ---------------------------------------------------------------- attention
// attn.cu:355-363 (prefill) / :423-431 (decode): for q row i (absolute position
// q_start + i) and q head h, scores s_t = (q_h . k_{h/4, t}) / sqrt(128) for
// t = 0..q_start+i, p = softmax(s), out = sum_t p_t v_{h/4, t}, rounded to bf16,
// with p rounded as g_prob_round says (fp32 by default).  GQA mapping h -> h/4 is
// attn.cu:51-53 / HF repeat_kv.
// q: [n_q][32][128]; k/v planes: [8][ctx_stride][128]; out: [n_q][4096].
void orc_attention(int n_q, int q_start, const uint16_t* q, const uint16_t* kplane,
                   const uint16_t* vplane, int ctx_stride, uint16_t* out) {
  const float scale = 0.08838834764831845f;
  const float c2 = 0.08838834764831845f * 1.4426950408889634f;  // scale * log2(e)
  const int mode = g_prob_round;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int i = 0; i < n_q; ++i)
    for (int h = 0; h < kQHeads; ++h) {
      const int g = h / kGQA, S = q_start + i + 1;
      const uint16_t* qh = q + ((size_t)i * kQHeads + h) * kHeadDim;
      const uint16_t* K = kplane + (size_t)g * ctx_stride * kHeadDim;
      const uint16_t* V = vplane + (size_t)g * ctx_stride * kHeadDim;
      uint16_t* o = out + (size_t)i * kHidden + h * kHeadDim;
      std::vector<float> s(S);
      float acc[kHeadDim] = {};
      if (mode == 2) {
        for (int t = 0; t < S; ++t) s[t] = dot_bf16(qh, K + (size_t)t * kHeadDim, kHeadDim);
        float m = -INFINITY, l = 0.f;
        for (int t0 = 0; t0 < S; t0 += 64) {
          const int t1 = std::min(S, t0 + 64);
          float mt = -INFINITY;
          for (int t = t0; t < t1; ++t) mt = std::max(mt, s[t]);
          const float mn = std::max(m, mt);
          const float nb = -(mn * c2);
          const float alpha = m == -INFINITY ? 0.f : std::exp2(std::fma(m, c2, nb));
          l *= alpha;
          for (int d = 0; d < kHeadDim; ++d) acc[d] *= alpha;
          for (int t = t0; t < t1; ++t) {
            const float p = bf2f(f2bf(std::exp2(std::fma(s[t], c2, nb))));
            l += p;
            const uint16_t* vt = V + (size_t)t * kHeadDim;
            for (int d = 0; d < kHeadDim; ++d) acc[d] += p * bf2f(vt[d]);
          }
          m = mn;
        }
        const float inv = 1.0f / l;
        for (int d = 0; d < kHeadDim; ++d) o[d] = f2bf(acc[d] * inv);
        continue;
      }
      float mx = -INFINITY;
      for (int t = 0; t < S; ++t) {
        s[t] = dot_bf16(qh, K + (size_t)t * kHeadDim, kHeadDim) * scale;
        mx = std::max(mx, s[t]);
      }
      float sum = 0.f;
      for (int t = 0; t < S; ++t) {
        s[t] = std::exp(s[t] - mx);
        sum += s[t];
      }
      if (mode == 1) {
        for (int t = 0; t < S; ++t) {
          const float p = bf2f(f2bf(s[t] / sum));
          const uint16_t* vt = V + (size_t)t * kHeadDim;
          for (int d = 0; d < kHeadDim; ++d) acc[d] += p * bf2f(vt[d]);
        }
        for (int d = 0; d < kHeadDim; ++d) o[d] = f2bf(acc[d]);
        continue;
      }
      for (int t = 0; t < S; ++t) {
        const uint16_t* vt = V + (size_t)t * kHeadDim;
        for (int d = 0; d < kHeadDim; ++d) acc[d] += s[t] * bf2f(vt[d]);
      }
      for (int d = 0; d < kHeadDim; ++d) o[d] = f2bf(acc[d] / sum);
    }
}

// ---------------------------------------------------------------- decoder layer
// One Llama decoder layer over S rows at positions start_pos..start_pos+S-1, in
// the order of decode.cu:17-39 / prefill.cu:17-38 (= HF LlamaDecoderLayer):
//   xn = rmsnorm(x, ln1); q,k,v = bf16(W xn); rope(q,k); k,v -> cache rows;
//   a = attention; x = x + bf16(W_o a); xn = rmsnorm(x, ln2);
//   h = bf16(silu(bf16(W_g xn)) * bf16(W_u xn)); x = x + bf16(W_d h).
// kplane/vplane: [8][ctx_stride][128] of this layer (rows < start_pos already
// hold earlier positions).
void orc_decoder_layer(int S, int start_pos, uint16_t* x, const uint16_t* ln1,
                       const uint16_t* wq, const uint16_t* wk, const uint16_t* wv,
                       const uint16_t* wo, const uint16_t* ln2, const uint16_t* wg,
                       const uint16_t* wu, const uint16_t* wd, const float* cos_t,
                       const float* sin_t, uint16_t* kplane, uint16_t* vplane, int ctx_stride) {
  std::vector<uint16_t> xn((size_t)S * kHidden), q((size_t)S * kHidden),
      k((size_t)S * 1024), v((size_t)S * 1024), a((size_t)S * kHidden), o((size_t)S * kHidden);
  orc_rmsnorm(S, kHidden, x, ln1, xn.data());
  orc_matmul_bf16(S, kHidden, kHidden, xn.data(), wq, q.data());
  orc_matmul_bf16(S, kHidden, 1024, xn.data(), wk, k.data());
  orc_matmul_bf16(S, kHidden, 1024, xn.data(), wv, v.data());
  // [S][heads][128] -> rotate per (t, head): rows of one token are contiguous here
  std::vector<uint16_t> qr((size_t)S * kHidden), kr((size_t)S * 1024);
  for (int t = 0; t < S; ++t) {
    orc_apply_rope(start_pos + t, kQHeads, 1, 1, cos_t, sin_t, q.data() + (size_t)t * kHidden,
                   qr.data() + (size_t)t * kHidden);
    orc_apply_rope(start_pos + t, kKVHeads, 1, 1, cos_t, sin_t, k.data() + (size_t)t * 1024,
                   kr.data() + (size_t)t * 1024);
  }
  for (int t = 0; t < S; ++t)
    for (int g = 0; g < kKVHeads; ++g) {
      const size_t dst = ((size_t)g * ctx_stride + start_pos + t) * kHeadDim;
      std::memcpy(kplane + dst, kr.data() + (size_t)t * 1024 + g * kHeadDim, kHeadDim * 2);
      std::memcpy(vplane + dst, v.data() + (size_t)t * 1024 + g * kHeadDim, kHeadDim * 2);
    }
  orc_attention(S, start_pos, qr.data(), kplane, vplane, ctx_stride, a.data());
  orc_matmul_bf16(S, kHidden, kHidden, a.data(), wo, o.data());
  orc_residual_add((size_t)S * kHidden, x, o.data());
  orc_rmsnorm(S, kHidden, x, ln2, xn.data());
  std::vector<uint16_t> gg((size_t)S * kFFN), uu((size_t)S * kFFN), hh((size_t)S * kFFN);
  orc_matmul_bf16(S, kHidden, kFFN, xn.data(), wg, gg.data());
  orc_matmul_bf16(S, kHidden, kFFN, xn.data(), wu, uu.data());
  orc_swiglu((size_t)S * kFFN, gg.data(), uu.data(), hh.data());
  orc_matmul_bf16(S, kFFN, kHidden, hh.data(), wd, o.data());
  orc_residual_add((size_t)S * kHidden, x, o.data());
}

// ffn.cu:39-64: out = W_d (silu(W_g x) * W_u x), each product rounded to bf16
void orc_ffn(int S, const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
             const uint16_t* wd, uint16_t* out) {
  std::vector<uint16_t> gg((size_t)S * kFFN), uu((size_t)S * kFFN), hh((size_t)S * kFFN);
  orc_matmul_bf16(S, kHidden, kFFN, x, wg, gg.data());
  orc_matmul_bf16(S, kHidden, kFFN, x, wu, uu.data());
  orc_swiglu((size_t)S * kFFN, gg.data(), uu.data(), hh.data());
  orc_matmul_bf16(S, kFFN, kHidden, hh.data(), wd, out);
}

// ---------------------------------------------------------------- sampling
// Greedy argmax with torch.argmax semantics (the reference's own tie rule,
// sampling.cu:18-21,39-44, is layout-dependent and deliberately not followed):
// largest value, first index among ties, NaN beats everything, -0.0 == +0.0.
int orc_argmax(int n, const float* v) {
  int best = 0;
  for (int i = 0; i < n; ++i) {
    if (std::isnan(v[i])) return i;
    if (v[i] > v[best]) best = i;
  }
  return best;
}

// Temperature + top-p sampling, restated by sorting (the GPU uses a radix
// select; both must find the same kept set):
//   l_i = logit_i / T; e_i = exp(l_i - max l); q_i = floor(e_i * 2^40) (uint64)
//   target = max(1, floor(Z * p)), Z = sum q_i
//   kept = { i : mass of tokens with larger l is < target }  (HF TopPLogitsWarper)
//   t = floor(Z_kept * u), u = 24-bit counter uniform (seed, row, step)
//   token = smallest id with kept prefix mass (id order) > t.
// info (if non-null) receives {t, lo, hi, Z_kept} with [lo, hi) the winner's
// mass interval, so a caller can see how close t was to a boundary.
int orc_top_p(int vocab, const float* logits, float temperature, float top_p, uint64_t seed,
              int row, uint64_t step, double* info) {
  std::vector<float> l(vocab);
  float mx = -INFINITY;
  for (int i = 0; i < vocab; ++i) {
    l[i] = logits[i] / temperature;
    mx = std::max(mx, l[i]);
  }
  std::vector<uint64_t> q(vocab);
  uint64_t z = 0;
  for (int i = 0; i < vocab; ++i) {
    q[i] = (uint64_t)(std::exp(l[i] - mx) * 1099511627776.0f);
    z += q[i];
  }
  uint64_t target = (uint64_t)((double)z * (double)top_p);
  if (target < 1) target = 1;
  std::vector<int> idx(vocab);
  for (int i = 0; i < vocab; ++i) idx[i] = i;
  std::sort(idx.begin(), idx.end(), [&](int a, int b) { return l[a] > l[b]; });
  // walk groups of equal value in descending order
  float cut = l[idx[0]];
  uint64_t above = 0;
  for (int i = 0; i < vocab;) {
    int j = i;
    uint64_t grp = 0;
    while (j < vocab && l[idx[j]] == l[idx[i]]) grp += q[idx[j++]];
    cut = l[idx[i]];
    if (above + grp >= target) break;
    above += grp;
    i = j;
  }
  uint64_t zk = 0;
  for (int i = 0; i < vocab; ++i)
    if (l[i] >= cut) zk += q[i];
  const uint64_t bits = splitmix64(synth_base(seed, 0x70707070ull + (uint64_t)row) + step) >> 40;
  const uint64_t t = (zk >> 24) * bits + (((zk & 0xFFFFFFull) * bits) >> 24);
  uint64_t cum = 0;
  int tok = -1;
  for (int i = 0; i < vocab; ++i) {
    if (l[i] < cut) continue;
    if (cum + q[i] > t) {
      tok = i;
      break;
    }
    cum += q[i];
  }
  if (info) {
    info[0] = (double)t;
    info[1] = (double)cum;
    info[2] = tok >= 0 ? (double)(cum + q[tok]) : 0.0;
    info[3] = (double)zk;
  }
  return tok;
}

}  // extern "C"
