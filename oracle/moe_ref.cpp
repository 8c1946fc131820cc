// C++/OpenMP restatement of MLX's unpatched quantized MoE block on the CPU.
//
// TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py and a second,
// independently written implementation the numpy oracle (moe_oracle.py) is
// cross-checked against in tests/.  Never linked into the zmlx_amd library.
//
// Follows the same reference points as moe_oracle.py:
//   dequant            src/zmlx/kernels/quant.py:736-745 (element i at bits 4*i)
//   gather_qmm         MLX mx.gather_qmm (fp32 accumulation, bf16 result)
//   SwiGLU             nn.silu(g) * u  (tests/test_gather_qmm_swiglu.py:73)
//   Qwen gating        patch/patterns/moe_mlp.py:255-266
//   native combine     (y * w[..., None]).sum(-2)   moe_mlp.py:1043
// Accumulation is fp32 per group (s*sum(q*x) + b*sum(x), the factoring MLX's
// qmv kernels use), so results agree with the float64 oracle to within fp32
// rounding, not bit for bit.
//
// Built for x86-64-v3 (AVX2 + FMA): the nibbles of one packed word are
// unpacked into 8 int32 lanes with one variable shift and a mask, converted
// and multiplied into 8 activations with one FMA.  One OpenMP parallel region
// per token covers the router, the gate/up rows of all selected experts, the
// down rows and the combine (barriers between them), so the threads stay in
// one team for the whole token.
#include <immintrin.h>
#include <omp.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace {

inline float bf(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint16_t to_bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline float rbf(float f) { return bf(to_bf(f)); }

inline float hsum8(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
  lo = _mm_add_ps(lo, hi);
  lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
  lo = _mm_add_ss(lo, _mm_movehdup_ps(lo));
  return _mm_cvtss_f32(lo);
}

// One row of an affine 4-bit matrix against fp32 activations x[K] whose
// per-group sums are xg[K/gs]:  bf16( sum_g s_g * sum(q*x) + b_g * sum(x) ).
inline uint16_t qrow_affine(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x, const float* xg,
                            int K, int gs) {
  const __m256i shifts = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
  const __m256i mask = _mm256_set1_epi32(0xF);
  const int G = K / gs, wpg = gs / 8;
  float acc = 0.0f;
  for (int g = 0; g < G; ++g) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    const uint32_t* wg = w + g * wpg;
    const float* xp = x + g * gs;
    int j = 0;
    for (; j + 1 < wpg; j += 2) {
      const __m256i q0 = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32(static_cast<int>(wg[j])), shifts), mask);
      const __m256i q1 = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32(static_cast<int>(wg[j + 1])), shifts), mask);
      a0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(q0), _mm256_loadu_ps(xp + 8 * j), a0);
      a1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(q1), _mm256_loadu_ps(xp + 8 * j + 8), a1);
    }
    for (; j < wpg; ++j) {
      const __m256i q0 = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32(static_cast<int>(wg[j])), shifts), mask);
      a0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(q0), _mm256_loadu_ps(xp + 8 * j), a0);
    }
    const float qx = hsum8(_mm256_add_ps(a0, a1));
    acc += bf(s[g]) * qx + bf(b[g]) * xg[g];
  }
  return to_bf(acc);
}

// Dot of fp32 x[H] with one bf16 row.
inline float dot_bf16(const float* x, const uint16_t* r, int H) {
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  int h = 0;
  for (; h + 16 <= H; h += 16) {
    const __m256i v0 = _mm256_slli_epi32(_mm256_cvtepu16_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(r + h))), 16);
    const __m256i v1 =
        _mm256_slli_epi32(_mm256_cvtepu16_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(r + h + 8))), 16);
    a0 = _mm256_fmadd_ps(_mm256_castsi256_ps(v0), _mm256_loadu_ps(x + h), a0);
    a1 = _mm256_fmadd_ps(_mm256_castsi256_ps(v1), _mm256_loadu_ps(x + h + 8), a1);
  }
  float acc = hsum8(_mm256_add_ps(a0, a1));
  for (; h < H; ++h) acc += x[h] * bf(r[h]);
  return acc;
}

void group_sums(const float* x, int K, int gs, float* xg) {
  for (int g = 0; g < K / gs; ++g) {
    float s = 0.0f;
    for (int i = g * gs; i < (g + 1) * gs; ++i) s += x[i];
    xg[g] = s;
  }
}

}  // namespace

extern "C" {

int oref_num_threads(void) { return omp_get_max_threads(); }

void oref_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}

// Qwen3-style MoE block for B tokens (affine 4-bit, bf16 activations):
//   logits = bf16(x Wr^T); p = bf16(softmax(logits)); top-k by p (ties ->
//   lower index); w = bf16(p_k / bf16(sum p_k)) if norm; experts; native
//   combine.  All arrays row-major; bf16 passed as uint16.
void oref_moe_layer_qwen(const uint16_t* x, int B, int H, int E, int K, int I, int gs, int norm,
                         const uint16_t* wr, const uint32_t* gw, const uint16_t* gsc, const uint16_t* gb,
                         const uint32_t* uw, const uint16_t* usc, const uint16_t* ub, const uint32_t* dw,
                         const uint16_t* dsc, const uint16_t* db, uint16_t* out, int32_t* out_idx) {
  std::vector<float> xf(H), xg(H / gs), logit(E), p(E), act(static_cast<size_t>(K) * I), ag(static_cast<size_t>(K) * (I / gs)),
      wk(K);
  std::vector<uint16_t> y(static_cast<size_t>(K) * H);
  std::vector<int> sel(K);
  const int64_t gsz = static_cast<int64_t>(I) * (H / 8), gss = static_cast<int64_t>(I) * (H / gs);
  const int64_t dsz = static_cast<int64_t>(H) * (I / 8), dss = static_cast<int64_t>(H) * (I / gs);
  for (int t = 0; t < B; ++t) {
    for (int h = 0; h < H; ++h) xf[h] = bf(x[static_cast<int64_t>(t) * H + h]);
#pragma omp parallel
    {
#pragma omp for schedule(static)
      for (int e = 0; e < E; ++e) logit[e] = rbf(dot_bf16(xf.data(), wr + static_cast<int64_t>(e) * H, H));
#pragma omp single
      {
        group_sums(xf.data(), H, gs, xg.data());
        float m = -INFINITY;
        for (int e = 0; e < E; ++e) m = std::max(m, logit[e]);
        float sum = 0.0f;
        for (int e = 0; e < E; ++e) sum += (p[e] = std::exp(logit[e] - m));
        for (int e = 0; e < E; ++e) p[e] = rbf(p[e] / sum);
        std::vector<int> order(E);
        for (int e = 0; e < E; ++e) order[e] = e;
        std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return p[a] > p[c]; });
        float tot = 0.0f;
        for (int k = 0; k < K; ++k) tot += p[order[k]];
        const float sb = rbf(tot);
        for (int k = 0; k < K; ++k) {
          sel[k] = order[k];
          wk[k] = norm ? rbf(p[order[k]] / sb) : p[order[k]];
          if (out_idx) out_idx[static_cast<int64_t>(t) * K + k] = order[k];
        }
      }
      // gate/up + SwiGLU rows of every selected expert
#pragma omp for schedule(static)
      for (int it = 0; it < K * I; ++it) {
        const int k = it / I, n = it - k * I, e = sel[k];
        const float gv = bf(qrow_affine(gw + e * gsz + static_cast<int64_t>(n) * (H / 8), gsc + e * gss + static_cast<int64_t>(n) * (H / gs),
                                        gb + e * gss + static_cast<int64_t>(n) * (H / gs), xf.data(), xg.data(), H, gs));
        const float u = bf(qrow_affine(uw + e * gsz + static_cast<int64_t>(n) * (H / 8), usc + e * gss + static_cast<int64_t>(n) * (H / gs),
                                       ub + e * gss + static_cast<int64_t>(n) * (H / gs), xf.data(), xg.data(), H, gs));
        const float sig = rbf(1.0f / (1.0f + std::exp(-gv)));
        act[it] = bf(to_bf(rbf(gv * sig) * u));
      }
#pragma omp for schedule(static)
      for (int k = 0; k < K; ++k) group_sums(act.data() + static_cast<size_t>(k) * I, I, gs, ag.data() + static_cast<size_t>(k) * (I / gs));
      // down rows of every selected expert
#pragma omp for schedule(static)
      for (int it = 0; it < K * H; ++it) {
        const int k = it / H, h = it - k * H, e = sel[k];
        y[it] = qrow_affine(dw + e * dsz + static_cast<int64_t>(h) * (I / 8), dsc + e * dss + static_cast<int64_t>(h) * (I / gs),
                            db + e * dss + static_cast<int64_t>(h) * (I / gs), act.data() + static_cast<size_t>(k) * I,
                            ag.data() + static_cast<size_t>(k) * (I / gs), I, gs);
      }
      // native combine, k ascending
#pragma omp for schedule(static)
      for (int h = 0; h < H; ++h) {
        float acc = 0.0f;
        for (int k = 0; k < K; ++k) acc += rbf(wk[k] * bf(y[static_cast<int64_t>(k) * H + h]));
        out[static_cast<int64_t>(t) * H + h] = to_bf(acc);
      }
    }
  }
}

}  // extern "C"
