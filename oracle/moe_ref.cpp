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
// Accumulation here is fp32 per group (s*sum(q*x) + b*sum(x), the factoring
// MLX's qmv kernels use), so results agree with the float64 oracle to within
// fp32 rounding, not bit for bit.
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

// y[n] = bf16( sum_g s[n,g]*sum(q*x) + b[n,g]*sum(x) ) for rows n of one
// affine 4-bit matrix [N, K/8].
void qmv_affine(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x, int N, int K, int gs,
                uint16_t* y) {
  const int G = K / gs;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint32_t* wr = w + static_cast<int64_t>(n) * (K / 8);
    float acc = 0.0f;
    for (int g = 0; g < G; ++g) {
      float qx = 0.0f, sx = 0.0f;
      for (int i = g * gs; i < (g + 1) * gs; ++i) {
        const float q = static_cast<float>((wr[i >> 3] >> ((i & 7) * 4)) & 0xFu);
        qx += q * x[i];
        sx += x[i];
      }
      acc += bf(s[static_cast<int64_t>(n) * G + g]) * qx + bf(b[static_cast<int64_t>(n) * G + g]) * sx;
    }
    y[n] = to_bf(acc);
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
  std::vector<float> xf(H), logit(E), act_f(I);
  std::vector<uint16_t> g(I), u(I), act(I), y(static_cast<size_t>(K) * H);
  const int64_t gsz = static_cast<int64_t>(I) * (H / 8), gss = static_cast<int64_t>(I) * (H / gs);
  const int64_t dsz = static_cast<int64_t>(H) * (I / 8), dss = static_cast<int64_t>(H) * (I / gs);
  for (int t = 0; t < B; ++t) {
    for (int h = 0; h < H; ++h) xf[h] = bf(x[static_cast<int64_t>(t) * H + h]);
#pragma omp parallel for schedule(static)
    for (int e = 0; e < E; ++e) {
      float acc = 0.0f;
      for (int h = 0; h < H; ++h) acc += xf[h] * bf(wr[static_cast<int64_t>(e) * H + h]);
      logit[e] = rbf(acc);
    }
    float m = -INFINITY;
    for (int e = 0; e < E; ++e) m = std::max(m, logit[e]);
    float sum = 0.0f;
    std::vector<float> p(E);
    for (int e = 0; e < E; ++e) sum += (p[e] = std::exp(logit[e] - m));
    for (int e = 0; e < E; ++e) p[e] = rbf(p[e] / sum);
    std::vector<int> order(E);
    for (int e = 0; e < E; ++e) order[e] = e;
    std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return p[a] > p[c]; });
    float tot = 0.0f;
    for (int k = 0; k < K; ++k) tot += p[order[k]];
    const float sb = rbf(tot);
    for (int k = 0; k < K; ++k) {
      const int e = order[k];
      if (out_idx) out_idx[static_cast<int64_t>(t) * K + k] = e;
      qmv_affine(gw + e * gsz, gsc + e * gss, gb + e * gss, xf.data(), I, H, gs, g.data());
      qmv_affine(uw + e * gsz, usc + e * gss, ub + e * gss, xf.data(), I, H, gs, u.data());
      for (int i = 0; i < I; ++i) {
        const float gv = bf(g[i]);
        const float sig = rbf(1.0f / (1.0f + std::exp(-gv)));
        act_f[i] = bf(to_bf(rbf(gv * sig) * bf(u[i])));
      }
      qmv_affine(dw + e * dsz, dsc + e * dss, db + e * dss, act_f.data(), H, I, gs, y.data() + static_cast<int64_t>(k) * H);
    }
    for (int h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) {
        const float wk = norm ? rbf(p[order[k]] / sb) : p[order[k]];
        acc += rbf(wk * bf(y[static_cast<int64_t>(k) * H + h]));
      }
      out[static_cast<int64_t>(t) * H + h] = to_bf(acc);
    }
  }
}

}  // extern "C"
