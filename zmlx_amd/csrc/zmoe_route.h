// Wave-level routing over one token row held in LDS, shared by the
// standalone router kernels and the single-launch layer kernel so both
// produce bit-identical routing.  Written for small code size (loops, no
// dynamically indexed register arrays): the whole wave cooperates on one
// row; values live in wave-private LDS.
//
// Selection order everywhere: value descending, lower expert index first on
// ties.  Top-k is a radix select of the k-th key on wave ballots, then the
// k winners are ranked.
#pragma once

#include "zmoe_common.h"

namespace zmoe {

constexpr int kMaxTopK = 16;

// Per-wave LDS scratch of the router (besides the two E-float rows `v`,
// the working values, and `aff`, the sigmoid affinities of the grouped
// router, which the caller places).
struct RouteLds {
  float gsc[64];    // group scores
  int cnt;          // winner list length
  uint32_t wkey[kMaxTopK];
  int widx[kMaxTopK];
  int sel[kMaxTopK];
  float w[kMaxTopK];
};

// Orders LDS traffic between the lanes of one wave (compiler barrier; the
// hardware executes a wave's LDS operations in order).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t lanes_below_mask(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Sum / max of v[0..n) over the wave: each lane folds its entries
// (lane, lane+64, ...) in order, then a fixed butterfly -- reproducible.
__device__ __forceinline__ float lds_row_sum(const float* v, int n) {
  float s = 0.0f;
  for (int e = __lane_id(); e < n; e += kWave) s += v[e];
  return wave_sum(s);
}

__device__ __forceinline__ float lds_row_max(const float* v, int n) {
  float m = -INFINITY;
  for (int e = __lane_id(); e < n; e += kWave) m = fmaxf(m, v[e]);
  return wave_max(m);
}

// Writes into R.sel[0..k) the k largest of vals[0..n) ordered by
// (value desc, index asc).  All 64 lanes must call it.
__device__ __forceinline__ void lds_topk(const float* vals, int n, int k, RouteLds& R) {
  const int lane = __lane_id();
  uint32_t T = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    int cnt = 0;
    for (int e0 = 0; e0 < n; e0 += kWave) {
      const int e = e0 + lane;
      cnt += __popcll(__ballot(e < n && order_key(vals[e]) >= cand));
    }
    if (cnt >= k) T = cand;
  }
  int need = k;
  for (int e0 = 0; e0 < n; e0 += kWave) {
    const int e = e0 + lane;
    need -= __popcll(__ballot(e < n && order_key(vals[e]) > T));
  }
  if (lane == 0) R.cnt = 0;
  wave_lds_sync();
  for (int e0 = 0; e0 < n; e0 += kWave) {
    const int e = e0 + lane;
    const uint32_t key = e < n ? order_key(vals[e]) : 0u;
    const bool tie = e < n && key == T;
    const uint64_t tm = __ballot(tie);
    const bool take = (e < n && key > T) || (tie && __popcll(tm & lanes_below_mask(lane)) < need);
    need -= min(need, __popcll(tm));
    if (take) {
      const int pos = atomicAdd(&R.cnt, 1);
      R.wkey[pos] = key;
      R.widx[pos] = e;
    }
  }
  wave_lds_sync();
  if (lane < k) {
    const uint32_t kr = R.wkey[lane];
    const int er = R.widx[lane];
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      const uint32_t kj = R.wkey[j];
      const int ej = R.widx[j];
      rank += (kj > kr || (kj == kr && ej < er)) ? 1 : 0;
    }
    R.sel[rank] = er;
  }
  wave_lds_sync();
}

// a/b rounded once to bf16 (the fp32 quotient is corrected when it lands
// exactly on a bf16 rounding midpoint, so no double rounding occurs).
__device__ __forceinline__ float div_to_bf16(float a, float b) {
  float q = a / b;
  const uint32_t u = __float_as_uint(q);
  if ((u & 0xFFFFu) == 0x8000u) {
    const float r = fmaf(-q, b, a);  // exact residual
    if (r != 0.0f) {
      const bool up = (r > 0.0f) == (b > 0.0f);
      q = __uint_as_float(up ? ((q >= 0.0f) ? u + 1 : u - 1) : ((q >= 0.0f) ? u - 1 : u + 1));
    }
  }
  return round_bf16(q);
}

// Router kinds (values of ZMOE_ROUTER_*).
constexpr int kRouteSoftmaxProbs = 0;
constexpr int kRouteTopkLogits = 1;
constexpr int kRouteSigmoidGrouped = 2;

struct RouteArgs {
  int kind, E, k, norm, n_group, topk_group;
  float scale;
  const float* bias;  // global, f32 [E] or null
  int w_bf16;         // round the weights to bf16 (topk-logits router in a bf16 model)
};

// Routes the row already written to v[0..E) (entries are logits); `aff` is
// E floats of scratch (grouped router only).  Results: R.sel[0..k),
// R.w[0..k).  All 64 lanes must call it.
__device__ __noinline__ void route_row(const RouteArgs& a, float* v, float* aff, RouteLds& R) {
  const int lane = __lane_id();
  const int E = a.E, k = a.k;
  if (a.kind == kRouteSoftmaxProbs) {
    // Qwen (moe_mlp.py:255-266): precise softmax -> bf16 probs -> top-k ->
    // /bf16(sum) in bf16 when norm
    const float m = lds_row_max(v, E);
    for (int e = lane; e < E; e += kWave) v[e] = expf(v[e] - m);
    wave_lds_sync();
    const float s = lds_row_sum(v, E);
    for (int e = lane; e < E; e += kWave) v[e] = div_to_bf16(v[e], s);
    wave_lds_sync();
    lds_topk(v, E, k, R);
    float tot = 0.0f;
    for (int r = 0; r < k; ++r) tot += v[R.sel[r]];
    const float sb = round_bf16(tot);
    if (lane < k) {
      const float pr = v[R.sel[lane]];
      R.w[lane] = a.norm ? div_to_bf16(pr, sb) : pr;
    }
  } else if (a.kind == kRouteTopkLogits) {
    // moe.topk_gating_softmax (moe.py:1239-1396), f32 compute
    if (a.bias == nullptr && a.norm) {
      lds_topk(v, E, k, R);
      const float m = v[R.sel[0]];
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s += expf(v[R.sel[r]] - m);
      if (lane < k) R.w[lane] = expf(v[R.sel[lane]] - m) / s;
    } else {
      const float m = lds_row_max(v, E);
      for (int e = lane; e < E; e += kWave) v[e] = expf(v[e] - m);
      wave_lds_sync();
      const float s = lds_row_sum(v, E);
      for (int e = lane; e < E; e += kWave) v[e] = v[e] / s + (a.bias ? a.bias[e] : 0.0f);
      wave_lds_sync();
      lds_topk(v, E, k, R);
      float t = 0.0f;
      for (int r = 0; r < k; ++r) t += v[R.sel[r]];
      if (lane < k) R.w[lane] = a.norm ? v[R.sel[lane]] / (t + 1e-20f) : v[R.sel[lane]];
    }
    if (a.w_bf16 && lane < k) R.w[lane] = round_bf16(R.w[lane]);
  } else {
    // DeepSeek/GLM grouped sigmoid router (moe.py:1501-1742,
    // deepseek_router.py:118)
    for (int e = lane; e < E; e += kWave) {
      const float af = sigmoid_abs(v[e]);
      aff[e] = af;
      v[e] = af + a.bias[e];
    }
    wave_lds_sync();
    if (a.n_group > 1 && a.topk_group < a.n_group) {
      const int gsz = E / a.n_group;
      if (lane < a.n_group) {
        float t1 = -INFINITY, t2 = -INFINITY;
        for (int j = 0; j < gsz; ++j) {
          const float x = v[lane * gsz + j];
          if (x > t1) {
            t2 = t1;
            t1 = x;
          } else if (x > t2) {
            t2 = x;
          }
        }
        R.gsc[lane] = t1 + t2;
      }
      wave_lds_sync();
      // keep the topk_group best groups (ties -> lower group index): mark
      // them through the same radix select
      uint32_t T = 0;
      const int ng = a.n_group, kg = a.topk_group;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        if (__popcll(__ballot(lane < ng && order_key(R.gsc[lane]) >= cand)) >= kg) T = cand;
      }
      int need = kg - __popcll(__ballot(lane < ng && order_key(R.gsc[lane]) > T));
      const uint32_t gk = lane < ng ? order_key(R.gsc[lane]) : 0u;
      const uint64_t tm = __ballot(lane < ng && gk == T);
      const bool keep = lane < ng && (gk > T || (gk == T && __popcll(tm & lanes_below_mask(lane)) < need));
      const uint64_t keepm = __ballot(keep);
      for (int e = lane; e < E; e += kWave)
        if (!((keepm >> (e / gsz)) & 1ull)) v[e] = 0.0f;
      wave_lds_sync();
    }
    lds_topk(v, E, k, R);
    float s = 0.0f;
    for (int r = 0; r < k; ++r) s += aff[R.sel[r]];
    if (lane < k) {
      float x = aff[R.sel[lane]] / s;
      if (a.scale != 1.0f) x = x * a.scale;
      R.w[lane] = x;
    }
  }
  wave_lds_sync();
}

}  // namespace zmoe
