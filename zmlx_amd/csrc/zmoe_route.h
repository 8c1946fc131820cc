// Wave-level routing of one token row, shared by the standalone router
// kernels and the single-launch layer kernel so both produce bit-identical
// routing.
//
// Layout: lane l holds experts l, l+64, ... (P values per lane, P = 1..16
// for E <= 64P) in registers; wave-private LDS holds only the short winner
// list.  Top-k is a radix select of the k-th key on wave ballots (32 steps,
// no memory traffic), then the winners are ranked.  Selection order
// everywhere: value descending, lower expert index first on ties.
#pragma once

#include "zmoe_common.h"

namespace zmoe {

constexpr int kMaxTopK = 16;

// Per-wave LDS scratch of the router.
struct RouteLds {
  float gsc[64];  // group scores (grouped router)
  int cnt;        // winner list length
  uint32_t wkey[kMaxTopK];
  int widx[kMaxTopK];
  float wval[kMaxTopK];
  float waux[kMaxTopK];
  int sel[kMaxTopK];   // result: selected experts in order
  float sval[kMaxTopK];
  float saux[kMaxTopK];
  float w[kMaxTopK];   // result: weights
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

// Wave sum / max of a lane-strided row: each lane folds its P values in
// slot order, then a fixed butterfly -- reproducible.
template <int P>
__device__ __forceinline__ float reg_row_sum(const float (&v)[P], int E) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < P; ++i)
    if (__lane_id() + 64 * i < E) s += v[i];
  return wave_sum(s);
}

template <int P>
__device__ __forceinline__ float reg_row_max(const float (&v)[P], int E) {
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < P; ++i)
    if (__lane_id() + 64 * i < E) m = fmaxf(m, v[i]);
  return wave_max(m);
}

// k largest of v[0..n) (lane-strided registers), ties to the lower index.
// Fills R.sel / R.sval (value) / R.saux (aux[] of the winner) in order
// (value desc, index asc).  All 64 lanes call it.
template <int P>
__device__ __forceinline__ void reg_topk(const float (&v)[P], const float (&aux)[P], int n, int k, ZMOE_LDS RouteLds& R) {
  const int lane = __lane_id();
  uint32_t key[P];
#pragma unroll
  for (int i = 0; i < P; ++i) key[i] = (lane + 64 * i < n) ? order_key(v[i]) : 0u;
  uint32_t T = 0;  // largest threshold with |{key >= T}| >= k
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) cnt += __popcll(__ballot(key[i] >= cand));
    if (cnt >= k) T = cand;
  }
  int need = k;
#pragma unroll
  for (int i = 0; i < P; ++i) need -= __popcll(__ballot(key[i] > T));
  if (lane == 0) R.cnt = 0;
  wave_lds_sync();
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const bool tie = key[i] == T && key[i] != 0u;
    const uint64_t tm = __ballot(tie);
    const bool take = key[i] > T || (tie && __popcll(tm & lanes_below_mask(lane)) < need);
    need -= min(need, __popcll(tm));
    if (take) {
      const int pos = __hip_atomic_fetch_add(&R.cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
      R.wkey[pos] = key[i];
      R.widx[pos] = lane + 64 * i;
      R.wval[pos] = v[i];
      R.waux[pos] = aux[i];
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
    R.sval[rank] = R.wval[lane];
    R.saux[rank] = R.waux[lane];
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

// One row of scores in lane-strided registers (passed by value so a call
// keeps it in VGPRs).
template <int P>
struct RowVals {
  float v[P];
};

// Routes one row of logits given lane-strided in row.v (entries >= E
// ignored).  Results: R.sel[0..k), R.w[0..k).  All 64 lanes call it.
// `grow` is E floats of wave-private LDS (grouped router only).
template <int P>
__device__ __forceinline__ void route_row(const RouteArgs a, RowVals<P> row, ZMOE_LDS RouteLds& R, ZMOE_LDS float* grow) {
  float (&v)[P] = row.v;
  const int lane = __lane_id();
  const int E = a.E, k = a.k;
  float aux[P];
#pragma unroll
  for (int i = 0; i < P; ++i) aux[i] = 0.0f;
  if (a.kind == kRouteSoftmaxProbs) {
    // Qwen (moe_mlp.py:255-266): precise softmax -> bf16 probs -> top-k ->
    // /bf16(sum) in bf16 when norm
    const float m = reg_row_max(v, E);
#pragma unroll
    for (int i = 0; i < P; ++i) v[i] = expf(v[i] - m);
    const float s = reg_row_sum(v, E);
#pragma unroll
    for (int i = 0; i < P; ++i) v[i] = div_to_bf16(v[i], s);
    reg_topk(v, aux, E, k, R);
    float tot = 0.0f;
    for (int r = 0; r < k; ++r) tot += R.sval[r];
    const float sb = round_bf16(tot);
    if (lane < k) R.w[lane] = a.norm ? div_to_bf16(R.sval[lane], sb) : R.sval[lane];
  } else if (a.kind == kRouteTopkLogits) {
    // moe.topk_gating_softmax (moe.py:1239-1396), f32 compute
    if (a.bias == nullptr && a.norm) {
      reg_topk(v, aux, E, k, R);
      const float m = R.sval[0];
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s += expf(R.sval[r] - m);
      if (lane < k) R.w[lane] = expf(R.sval[lane] - m) / s;
    } else {
      const float m = reg_row_max(v, E);
#pragma unroll
      for (int i = 0; i < P; ++i) v[i] = expf(v[i] - m);
      const float s = reg_row_sum(v, E);
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        v[i] = v[i] / s + ((a.bias && e < E) ? gload(a.bias + e) : 0.0f);
      }
      reg_topk(v, aux, E, k, R);
      float t = 0.0f;
      for (int r = 0; r < k; ++r) t += R.sval[r];
      if (lane < k) R.w[lane] = a.norm ? R.sval[lane] / (t + 1e-20f) : R.sval[lane];
    }
    if (a.w_bf16 && lane < k) R.w[lane] = round_bf16(R.w[lane]);
  } else {
    // DeepSeek/GLM grouped sigmoid router (moe.py:1501-1742,
    // deepseek_router.py:118): scores = sigmoid + bias select, weights are
    // the normalised sigmoids
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int e = lane + 64 * i;
      aux[i] = sigmoid_abs(v[i]);
      v[i] = aux[i] + (e < E ? gload(a.bias + e) : 0.0f);
    }
    if (a.n_group > 1 && a.topk_group < a.n_group) {
      const int gsz = E / a.n_group, ng = a.n_group, kg = a.topk_group;
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (lane + 64 * i < E) grow[lane + 64 * i] = v[i];
      wave_lds_sync();
      if (lane < ng) {
        float t1 = -INFINITY, t2 = -INFINITY;
#pragma unroll 8
        for (int j = 0; j < gsz; ++j) {
          const float x = grow[lane * gsz + j];
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
      // keep the topk_group best groups (ties -> lower group index)
      const uint32_t gk = lane < ng ? order_key(R.gsc[lane]) : 0u;
      uint32_t T = 0;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        if (__popcll(__ballot(gk >= cand)) >= kg) T = cand;
      }
      const int need = kg - __popcll(__ballot(gk > T));
      const uint64_t tm = __ballot(gk == T && gk != 0u);
      const bool keep = gk > T || (gk == T && gk != 0u && __popcll(tm & lanes_below_mask(lane)) < need);
      const uint64_t keepm = __ballot(keep);
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((keepm >> (e / gsz)) & 1ull)) v[i] = 0.0f;
      }
    }
    reg_topk(v, aux, E, k, R);
    float s = 0.0f;
    for (int r = 0; r < k; ++r) s += R.saux[r];
    if (lane < k) {
      float x = R.saux[lane] / s;
      if (a.scale != 1.0f) x = x * a.scale;
      R.w[lane] = x;
    }
  }
  wave_lds_sync();
}

// Values per lane needed for E experts.
__host__ __device__ constexpr int route_slots(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16; }

// Loads a row through `get(e)` into P lane-strided registers and routes it.
template <int P, typename F>
__device__ __forceinline__ void route_row_p(const RouteArgs& a, F get, ZMOE_LDS RouteLds& R, ZMOE_LDS float* grow) {
  const int lane = __lane_id();
  RowVals<P> row;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int e = lane + 64 * i;
    row.v[i] = e < a.E ? get(e) : -INFINITY;
  }
  route_row<P>(a, row, R, grow);
}

// Loads a row through `get(e)` into lane-strided registers and routes it with
// the smallest register footprint that holds E.
template <typename F>
__device__ __forceinline__ void route_row_any(const RouteArgs& a, F get, ZMOE_LDS RouteLds& R, ZMOE_LDS float* grow) {
  const int lane = __lane_id();
#define ZMOE_ROUTE_P(PP)                                             \
  {                                                                  \
    RowVals<PP> row;                                                 \
    _Pragma("unroll") for (int i = 0; i < PP; ++i) {                 \
      const int e = lane + 64 * i;                                   \
      row.v[i] = e < a.E ? get(e) : -INFINITY;                       \
    }                                                                \
    route_row<PP>(a, row, R, grow);                                  \
  }
  switch (route_slots(a.E)) {
    case 1: ZMOE_ROUTE_P(1) break;
    case 2: ZMOE_ROUTE_P(2) break;
    case 4: ZMOE_ROUTE_P(4) break;
    case 8: ZMOE_ROUTE_P(8) break;
    default: ZMOE_ROUTE_P(16) break;
  }
#undef ZMOE_ROUTE_P
}

}  // namespace zmoe
