// Wave-level routing of one token row, shared by the standalone router
// kernels and the single-launch layer kernel so both produce bit-identical
// routing.
//
// Layout: lane l holds experts l, l+64, ... (P values per lane, P = 1..16
// for E <= 64P) in registers; wave-private LDS holds only the short winner
// list.  Top-k is k rounds of wave argmax on order-preserving integer keys
// (DPP max, then a ballot for the lowest index holding it), no memory
// traffic.  Selection order everywhere: value descending, lower expert index
// first on ties.
#pragma once

#include "zmoe_common.h"

namespace zmoe {

constexpr int kMaxTopK = 16;

// Per-wave LDS scratch of the router.
struct RouteLds {
  float gsc[64];  // group scores (grouped router)
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

// Wave maximum of an unsigned key (every lane gets it).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#define ZMOE_DPP_UMAX(ctrl) \
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), (ctrl), 0xF, 0xF, false)))
  ZMOE_DPP_UMAX(kDppQuadSwap1);
  ZMOE_DPP_UMAX(kDppQuadSwap2);
  ZMOE_DPP_UMAX(kDppHalfMirror);
  ZMOE_DPP_UMAX(kDppRowMirror);
#undef ZMOE_DPP_UMAX
  const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(static_cast<uint32_t>(q[0]), static_cast<uint32_t>(q[1]));
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(static_cast<uint32_t>(r[0]), static_cast<uint32_t>(r[1]));
}

// Winner r of a top-k, held by lane r (r < k).
struct TopK {
  int e;
  float val;
  float aux;
};

// k largest of v[0..n) (lane-strided registers), ties to the lower index,
// by k rounds of wave argmax.  Lane r < k returns winner r (index, value,
// aux[] of the winner); R.sel / R.sval / R.saux get the same lists.  All 64
// lanes call it.
template <int P>
__device__ __forceinline__ TopK reg_topk(const float (&v)[P], const float (&aux)[P], int n, int k, ZMOE_LDS RouteLds& R,
                                         bool want_aux = false) {
  const int lane = __lane_id();
  uint32_t key[P];
  bool bf = true;  // every value bf16-representable (low 16 bits zero)
#pragma unroll
  for (int i = 0; i < P; ++i) {
    key[i] = (lane + 64 * i < n) ? order_key(v[i]) : 0u;
    bf = bf && ((lane + 64 * i >= n) || (__float_as_uint(v[i]) & 0xFFFFu) == 0u);
  }
  TopK mine{0, 0.0f, 0.0f};
  if (__all(bf) && n <= 0xFFFF) {
    // bf16 values: (16-bit order key << 16) | (0xFFFF - index) is unique and
    // orders like (value desc, index asc), so one max finds the winner and
    // its value decodes from the key.
    uint32_t pk[P];
#pragma unroll
    for (int i = 0; i < P; ++i)
      pk[i] = (lane + 64 * i < n) ? ((key[i] & 0xFFFF0000u) | (0xFFFFu - static_cast<uint32_t>(lane + 64 * i))) : 0u;
    uint32_t mine_m = 0;
    for (int r = 0; r < k; ++r) {
      uint32_t m = pk[0];
#pragma unroll
      for (int i = 1; i < P; ++i) m = max(m, pk[i]);
      m = wave_max_u32(m);
#pragma unroll
      for (int i = 0; i < P; ++i) pk[i] = (pk[i] == m) ? 0u : pk[i];
      mine_m = (lane == r) ? m : mine_m;
      if (want_aux) {
        const int e = __builtin_amdgcn_readfirstlane(static_cast<int>(0xFFFFu - (m & 0xFFFFu)));  // uniform
        const int wl = e & 63, wi = e >> 6;
        float wa = 0.0f;
#pragma unroll
        for (int i = 0; i < P; ++i)
          if (i == wi) wa = readlane_f(aux[i], wl);
        if (lane == r) mine.aux = wa;
      }
    }
    {
      const uint32_t ok = mine_m >> 16;
      const uint32_t u16 = (ok & 0x8000u) ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
      mine.e = static_cast<int>(0xFFFFu - (mine_m & 0xFFFFu));
      mine.val = __uint_as_float(u16 << 16);
    }
    if (lane < k) {
      R.sel[lane] = mine.e;
      R.sval[lane] = mine.val;
      R.saux[lane] = mine.aux;
    }
    wave_lds_sync();
    return mine;
  }
  for (int r = 0; r < k; ++r) {
    uint32_t m = key[0];
#pragma unroll
    for (int i = 1; i < P; ++i) m = max(m, key[i]);
    m = wave_max_u32(m);
    // lowest expert index holding the maximum: lowest slot, then lowest lane
    int wi = 0;
    uint64_t hit = 0;
#pragma unroll
    for (int i = P - 1; i >= 0; --i) {
      const uint64_t b = __ballot(key[i] == m);
      if (b) {
        hit = b;
        wi = i;
      }
    }
    const int wl = __ffsll(static_cast<unsigned long long>(hit)) - 1;
    float wv = 0.0f, wa = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if (i == wi) {
        wv = readlane_f(v[i], wl);
        wa = readlane_f(aux[i], wl);
      }
    }
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (i == wi && lane == wl) key[i] = 0u;
    if (lane == r) {
      mine.e = wl + 64 * wi;
      mine.val = wv;
      mine.aux = wa;
    }
  }
  if (lane < k) {
    R.sel[lane] = mine.e;
    R.sval[lane] = mine.val;
    R.saux[lane] = mine.aux;
  }
  wave_lds_sync();
  return mine;
}

// ((0 + x[lane 0]) + x[lane 1]) + ... + x[lane k-1]: a sum in selection order
// of per-lane winner values (uniform result).
__device__ __forceinline__ float ordered_lane_sum(float x, int k) {
  float s = 0.0f;
  for (int r = 0; r < k; ++r) s += readlane_f(x, r);
  return s;
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
// Top-2 of the 32 values held by a 32-lane half of the wave (lanes h*32 ..
// h*32+31), returned to every lane of the half: butterfly merges of
// (first, second) pairs.  max/min of floats are exact, so the pair equals
// the serial scan's.
__device__ __forceinline__ void half_top2(float x, float& t1, float& t2) {
  t1 = x;
  t2 = -INFINITY;
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) {
    const float b1 = __shfl_xor(t1, o), b2 = __shfl_xor(t2, o);
    const float n2 = fmaxf(fminf(t1, b1), fmaxf(t2, b2));
    t1 = fmaxf(t1, b1);
    t2 = n2;
  }
}

// `bias_pre` (optional): the bias values bias[lane + 64 i], loaded by the
// caller ahead of time (grouped router), so route_row does not wait for them.
template <int P>
__device__ __forceinline__ void route_row(const RouteArgs a, RowVals<P> row, ZMOE_LDS RouteLds& R, ZMOE_LDS float* grow,
                                          const RowVals<P>* bias_pre = nullptr) {
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
    const TopK t = reg_topk(v, aux, E, k, R);
    const float sb = round_bf16(ordered_lane_sum(t.val, k));
    if (lane < k) R.w[lane] = a.norm ? div_to_bf16(t.val, sb) : t.val;
  } else if (a.kind == kRouteTopkLogits) {
    // moe.topk_gating_softmax (moe.py:1239-1396), f32 compute
    if (a.bias == nullptr && a.norm) {
      const TopK t = reg_topk(v, aux, E, k, R);
      const float m = readlane_f(t.val, 0);
      const float ex = expf(t.val - m);
      const float s = ordered_lane_sum(ex, k);
      if (lane < k) R.w[lane] = ex / s;
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
      const TopK t = reg_topk(v, aux, E, k, R);
      const float tot = ordered_lane_sum(t.val, k);
      if (lane < k) R.w[lane] = a.norm ? t.val / (tot + 1e-20f) : t.val;
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
      v[i] = aux[i] + (e < E ? (bias_pre ? bias_pre->v[i] : gload(a.bias + e)) : 0.0f);
    }
    if (a.n_group > 1 && a.topk_group < a.n_group) {
      const int gsz = E / a.n_group, ng = a.n_group, kg = a.topk_group;
      if (gsz == 32 && E == 64 * P) {
        // group g = register g / 2, lane half g % 2: a 32-lane top-2 each
#pragma unroll
        for (int i = 0; i < P; ++i) {
          float t1, t2;
          half_top2(v[i], t1, t2);
          if ((lane & 31) == 0) R.gsc[2 * i + (lane >> 5)] = t1 + t2;
        }
      } else {
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
      }
      wave_lds_sync();
      // keep the topk_group best groups (ties -> lower group index)
      uint32_t gk = lane < ng ? order_key(R.gsc[lane]) : 0u;
      uint64_t keepm = 0;
      for (int r = 0; r < kg; ++r) {
        const uint32_t m = wave_max_u32(gk);
        const int wl = __ffsll(static_cast<unsigned long long>(__ballot(gk == m))) - 1;
        keepm |= 1ull << wl;
        if (lane == wl) gk = 0u;
      }
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((keepm >> (e / gsz)) & 1ull)) v[i] = 0.0f;
      }
    }
    const TopK t = reg_topk(v, aux, E, k, R, true);
    const float s = ordered_lane_sum(t.aux, k);
    if (lane < k) {
      float x = t.aux / s;
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
