// One-token MoE decode layer in a single launch (B = 1; the path of
// zmoe_moe_layer for single-token decode, moe_mlp.py:787-1072 patched_call).
//
// Same phases, workspace, tagged cross-workgroup exchange and arithmetic as
// the small-batch kernel of layer_fused.hip (results are bit-identical to it
// and to the kernel sequence), specialised for one token so that little code
// sits on the critical path:
//
//   R  router partial dots, spread over every workgroup (unit u -> workgroup
//      u % G, wave u / G) so that each one's weight load is the only HBM
//      latency before the exchange; x is staged in LDS meanwhile.
//   T  wave 0 of every workgroup polls the tagged partials, routes, and writes
//      a per-unit pointer table (gate/up/down weights, scales, biases of each
//      selected expert and of the shared expert) to LDS.
//   A  gate/up + SwiGLU: every wave owns a contiguous range of (unit, row)
//      pairs; the whole range's loads are issued at once, followed at once by
//      the wave's down-projection loads, so all the layer's weight bytes are in
//      flight right after routing.  act rows go to the workspace, tagged.
//   D  every workgroup stages the act rows in LDS (polling their tags); each
//      wave owns output rows h of every unit, whose weights are already in its
//      registers, and finishes them with the k-ordered combine and the
//      shared-expert add without a workgroup barrier.
//
// The unit table keeps per-item address arithmetic to one 64-bit add and
// keeps the kernel within the scalar register file (no spills).
#include "zmoe_decode1.h"

#include <cstddef>
#include <cstdlib>
#include <vector>
#include <type_traits>

namespace zmoe {

// arrival counters of the act exchange, in the workspace block at p.aflag:
// kD1Ctrs counters kD1CtrStride words apart, then one launch count per
// workgroup at word kD1CtrEpoch
constexpr int kD1Ctrs = 32;
constexpr int kD1CtrStride = 32;
constexpr int kD1CtrEpoch = kD1Ctrs * kD1CtrStride;

struct D1Layout {
  size_t xs, sx, as, asx, ybuf, grow, total;
};

__host__ __device__ inline D1Layout d1_layout(int H, int I, int E, int Uall, int rpw) {
  D1Layout o;
  const int S_H = H / 32, S_I = I / 32;
  size_t off = (sizeof(D1Lds) + 15) & ~static_cast<size_t>(15);
  o.xs = off;
  off += static_cast<size_t>(lds_row_words(S_H)) * 4;
  o.sx = off;
  off += static_cast<size_t>(S_H) * 4;
  off = (off + 15) & ~static_cast<size_t>(15);
  o.as = off;
  off += static_cast<size_t>(Uall) * lds_row_words(S_I) * 4;
  o.asx = off;
  off += static_cast<size_t>(Uall) * S_I * 4;
  o.ybuf = off;
  off += static_cast<size_t>(kFWaves) * rpw * Uall * 4;
  o.grow = off;
  off += static_cast<size_t>(E) * 4;
  o.total = off;
  return o;
}

// Grouped sigmoid router (moe.py:1501-1742, deepseek_router.py:118) for
// E = 64 P experts, groups of 32 (or no group limit), wave 0: the selection
// scores sigmoid + bias with the dropped groups' scores set to 0, as unique
// keys (order key << 32 | ~e: value descending, then lower index) in
// keys[e], and the sigmoids in aux[e].  The group top-2 sums are
// 32-lane butterflies; the kept groups are the topk_group best by rank
// (ties to the lower group), the set the argmax rounds of route_row keep.
template <int P>
__device__ __forceinline__ void sig_scores(const RouteArgs& a, RowVals<P> row, const RowVals<P>* bias_pre,
                                           ZMOE_LDS RouteLds& R, uint64_t* keys, float* aux) {
  const int lane = __lane_id();
  float v[P], sg[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    sg[i] = sigmoid_abs(row.v[i]);
    v[i] = sg[i] + (bias_pre ? bias_pre->v[i] : 0.0f);
  }
  if (a.n_group > 1 && a.topk_group < a.n_group) {
    const int ng = a.n_group;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      float t1, t2;
      half_top2(v[i], t1, t2);
      if ((lane & 31) == 0) R.gsc[2 * i + (lane >> 5)] = t1 + t2;
    }
    wave_lds_sync();
    const uint32_t gk = lane < ng ? order_key(R.gsc[lane]) : 0u;
    int rank = 0;
    for (int g = 0; g < ng; ++g) {
      const uint32_t o = order_key(R.gsc[g]);
      rank += (o > gk || (o == gk && g < lane)) ? 1 : 0;
    }
    const uint64_t keepm = __ballot(lane < ng && rank < a.topk_group);
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (!((keepm >> ((lane + 64 * i) >> 5)) & 1ull)) v[i] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < P; ++i) {
    keys[lane + 64 * i] = static_cast<uint64_t>(order_key(v[i])) << 32 | (0xFFFFFFFFu - static_cast<uint32_t>(lane + 64 * i));
    aux[lane + 64 * i] = sg[i];
  }
}

// Weights of the grouped sigmoid router's ranked winners (wave 0; lane r < K
// holds winner r): the sigmoids normalised in selection order, scaled; then
// the routing outputs of workgroup 0.
__device__ __forceinline__ void sig_weights(const FusedParams& p, D1Lds& L, int K) {
  const int lane = __lane_id();
  const float a = lane < K ? L.route.saux[lane] : 0.0f;
  const float sum = ordered_lane_sum(a, K);
  float x = a / sum;
  if (p.route.scale != 1.0f) x = x * p.route.scale;
  if (lane < K) {
    L.route.w[lane] = x;
    if (blockIdx.x == 0) {
      if (p.out_idx) gstore(p.out_idx + lane, static_cast<uint32_t>(L.route.sel[lane]));
      if (p.out_w) gstore(p.out_w + lane, x);
    }
  }
}

template <int QMODE, int P, bool XR>
__global__ __launch_bounds__(kFThreads) void k_moe_decode1(FusedParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  D1Lds& L = *reinterpret_cast<D1Lds*>(smem);
  wg_dead_clear();

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int lane = __lane_id();
  const int G = gridDim.x;
  const int W = G * kFWaves;
  const int gw = blockIdx.x * kFWaves + wave;
  const int E = p.E, K = p.K, H = p.H, I = p.I;
  const int NC = H >> 9;
  const int S_H = H >> 5, S_I = I >> 5;
  const AffineK ak = affine_k();
  const bool has_shared = p.Is > 0;
  const D1Plan& pl = p.d1;
  const int Uall = pl.Uall;
  const int rpw = pl.rpw;
  const D1Layout lay = d1_layout(H, I, E, Uall, rpw);
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem + lay.xs);
  float* sx = reinterpret_cast<float*>(smem + lay.sx);
  uint32_t* as = reinterpret_cast<uint32_t*>(smem + lay.as);
  float* asx = reinterpret_cast<float*>(smem + lay.asx);
  float* ybuf = reinterpret_cast<float*>(smem + lay.ybuf);
  float* grow = reinterpret_cast<float*>(smem + lay.grow);

  trace_mark(p, 0);
  const unsigned epoch = dev_load(p.sync + kEpochWord + blockIdx.x);
  const unsigned tag = epoch + 1u;
  const unsigned tag16 = tag & 0xFFFFu;
  // launches of this kernel this workgroup completed (arrival-counter target)
  const unsigned ctag = dev_load(p.aflag + kD1CtrEpoch + blockIdx.x) + 1u;

  // Work assignment (independent of the routing, computed and pinned here so
  // that none of it runs after the routing wait):
  // phase D: output rows [h0, h0 + nrows); slot = (row, unit), unit fastest;
  // RPID slots per load instruction (lane group rsD), TD segments per lane.
  const int LI = 1 << pl.lLI, RPID = kWave >> pl.lLI;
  const int rsD = lane >> pl.lLI, liD = lane & (LI - 1);
  const int TD = pl.TD;
  int h0 = gw * rpw;
  int nrows = max(0, min(H, h0 + rpw) - h0);
  int slots = nrows * Uall;
  int n_itemsD = ((slots + RPID - 1) >> (6 - pl.lLI)) * TD;
  int d_hl = static_cast<int>(fdiv(static_cast<uint32_t>(rsD), pl.by_Uall));
  int d_u = rsD - d_hl * Uall, d_t = 0, d_g = 0;
  pin_s(h0);
  pin_s(nrows);
  pin_s(slots);
  pin_s(n_itemsD);
  asm volatile("" : "+v"(d_hl), "+v"(d_u));
  // phase A: a contiguous range of (unit, row-group) items
  int a_g0, a_g1, a_cu, a_cr;
  {
    const int rg_total = (pl.shpre ? K : Uall) * pl.rgu;  // (shpre: the shared unit's rows come earlier)
    a_g0 = min(rg_total, gw * pl.perA);
    a_g1 = min(rg_total, a_g0 + pl.perA);
    a_cu = static_cast<int>(fdiv(static_cast<uint32_t>(a_g0), pl.by_rgu));
    a_cr = a_g0 - a_cu * pl.rgu;
  }
  pin_s(a_g0);
  pin_s(a_g1);
  pin_s(a_cu);
  pin_s(a_cr);

  // ---------------- R: router partials ----------------
  // Unit (e, c) = 512-column chunk c of router row e, on workgroup u % G,
  // wave u / G: the lane's 8-element dot and a wave sum, published as one
  // tagged word (f32 | tag << 32); readers add the chunks in order.
  for (int u = wave * G + blockIdx.x; u < E * NC; u += W) {
    const int e = static_cast<int>(fdiv(static_cast<uint32_t>(u), pl.by_NC)), c = u - e * NC;
    const uint4 wv = gload(reinterpret_cast<const uint4*>(p.wr + static_cast<int64_t>(e) * H + c * 512 + lane * 8));
    const uint4 xv = gload(reinterpret_cast<const uint4*>(p.x + c * 512 + lane * 8));
    float a = 0.0f;
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.x), __builtin_bit_cast(bf16x2_t, xv.x), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.y), __builtin_bit_cast(bf16x2_t, xv.y), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.z), __builtin_bit_cast(bf16x2_t, xv.z), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.w), __builtin_bit_cast(bf16x2_t, xv.w), a, false);
    a = wave_sum(a);
    if (lane == 0)
      dev_store(p.rpart + static_cast<int64_t>(e) * NC + c, (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(a));
  }
  stage_rows_lds<QMODE, false>(p, p.x, H, 1, S_H, xs, sx, 0u, p.by_S4H, p.by_SH);
  trace_mark(p, 1);
  lds_barrier();
  trace_mark(p, 2);

  // ---------------- S: the shared expert's gate/up rows, before routing ----------------
  // (general H) The shared expert does not depend on the routing: its
  // row-groups are dealt to the waves here, while the router partials are
  // still being exchanged, with phase A's arithmetic (segment steps in order,
  // the LH-lane sum) and its tagged act stores; phase A then covers the K
  // routed units only.
  if constexpr (!XR) {
    if (pl.shpre) {
      const int LH = 1 << pl.lLH, RPI = kWave >> pl.lLH;
      const int rs = lane >> pl.lLH, li = lane & (LH - 1);
      const int T = pl.TA;
      const int64_t wpr = H >> 3;
      const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S_H >> p.gshift) : S_H;
      constexpr int SB = 8;  // segment steps per batch of loads
      for (int g = gw; g < pl.rgu; g += W) {
        const int64_t row = static_cast<int64_t>(g) * RPI + rs;
        float ag = 0.0f, au = 0.0f;
        for (int t0 = 0; t0 < T; t0 += SB) {
          uint4 wgv[SB], wuv[SB];
          RawParam rgv[SB], ruv[SB];
#pragma unroll
          for (int j = 0; j < SB; ++j) {
            const int t = min(t0 + j, T - 1);  // past the last step: repeat it (loads stay unconditional)
            const int sgm = t * LH + li;
            const int64_t po = row * ppr + ((QMODE == ZMOE_Q_AFFINE) ? (sgm >> p.gshift) : sgm);
            wgv[j] = gload(reinterpret_cast<const uint4*>(p.w[3] + row * wpr + sgm * 4));
            wuv[j] = gload(reinterpret_cast<const uint4*>(p.w[4] + row * wpr + sgm * 4));
            rgv[j] = seg_param_load<QMODE>(p.s[3], p.b[3], po);
            ruv[j] = seg_param_load<QMODE>(p.s[4], p.b[4], po);
          }
#pragma unroll
          for (int j = 0; j < SB; ++j) {
            const int t = t0 + j;
            if (t < T) {
              const int sgm = t * LH + li;
              float sgj, cgj, suj, cuj;
              seg_param_decode<QMODE>(rgv[j], sgj, cgj);
              seg_param_decode<QMODE>(ruv[j], suj, cuj);
              const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[sgm] : 0.0f;
              ag = seg_accum<QMODE>(t == 0 ? 0.0f : ag, sgj, cgj, seg_dot_lds<QMODE>(wgv[j], xs, S_H, 0, sgm, ak), xsum);
              au = seg_accum<QMODE>(t == 0 ? 0.0f : au, suj, cuj, seg_dot_lds<QMODE>(wuv[j], xs, S_H, 0, sgm, ak), xsum);
            }
          }
        }
        const float gv = lanes_sum(ag, LH);
        const float uv = lanes_sum(au, LH);
        if (li == 0)
          dev_store(p.act + static_cast<int64_t>(K) * p.act_stride + row,
                    (tag16 << 16) | (wg_dead() ? kBf16NaN : swiglu_bf16(round_bf16(gv), round_bf16(uv))));
      }
    }
  }

  // ---------------- T: routing and the unit table ----------------
  // Softmax-probability routers (and top-k over logits with renormalised
  // weights) select by ranking: wave 0 writes one unique key per expert
  // (bf16 value order, then lower index first), every thread counts the keys
  // above one expert's key over a slice of the row, and the expert of rank r
  // becomes winner r -- the same winners in the same order as k rounds of
  // argmax, with a short dependency chain spread over the workgroup.  The
  // thread that finds rank r writes unit r's pointers; the gate weights are
  // only needed by the final combine, so wave 0 computes them later, while
  // its weight loads are in flight.  Other routers run route_row in wave 0.
  const int rkind = p.route.kind;
  const bool rank_route = E <= kD1RankMaxE && K <= kMaxTopK &&
                          (rkind == kRouteSoftmaxProbs ||
                           (rkind == kRouteTopkLogits && p.route.bias == nullptr && p.route.norm));
  const int Epad = E <= 64 ? 64 : (E <= 128 ? 128 : 256);
  // Routers that run route_row in wave 0 (grouped sigmoid, ...): with more
  // than 64 experts every wave polls 64 experts' partials (summed in chunk
  // order, rounded to bf16: the same logits), into L.keys, so the partials
  // are read with 8 waves' loads in flight instead of one.
  const bool par_poll = !rank_route && E > kWave && E <= kD1RankMaxE;
  // Grouped sigmoid routers with E = 64 P experts and groups of 32 (or no
  // group limit) also select by ranking, over fp32 score keys with index
  // ties; the others run route_row in wave 0.
  const bool sig_rank = !rank_route && rkind == kRouteSigmoidGrouped && E == kWave * P && K <= kMaxTopK &&
                        (p.route.n_group <= 1 || p.route.topk_group >= p.route.n_group ||
                         (p.route.n_group <= 64 && E == 32 * p.route.n_group));
  // the grouped router's bias, loaded before the logits are waited for
  RowVals<P> biasv;
  const bool pre_bias = !rank_route && rkind == kRouteSigmoidGrouped && p.route.bias != nullptr;
  // (a null bias is zero only on the ranking path; route_row requires one)
  if (wave == 0 && pre_bias) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int e = lane + 64 * i;
      biasv.v[i] = e < E ? gload(p.route.bias + e) : 0.0f;
    }
  }
  // Grouped sigmoid routers with more than 64 experts score in parallel:
  // wave w takes experts 64 w .. 64 w + 63 from its own poll (sigmoid, +
  // bias, its two groups' top-2 sums), then every scoring wave keeps the
  // same groups and writes its experts' keys -- sig_scores' arithmetic per
  // expert and per group, spread over E / 64 waves instead of wave 0 alone.
  const bool par_sig = sig_rank && par_poll;
  const bool grp_lim = p.route.n_group > 1 && p.route.topk_group < p.route.n_group;
  float bias_w = 0.0f, sg_w = 0.0f, v_w = 0.0f;
  if (par_sig && pre_bias && wave * kWave < E) bias_w = gload(p.route.bias + wave * kWave + lane);
  if (par_poll) {
    const int e = wave * kWave + lane;
    if (wave * kWave < E) {
      float a = 0.0f;
      for (unsigned n = 0;; ++n) {
        bool ok = true;
        a = 0.0f;
        if (e < E) {
          unsigned long long part[kMaxNC];
#pragma unroll
          for (int c = 0; c < kMaxNC; ++c)
            if (c < NC) part[c] = dev_load(p.rpart + static_cast<int64_t>(e) * NC + c);
#pragma unroll
          for (int c = 0; c < kMaxNC; ++c) {
            if (c < NC) {
              ok = ok && static_cast<unsigned>(part[c] >> 32) == tag;
              a += __uint_as_float(static_cast<uint32_t>(part[c]));  // chunks in order
            }
          }
        }
        if (__all(ok)) break;
        if (n > p.spin) {
          if (lane == 0) wait_timeout(p);
          break;
        }
      }
      if (e < E) L.keys[e] = __float_as_uint(round_bf16(a));
      if (par_sig) {
        sg_w = sigmoid_abs(round_bf16(a));
        v_w = sg_w + bias_w;
        if (grp_lim) {
          float t1, t2;
          half_top2(v_w, t1, t2);
          if ((lane & 31) == 0) L.route.gsc[2 * wave + (lane >> 5)] = t1 + t2;
        }
      }
    }
    lds_barrier();
  }
  if (par_sig) {
    if (wave * kWave < E) {
      const int e = wave * kWave + lane;
      if (grp_lim) {
        const int ng = p.route.n_group;
        const uint32_t gk = lane < ng ? order_key(L.route.gsc[lane]) : 0u;
        int rank = 0;
        for (int g = 0; g < ng; ++g) {
          const uint32_t o = order_key(L.route.gsc[g]);
          rank += (o > gk || (o == gk && g < lane)) ? 1 : 0;
        }
        const uint64_t keepm = __ballot(lane < ng && rank < p.route.topk_group);
        if (!((keepm >> (e >> 5)) & 1ull)) v_w = 0.0f;
      }
      reinterpret_cast<uint64_t*>(L.keys)[e] =
          static_cast<uint64_t>(order_key(v_w)) << 32 | (0xFFFFFFFFu - static_cast<uint32_t>(e));
      grow[e] = sg_w;
    }
    trace_mark(p, 3);
  } else if (wave == 0) {
    RowVals<P> row;
    if (par_poll) {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        row.v[i] = e < E ? __uint_as_float(L.keys[e]) : -INFINITY;
      }
    } else {
      row = poll_logits<P>(p, p.rpart, NC, tag);
    }
    trace_mark(p, 3);
    if (rank_route) {
      float(&v)[P] = row.v;
      if (rkind == kRouteSoftmaxProbs) {
        // moe_mlp.py:255-266: precise softmax, probabilities rounded to bf16
        const float m = reg_row_max(v, E);
#pragma unroll
        for (int i = 0; i < P; ++i) v[i] = expf(v[i] - m);
        const float sum = reg_row_sum(v, E);
#pragma unroll
        for (int i = 0; i < P; ++i) v[i] = div_to_bf16(v[i], sum);
      }
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        if (e < Epad)
          L.keys[e] = e < E ? ((order_key(v[i]) & 0xFFFF0000u) | (0xFFFFu - static_cast<uint32_t>(e))) : 0u;
      }
      trace_mark(p, 15);
    } else if (sig_rank) {
      sig_scores<P>(p.route, row, pre_bias ? &biasv : nullptr, *(ZMOE_LDS RouteLds*)(&L.route),
                    reinterpret_cast<uint64_t*>(L.keys), grow);
    } else {
      route_row<P>(p.route, row, *(ZMOE_LDS RouteLds*)(&L.route), (ZMOE_LDS float*)grow, pre_bias ? &biasv : nullptr);
      if (lane < Uall * 3) set_unit_e(p, L, lane / 3, lane % 3, lane / 3 < K ? L.route.sel[lane / 3] : -1);
      if (blockIdx.x == 0 && lane < K) {
        if (p.out_idx) gstore(p.out_idx + lane, static_cast<uint32_t>(L.route.sel[lane]));
        if (p.out_w) gstore(p.out_w + lane, L.route.w[lane]);
      }
    }
  }
  lds_barrier();
  trace_mark(p, 16);
  if (rank_route) {
    int i, r;
    uint32_t ki;
    if (Epad == 64) r = rank_in_row<64>(L.keys, i, ki);
    else if (Epad == 128) r = rank_in_row<128>(L.keys, i, ki);
    else r = rank_in_row<256>(L.keys, i, ki);
    if (r >= 0 && i < E && r < K) {
      const uint32_t ok = ki >> 16;
      const uint32_t u16 = (ok & 0x8000u) ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
      L.route.sel[r] = i;
      L.route.sval[r] = __uint_as_float(u16 << 16);
#pragma unroll
      for (int m = 0; m < 3; ++m) set_unit_e(p, L, r, m, i);
    }
    if (has_shared && threadIdx.x == kFThreads - 1) {
#pragma unroll
      for (int m = 0; m < 3; ++m) set_unit_e(p, L, K, m, -1);
    }
    trace_mark(p, 17);
  } else if (sig_rank) {
    int i, r;
    uint64_t kl;
    const uint64_t* k64 = reinterpret_cast<const uint64_t*>(L.keys);
    if (Epad == 64) r = rank_in_row64<64>(k64, i, kl);
    else if (Epad == 128) r = rank_in_row64<128>(k64, i, kl);
    else r = rank_in_row64<256>(k64, i, kl);
    if (r >= 0 && r < K) {
      const uint32_t ki = static_cast<uint32_t>(kl >> 32);
      L.route.sel[r] = i;
      L.route.sval[r] = __uint_as_float((ki & 0x80000000u) ? (ki & 0x7FFFFFFFu) : ~ki);
      L.route.saux[r] = grow[i];
#pragma unroll
      for (int m = 0; m < 3; ++m) set_unit_e(p, L, r, m, i);
    }
    if (has_shared && threadIdx.x == kFThreads - 1) {
#pragma unroll
      for (int m = 0; m < 3; ++m) set_unit_e(p, L, K, m, -1);
    }
  }
  trace_mark(p, 4);
  lds_barrier();
  trace_mark(p, 5);

  // ---------------- D setup: this wave's down-projection loads ----------------
  const int64_t wprD = I >> 3;
  const int64_t pprD = (QMODE == ZMOE_Q_AFFINE) ? (S_I >> p.gshift) : S_I;
  // Hidden 2048 (XR) fits a wave's down items in one batch.  Other shapes
  // keep two batches in registers, both loaded with the gate/up rows; the D
  // loop refills each batch once it is computed, so one is in flight while
  // the other is computed.
  constexpr int DB = XR ? 1 : 2;
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  uint4 wd[DB][kD1D];
  RawParam rd[DB][kD1D];
  int jhl[DB][kD1D], ju[DB][kD1D], jt[DB][kD1D];
  bool jvalid[DB][kD1D];
  // Loads are unconditional so that waits count them: items past the end
  // repeat the previous item's address (a cache hit), or read x if the wave
  // has no down work.
  auto load_down = [&](int base, auto bc) {
    constexpr int b = decltype(bc)::value;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(p.x);
    const void* sp = p.x;
    const void* bp = p.x;
    int64_t poff = 0;
#pragma unroll
    for (int j = 0; j < kD1D; ++j) {
      jhl[b][j] = min(d_hl, max(nrows - 1, 0));
      ju[b][j] = d_u;
      jt[b][j] = d_t;
      jvalid[b][j] = d_g * RPID + rsD < slots;
      if (base + j < n_itemsD) {
        const int s = d_t * LI + liD;
        const int64_t row = h0 + jhl[b][j];
        wp = L.w[2][d_u] + row * wprD + s * 4;
        sp = L.s[2][d_u];
        bp = L.b[2][d_u];
        poff = row * pprD + ((QMODE == ZMOE_Q_AFFINE) ? (s >> p.gshift) : s);
        if (++d_t == TD) {
          d_t = 0;
          ++d_g;
          const int t = d_u + RPID;
          const int q = static_cast<int>(fdiv(static_cast<uint32_t>(t), pl.by_Uall));
          d_hl += q;
          d_u = t - q * Uall;
          d_u = (d_hl >= nrows) ? 0 : d_u;
        }
      }
      wd[b][j] = gload(reinterpret_cast<const uint4*>(wp));
      rd[b][j] = seg_param_load<QMODE>(sp, bp, poff);
    }
  };

  // ---------------- A: gate/up + SwiGLU ----------------
  const int64_t wpr = H >> 3;
  const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S_H >> p.gshift) : S_H;
  if constexpr (XR) {
    // H = 2048: lane l owns x segment l of the row (registers), one segment
    // per lane, one wave-wide load per row.
    const int g0 = a_g0, g1 = a_g1;
    const uint4 x0 = *reinterpret_cast<const uint4*>(xs + ((0 * S_H) + lane) * 4);
    const uint4 x1 = *reinterpret_cast<const uint4*>(xs + ((1 * S_H) + lane) * 4);
    const uint4 x2 = *reinterpret_cast<const uint4*>(xs + ((2 * S_H) + lane) * 4);
    const uint4 x3 = *reinterpret_cast<const uint4*>(xs + ((3 * S_H) + lane) * 4);
    const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[lane] : 0.0f;
    const int pi = (QMODE == ZMOE_Q_AFFINE) ? (lane >> p.gshift) : lane;
    int cu = a_cu;
    int cr = a_cr;
    uint4 wg[kD1A], wu[kD1A];
    RawParam rg[kD1A], ru[kD1A];
    int jrow[kD1A], junit[kD1A];
    auto load_a = [&](int base) {
      const uint32_t *gwp = nullptr, *uwp = nullptr;
      const void *gsp = nullptr, *gbp = nullptr, *usp = nullptr, *ubp = nullptr;
      int64_t poff = 0;
#pragma unroll
      for (int j = 0; j < kD1A; ++j) {
        if (j == 0 || base + j < g1) {
          gwp = L.w[0][cu] + cr * wpr + lane * 4;
          uwp = L.w[1][cu] + cr * wpr + lane * 4;
          gsp = L.s[0][cu];
          gbp = L.b[0][cu];
          usp = L.s[1][cu];
          ubp = L.b[1][cu];
          poff = cr * ppr + pi;
          jrow[j] = cr;
          junit[j] = cu;
          if (++cr == I) {
            cr = 0;
            ++cu;
          }
        } else {
          jrow[j] = jrow[j - 1];
          junit[j] = junit[j - 1];
        }
        wg[j] = gload(reinterpret_cast<const uint4*>(gwp));
        wu[j] = gload(reinterpret_cast<const uint4*>(uwp));
        rg[j] = seg_param_load<QMODE>(gsp, gbp, poff);
        ru[j] = seg_param_load<QMODE>(usp, ubp, poff);
      }
    };
    // gate/up loads first, then the down loads: loads return in order, so
    // the gate/up rows are computed while the down bytes still stream
    if (g0 < g1) load_a(g0);
    load_down(0, B0{});
    if (rank_route && wave == 0) rank_weights(p, L, K);
    if (sig_rank && wave == 0) sig_weights(p, L, K);
    for (int base = g0; base < g1; base += kD1A) {
      if (base != g0) load_a(base);
      float gv[kD1A], uv[kD1A];
#pragma unroll
      for (int j = 0; j < kD1A; ++j) {
        gv[j] = uv[j] = 0.0f;
        if (j > 0 && base + j >= g1) continue;  // wave-uniform: past the range
        float sg, cg, su, cu2;
        seg_param_decode<QMODE>(rg[j], sg, cg);
        seg_param_decode<QMODE>(ru[j], su, cu2);
        gv[j] = wave_sum(seg_accum<QMODE>(0.0f, sg, cg, seg_dot<QMODE>(wg[j], x0, x1, x2, x3, ak), xsum));
        uv[j] = wave_sum(seg_accum<QMODE>(0.0f, su, cu2, seg_dot<QMODE>(wu[j], x0, x1, x2, x3, ak), xsum));
      }
      if (base == g0) trace_mark(p, 6);
      // lane j stores item j (every lane holds every item's sums)
      float gsel = gv[0], usel = uv[0];
      int rsel = jrow[0], usel_u = junit[0];
#pragma unroll
      for (int j = 1; j < kD1A; ++j) {
        if (lane == j) {
          gsel = gv[j];
          usel = uv[j];
          rsel = jrow[j];
          usel_u = junit[j];
        }
      }
      if (lane < kD1A && base + lane < g1)
        dev_store(p.act + static_cast<int64_t>(usel_u) * p.act_stride + rsel,
                  (tag16 << 16) | (wg_dead() ? kBf16NaN : swiglu_bf16(round_bf16(gsel), round_bf16(usel))));
    }
  } else {
    // general H: LH lanes per row (RPI rows per load), T segments per lane,
    // x from LDS
    const int LH = 1 << pl.lLH, RPI = kWave >> pl.lLH;
    const int rs = lane >> pl.lLH, li = lane & (LH - 1);
    const int T = pl.TA;
    const int rgu = pl.rgu;
    const int n_items = (a_g1 - a_g0) * T;
    int cu = a_cu;
    int crg = a_cr;
    int ct = 0;
    // two batches of items in registers: one in flight while the other is
    // computed; loads are unconditional (items past the end repeat the
    // previous item's address, or read x if the wave has no items)
    uint4 wg[2][kD1A], wu[2][kD1A];
    RawParam rg[2][kD1A], ru[2][kD1A];
    int iu[2][kD1A], irow[2][kD1A], it_[2][kD1A];
    auto load_a = [&](int base, auto bc) {
      constexpr int b = decltype(bc)::value;
      const uint32_t* gwp = reinterpret_cast<const uint32_t*>(p.x);
      const uint32_t* uwp = gwp;
      const void *gsp = p.x, *gbp = p.x, *usp = p.x, *ubp = p.x;
      int64_t poff = 0;
#pragma unroll
      for (int j = 0; j < kD1A; ++j) {
        iu[b][j] = cu;
        irow[b][j] = crg * RPI + rs;
        it_[b][j] = ct;
        if (base + j < n_items) {
          const int s = ct * LH + li;
          const int64_t row = irow[b][j];
          gwp = L.w[0][cu] + row * wpr + s * 4;
          uwp = L.w[1][cu] + row * wpr + s * 4;
          gsp = L.s[0][cu];
          gbp = L.b[0][cu];
          usp = L.s[1][cu];
          ubp = L.b[1][cu];
          poff = row * ppr + ((QMODE == ZMOE_Q_AFFINE) ? (s >> p.gshift) : s);
          if (++ct == T) {
            ct = 0;
            if (++crg == rgu) {
              crg = 0;
              ++cu;
            }
          }
        }
        wg[b][j] = gload(reinterpret_cast<const uint4*>(gwp));
        wu[b][j] = gload(reinterpret_cast<const uint4*>(uwp));
        rg[b][j] = seg_param_load<QMODE>(gsp, gbp, poff);
        ru[b][j] = seg_param_load<QMODE>(usp, ubp, poff);
      }
    };
    float ag = 0.0f, au = 0.0f;
    auto compute_a = [&](int base, auto bc) {
      constexpr int b = decltype(bc)::value;
#pragma unroll
      for (int j = 0; j < kD1A; ++j) {
        if (base + j < n_items) {
          const int t = it_[b][j];
          const int s = t * LH + li;
          float sgj, cgj, suj, cuj;
          seg_param_decode<QMODE>(rg[b][j], sgj, cgj);
          seg_param_decode<QMODE>(ru[b][j], suj, cuj);
          const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[s] : 0.0f;
          ag = seg_accum<QMODE>(t == 0 ? 0.0f : ag, sgj, cgj, seg_dot_lds<QMODE>(wg[b][j], xs, S_H, 0, s, ak), xsum);
          au = seg_accum<QMODE>(t == 0 ? 0.0f : au, suj, cuj, seg_dot_lds<QMODE>(wu[b][j], xs, S_H, 0, s, ak), xsum);
          if (base == 0 && j == 0) trace_mark(p, 6);
          if (t == T - 1) {
            const float gv = lanes_sum(ag, LH);
            const float uv = lanes_sum(au, LH);
            if (li == 0)
              dev_store(p.act + static_cast<int64_t>(iu[b][j]) * p.act_stride + irow[b][j],
                        (tag16 << 16) | (wg_dead() ? kBf16NaN : swiglu_bf16(round_bf16(gv), round_bf16(uv))));
          }
        }
      }
    };
    // gate/up loads first, then the down loads (loads return in order)
    load_a(0, B0{});
    load_a(kD1A, B1{});
    load_down(0, B0{});
    load_down(kD1D, B1{});
    if (rank_route && wave == 0) rank_weights(p, L, K);
    if (sig_rank && wave == 0) sig_weights(p, L, K);
    // while another pair of batches follows, compute one and refill it; the
    // last one or two batches are computed without loads behind them, so the
    // act stores are not left waiting on loads past the end
    int base = 0;
    for (; base + 2 * kD1A < n_items; base += 2 * kD1A) {
      compute_a(base, B0{});
      load_a(base + 2 * kD1A, B0{});
      compute_a(base + kD1A, B1{});
      load_a(base + 3 * kD1A, B1{});
    }
    compute_a(base, B0{});
    compute_a(base + kD1A, B1{});
  }
  trace_mark(p, 7);
  // All act rows of the grid are stored once every workgroup has arrived:
  // each wave waits for its own stores (its loads are back already), the
  // workgroup adds 1 to arrival counter g % 32 (one 128-byte line each), and
  // wave 0 polls the 32 counters until each holds  launches x its share of
  // workgroups.  The act read below still verifies every tag.
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  trace_mark(p, 13);
  if (threadIdx.x == 0)
    (void)__hip_atomic_fetch_add((ZMOE_GLOBAL unsigned*)(p.aflag + (blockIdx.x % kD1Ctrs) * kD1CtrStride), 1u,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (wave == 0) {
    const int c = lane;
    const unsigned share = c < kD1Ctrs ? G / kD1Ctrs + (c < G % kD1Ctrs ? 1u : 0u) : 0u;
    const unsigned target = ctag * share;  // modulo 2^32, compared by difference
    unsigned spins = 0;
    for (;;) {
      const bool ok = c >= kD1Ctrs || static_cast<int>(dev_load(p.aflag + c * kD1CtrStride) - target) >= 0;
      if (__all(ok)) break;
      if (++spins > p.spin) {
        if (lane == 0) wait_timeout(p);
        break;
      }
    }
    trace_mark(p, 14);
  }
  lds_barrier();
  trace_mark(p, 8);

  // ---------------- D: down projection ----------------
  stage_rows_lds<QMODE, true>(p, p.act, p.act_stride, Uall, S_I, as, asx, tag16, p.by_S4I, p.by_SI);
  trace_mark(p, 9);
  lds_barrier();
  trace_mark(p, 10);
  float acc = 0.0f;
  // The lane-group width of the row sums is a template constant of the loop
  // (a runtime width costs a branch tree per item).
  auto compute_d = [&](int base, auto bc, auto lic) {
    constexpr int b = decltype(bc)::value;
    constexpr int LIc = decltype(lic)::value;
#pragma unroll
    for (int j = 0; j < kD1D; ++j) {
      if (base + j < n_itemsD) {
        const int u = ju[b][j], t = jt[b][j];
        const int s = t * LIc + liD;
        float sdj, cdj;
        seg_param_decode<QMODE>(rd[b][j], sdj, cdj);
        const float xsum = (QMODE == ZMOE_Q_AFFINE) ? asx[u * S_I + s] : 0.0f;
        acc = seg_accum<QMODE>(t == 0 ? 0.0f : acc, sdj, cdj, seg_dot_lds<QMODE>(wd[b][j], as, S_I, u, s, ak), xsum);
        if (t == TD - 1) {
          const float y = wave_sum_width<LIc>(acc);
          if (liD == 0 && jvalid[b][j]) ybuf[(wave * rpw + jhl[b][j]) * Uall + u] = round_bf16(y);
        }
      }
    }
  };
  auto d_loop = [&](auto lic) {
    if constexpr (XR) {
      for (int base = 0; base < n_itemsD; base += kD1D) {
        if (base > 0) load_down(base, B0{});
        compute_d(base, B0{}, lic);
      }
    } else {
      int base = 0;
      for (; base + 2 * kD1D < n_itemsD; base += 2 * kD1D) {
        compute_d(base, B0{}, lic);
        load_down(base + 2 * kD1D, B0{});
        compute_d(base + kD1D, B1{}, lic);
        load_down(base + 3 * kD1D, B1{});
      }
      compute_d(base, B0{}, lic);
      compute_d(base + kD1D, B1{}, lic);
    }
  };
  switch (LI) {  // LI = gcd(I / 32, 64), as lanes_sum
    case 64: d_loop(std::integral_constant<int, 64>{}); break;
    case 32: d_loop(std::integral_constant<int, 32>{}); break;
    case 16: d_loop(std::integral_constant<int, 16>{}); break;
    case 8: d_loop(std::integral_constant<int, 8>{}); break;
    case 4: d_loop(std::integral_constant<int, 4>{}); break;
    default: d_loop(std::integral_constant<int, 2>{});
  }
  wave_lds_sync();
  trace_mark(p, 11);

  // ---------------- combine (+ shared expert), per wave ----------------
  if (lane < nrows) {
    const float* yr = ybuf + (wave * rpw + lane) * Uall;
    const float* wk = L.route.w;
    float o = round_bf16(combine_one(p.combine_mode, K, [&](int k) { return yr[k]; }, [&](int k) { return wk[k]; }));
    if (has_shared) o = add_nofma(o, yr[K]);
    if (wg_dead()) o = kPoison;
    gstore(p.out + h0 + lane, static_cast<uint16_t>(f32_to_bf16_bits(o)));
  }
  trace_mark(p, 12);
  if (threadIdx.x == 0) {
    dev_store(p.sync + kEpochWord + blockIdx.x, epoch + 1);
    dev_store(p.aflag + kD1CtrEpoch + blockIdx.x, ctag);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static bool d1_enabled() {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("ZMOE_DECODE1");
    on = (e && e[0] == '0') ? 0 : 1;
  }
  return on == 1;
}

// ZMOE_DECODE1_SHARED_EARLY=0: the one-token kernel computes the shared
// expert's gate/up rows with the routed ones, after the routing.
static bool d1_shared_early_enabled() {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("ZMOE_DECODE1_SHARED_EARLY");
    on = (e && e[0] == '0') ? 0 : 1;
  }
  return on == 1;
}

size_t decode1_lds_bytes(const zmoe_layer_desc* d, int grid) {
  const int Uall = d->top_k + (d->shared_inter > 0 ? 1 : 0);
  const int W = grid * kFWaves;
  const int rpw = (d->hidden + W - 1) / W;
  return d1_layout(d->hidden, d->inter, d->n_experts, Uall, rpw).total;
}

bool decode1_supported(const zmoe_layer_desc* d, int grid) {
  if (!d1_enabled()) return false;
  const int LH = gcd_int(d->hidden / 32, kWave);
  const int LI = gcd_int(d->inter / 32, kWave);
  if (d->inter % (kWave / LH) != 0) return false;
  if (d->top_k + 1 > kD1MaxUnits) return false;
  (void)LI;
  return decode1_lds_bytes(d, grid) <= 160 * 1024;
}

template <int QMODE, int P, bool XR>
static int launch_d1_t(hipStream_t st, const FusedParams& fp, size_t lds, int grid) {
  static bool prepared = false;
  const void* fn = reinterpret_cast<const void*>(&k_moe_decode1<QMODE, P, XR>);
  if (!prepared) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    prepared = true;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kFThreads, lds) != hipSuccess || occ < 1)
    return fail(ZMOE_EUNSUPPORTED, "[moe_layer] one-token kernel cannot be resident on every CU");
  hipLaunchKernelGGL((k_moe_decode1<QMODE, P, XR>), dim3(grid), dim3(kFThreads), lds, st, fp);
  return check_launch("moe_layer(one-token launch)");
}

template <int QMODE, bool XR>
static int launch_d1_q(hipStream_t st, const FusedParams& fp, size_t lds, int grid) {
  switch (route_slots(fp.E)) {
    case 1: return launch_d1_t<QMODE, 1, XR>(st, fp, lds, grid);
    case 2: return launch_d1_t<QMODE, 2, XR>(st, fp, lds, grid);
    case 4: return launch_d1_t<QMODE, 4, XR>(st, fp, lds, grid);
    case 8: return launch_d1_t<QMODE, 8, XR>(st, fp, lds, grid);
    default: return launch_d1_t<QMODE, 16, XR>(st, fp, lds, grid);
  }
}

int launch_decode1(hipStream_t st, const zmoe_layer_desc* d, const FusedParams& fp_in, int grid) {
  {
    const int rc = try_decode1x(st, d, fp_in, grid);
    if (rc >= 0) return rc;
  }
  FusedParams fp = fp_in;
  D1Plan& pl = fp.d1;
  const int W = grid * kFWaves;
  const int H = d->hidden, I = d->inter, S_H = H / 32, S_I = I / 32;
  pl.Uall = d->top_k + (d->shared_inter > 0 ? 1 : 0);
  pl.rpw = (H + W - 1) / W;
  const int LH = gcd_int(S_H, kWave), LI = gcd_int(S_I, kWave);
  pl.lLH = 0;
  while ((1 << pl.lLH) < LH) ++pl.lLH;
  pl.lLI = 0;
  while ((1 << pl.lLI) < LI) ++pl.lLI;
  pl.TA = S_H / LH;
  pl.TD = S_I / LI;
  pl.rgu = I / (kWave / LH);
  // the shared expert's gate/up rows before the routing wait (general H)
  pl.shpre = (d->shared_inter > 0 && !(fp.LH == kWave && fp.H == 32 * kWave) && d1_shared_early_enabled()) ? 1 : 0;
  pl.perA = ((pl.shpre ? d->top_k : pl.Uall) * pl.rgu + W - 1) / W;
  pl.by_rgu = make_fastdiv(static_cast<uint32_t>(pl.rgu));
  pl.by_Uall = make_fastdiv(static_cast<uint32_t>(pl.Uall));
  pl.by_NC = make_fastdiv(static_cast<uint32_t>(H / 512));
  for (int m = 0; m < 3; ++m) {
    const int64_t N = (m == 2) ? H : I, Kin = (m == 2) ? I : H;
    const int64_t groups = (d->quant_mode == ZMOE_Q_AFFINE) ? Kin / d->group_size : Kin / 32;
    pl.wst[m] = N * (Kin / 8);
    pl.sst[m] = N * groups * ((d->quant_mode == ZMOE_Q_AFFINE) ? 2 : 1);
  }
  const size_t lds = decode1_lds_bytes(d, grid);
  const bool xr = fp.LH == kWave && fp.H == 32 * kWave;
  if (d->quant_mode == ZMOE_Q_AFFINE)
    return xr ? launch_d1_q<ZMOE_Q_AFFINE, true>(st, fp, lds, grid) : launch_d1_q<ZMOE_Q_AFFINE, false>(st, fp, lds, grid);
  return xr ? launch_d1_q<ZMOE_Q_MXFP4, true>(st, fp, lds, grid) : launch_d1_q<ZMOE_Q_MXFP4, false>(st, fp, lds, grid);
}

}  // namespace zmoe
