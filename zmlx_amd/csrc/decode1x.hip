// XCD-partitioned one-token MoE decode layer (B = 1; the path of
// zmoe_moe_layer for single-token decode, moe_mlp.py:787-1072 patched_call).
//
// MI355X has 8 XCDs of 32 CUs, each XCD with its own L2, and the dispatcher
// deals the workgroups of a launch to the XCDs in turn.  A word that a CU
// stores with an ordinary store stays in its XCD's L2, where device-scope
// loads from the other CUs of the same XCD find it: an exchange inside one
// XCD costs a fraction of one across the chip.  When the layer has exactly 8
// units (top-8 routing and no shared expert, or top-7 plus one) this kernel
// gives the 32 workgroups of XCD x unit x, so that the only exchanges that
// leave an XCD are the 8 unit outputs of each output row.  With 4 units
// (LFM2-8B-A1B: top-4) two XCDs share a unit (R = 2): both compute all of
// its gate/up rows, and XCD x computes output rows of half x % 2.
//
//   R  every XCD computes all router logits: one wave per router row, the
//      chunk sums of k_dense_logits, one tagged word (bf16 | tag << 16) per
//      expert stored into the XCD's own region with an ordinary store;
//   T  every wave polls the XCD's logits, computes the softmax and writes the
//      routing keys to its own LDS copy; thread t ranks expert t / Q (as
//      k_moe_decode1), and the expert of rank x becomes this XCD's unit;
//   A  the XCD's 256 waves compute the unit's gate/up + SwiGLU rows (I / 256
//      each) and store them, tagged, into the XCD's act row; each wave then
//      loads its down-projection items (its gate/up rows have arrived);
//   D  every workgroup stages the act row from L2 (polling its tags) and
//      computes its H / (32 R) output rows of the unit's down projection,
//      stored as tagged words with device-scope stores;
//   C  per chunk of output rows, one workgroup of the XCDs that computed
//      them polls the units' values and writes the k-ordered combine.
//
// The layer shape is a template constant (hidden 2048 on a 256-CU device,
// expert intermediate I_), so the work assignment is folded at compile time.
// Results are bit-identical to k_moe_decode1 and to the kernel sequence: the
// same router chunk order, segment dots, wave sums and combine.
#include "zmoe_decode1.h"
#include "zmoe_xcd.h"

#include <cstdlib>
#include <type_traits>
#include <vector>

namespace zmoe {

// UX units, R XCDs per unit (UX * R <= 8; XCDs past UX * R idle): each
// computes all of its unit's gate/up rows and H / R of its output rows.
template <int I_, int R, int UX_>
struct D1XShape {
  static constexpr int H = kXH, S_H = kXH / 32, NC = kXH / 512;
  static constexpr int S_I = I_ / 32;
  static constexpr int UX = UX_;                      // units
  static_assert(UX * R <= kNX, "units x XCDs per unit");
  static constexpr int HR = H / R;                    // output rows per XCD
  static constexpr int RA = (I_ + kXWX - 1) / kXWX;   // gate/up rows per wave
  static constexpr int RD = HR / kXWX;                // output rows per wave of the XCD
  static constexpr int RW = RD * kFWaves;             // output rows per workgroup
  static constexpr int LI = cgcd(S_I, kWave);         // lanes per down row
  static constexpr int RPID = kWave / LI;             // down rows per load
  static constexpr int TD = S_I / LI;                 // segments per lane and row
  // When a wave's share is below one load's rows, the workgroup's rows go to
  // its last DW waves, RPID each (no lanes load a repeated row), and the
  // other waves stage the act row with no down loads queued ahead of them.
  static constexpr int DRW = RD >= RPID ? RD : RPID;  // rows per down wave
  static constexpr int DW = RW / DRW;                 // down waves per workgroup
  static constexpr int ND = ((DRW + RPID - 1) / RPID) * TD;  // down items per wave
  static_assert(I_ % 32 == 0 && kNX % R == 0 && HR % kXWX == 0 && RW % DRW == 0, "shape");
  static_assert(RA <= 8 && ND <= 8 && DRW * UX <= kWave, "work per wave");
  static_assert(DW == kFWaves || S_I * 4 <= (kFWaves - DW) * kWave, "act staging outside the down waves");
};

struct D1XLayout {
  size_t xs, as, asx, yl, keys, aux, total;
};

__host__ __device__ constexpr D1XLayout d1x_layout(int I) {
  D1XLayout o{};
  size_t off = (sizeof(D1Lds) + 15) & ~static_cast<size_t>(15);
  o.xs = off;
  off += static_cast<size_t>(lds_row_words(kXH / 32)) * 4;
  o.as = off;
  off += static_cast<size_t>(lds_row_words(I / 32)) * 4;
  o.asx = off;
  off += static_cast<size_t>(I / 32) * 4;
  off = (off + 15) & ~static_cast<size_t>(15);
  o.yl = off;
  off += static_cast<size_t>(kFWaves) * kWave * 4;
  o.keys = off;  // one copy of the routing keys per wave (64-bit keys: E <= 128)
  off += static_cast<size_t>(kFWaves) * kD1RankMaxE * 4;
  o.aux = off;   // sigmoid router: one copy of the sigmoids per wave
  off += static_cast<size_t>(kFWaves) * 128 * 4;
  o.total = off;
  return o;
}

// Kernel arguments: everything the kernel reads from its argument block,
// loaded into scalar registers in one batch at the start (an argument read
// first on the critical path costs a scalar-cache miss there).
struct D1XArgs {
  const uint16_t* x;
  uint16_t* out;
  const uint16_t* wr;
  const uint32_t* w[4];   // gate, up, down, and the shared expert's gate (its up/down follow in sh)
  const void* s[3];
  const void* b[3];
  const uint32_t* shw[3];  // shared expert (unit K when top-7 + shared)
  const void* shs[3];
  const void* shb[3];
  int64_t wst[3], sst[3];  // per-expert strides: packed words, scale (= bias) bytes
  unsigned* sync;
  uint32_t* lg;            // [1 + 8][E] logit words (region 1 + x: XCD x)
  uint32_t* act;           // [8][act_stride] act words, row x: XCD x
  uint32_t* xy;            // [8][H] unit outputs
  uint32_t* out_idx;
  float* out_w;
  unsigned long long* trace;
  unsigned* err_host;      // nullable host-visible flag, set when a wait gives up
  unsigned spin;           // polls before a wait gives up
  int E, K, gshift, combine_mode, act_stride;
  int route_kind, norm, w_bf16;
  const float* rbias;      // sigmoid router: per-expert selection bias
  float rscale;            // sigmoid router: routed scaling factor
};

// SIG: the sigmoid router (compiled only for the shapes that use it, so the
// other kernels carry none of its code).
template <int QMODE, int P, int I_, int R, int UX, bool SIG>
__global__ __launch_bounds__(kFThreads) void k_moe_decode1x(D1XArgs a) {
  using S = D1XShape<I_, R, UX>;
  constexpr D1XLayout lay = d1x_layout(I_);
  extern __shared__ __align__(16) unsigned char smem[];
  D1Lds& L = *reinterpret_cast<D1Lds*>(smem);
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem + lay.xs);
  uint32_t* as = reinterpret_cast<uint32_t*>(smem + lay.as);
  float* asx = reinterpret_cast<float*>(smem + lay.asx);
  float* yl = reinterpret_cast<float*>(smem + lay.yl);

  // every argument, in scalar registers before the first use
  const uint16_t* x = a.x;
  const uint16_t* wr = a.wr;
  unsigned* sync = a.sync;
  uint32_t* lg0 = a.lg;
  int E = a.E, K = a.K, gshift = a.gshift;
  ZMOE_PIN(x); ZMOE_PIN(wr); ZMOE_PIN(sync); ZMOE_PIN(lg0); ZMOE_PIN(E); ZMOE_PIN(K); ZMOE_PIN(gshift);
  const uint32_t* mw[3] = {a.w[0], a.w[1], a.w[2]};
  const void* ms[3] = {a.s[0], a.s[1], a.s[2]};
  const void* mb[3] = {a.b[0], a.b[1], a.b[2]};
  const uint32_t* hw[3] = {a.shw[0], a.shw[1], a.shw[2]};
  const void* hs[3] = {a.shs[0], a.shs[1], a.shs[2]};
  const void* hb[3] = {a.shb[0], a.shb[1], a.shb[2]};
  int64_t wst[3] = {a.wst[0], a.wst[1], a.wst[2]};
  int64_t sst[3] = {a.sst[0], a.sst[1], a.sst[2]};
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    ZMOE_PIN(mw[m]); ZMOE_PIN(ms[m]); ZMOE_PIN(mb[m]); ZMOE_PIN(hw[m]); ZMOE_PIN(hs[m]); ZMOE_PIN(hb[m]);
    ZMOE_PIN(wst[m]); ZMOE_PIN(sst[m]);
  }
  uint32_t* act = a.act;
  uint32_t* xy = a.xy;
  uint16_t* out = a.out;
  uint32_t* out_idx = a.out_idx;
  float* out_w = a.out_w;
  unsigned long long* trace = a.trace;
  unsigned* err_host = a.err_host;
  unsigned spin = a.spin;
  ZMOE_PIN(err_host); ZMOE_PIN(spin);
  int cmode = a.combine_mode, act_stride = a.act_stride, rkind = a.route_kind, norm = a.norm, wbf = a.w_bf16;
  const float* rbias = SIG ? a.rbias : nullptr;
  float rscale = SIG ? a.rscale : 1.0f;
  ZMOE_PIN(act); ZMOE_PIN(xy); ZMOE_PIN(out); ZMOE_PIN(out_idx); ZMOE_PIN(out_w); ZMOE_PIN(trace);
  ZMOE_PIN(cmode); ZMOE_PIN(act_stride); ZMOE_PIN(rkind); ZMOE_PIN(norm); ZMOE_PIN(wbf);
  if constexpr (SIG) {
    ZMOE_PIN(rbias); ZMOE_PIN(rscale);
  }

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = __lane_id();
  // the workgroups on physical XCD `xcd` (g, g + 8, g + 16, ...) compute unit
  // ux = xcd / R and its output rows of part xcd % R; gi is the index among
  // them
  const int xcd = xcc_id();
  const int ux = xcd / R, hpart = xcd % R;
  const int gi = blockIdx.x / kNX;
  const int q = gi * kFWaves + wave;  // wave index within the XCD
  const AffineK ak = affine_k();

  // phase stamps of thread 0, kept in registers and stored at the end
  unsigned long long tsr[kTraceSlots];
#pragma unroll
  for (int i = 0; i < kTraceSlots; ++i) tsr[i] = 0;
  auto mark = [&](int i) {
    if (trace) tsr[i] = wall_clock64();
  };
  auto timeout = [&]() { wait_timeout_at(sync, err_host); };
  wg_dead_clear();
  mark(0);
  const unsigned epoch = dev_load(sync + kEpochWord + blockIdx.x);
  const unsigned tag16 = (epoch + 1u) & 0xFFFFu;
  bool dead = false;  // a wait of this thread gave up (later waits give up at once)
  if (UX * R < kNX && ux >= UX) {  // an XCD without a unit: only its launch count advances
    if (threadIdx.x == 0) {
      dev_store(sync + kEpochWord + blockIdx.x, epoch + 1);
      if (trace) gstore(trace + blockIdx.x * kTraceSlots, tsr[0]);
    }
    return;
  }
  // the workgroup that writes the routing outputs (on an XCD with a unit)
  const bool writer = (UX * R == kNX) ? blockIdx.x == 0 : (xcd == 0 && gi == 0);
  // sigmoid router (moe.py:1501-1742, no group limit): selection scores are
  // sigmoid + bias; the bias is loaded before the logits are waited for
  constexpr bool sig = SIG;
  float bv[P];
  if constexpr (SIG) {
#pragma unroll
    for (int i = 0; i < P; ++i) bv[i] = lane + 64 * i < E ? gload(rbias + lane + 64 * i) : 0.0f;
  }

  // ---------------- R: router logits, XCD-local ----------------
  uint32_t* lg = lg0 + E * (1 + xcd);
  {
    // x in registers: lane l holds elements 8 l .. 8 l + 7 of each 512-chunk
    uint4 xv[S::NC];
#pragma unroll
    for (int c = 0; c < S::NC; ++c) xv[c] = gload(reinterpret_cast<const uint4*>(x + c * 512 + lane * 8));
    for (int u = q; u < E; u += kXWX) {
      uint4 wv[S::NC];
#pragma unroll
      for (int c = 0; c < S::NC; ++c)
        wv[c] = gload(reinterpret_cast<const uint4*>(wr + static_cast<int64_t>(u) * kXH + c * 512 + lane * 8));
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < S::NC; ++c) {
        float d = 0.0f;
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[c].x), __builtin_bit_cast(bf16x2_t, xv[c].x), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[c].y), __builtin_bit_cast(bf16x2_t, xv[c].y), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[c].z), __builtin_bit_cast(bf16x2_t, xv[c].z), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[c].w), __builtin_bit_cast(bf16x2_t, xv[c].w), d, false);
        acc += wave_sum(d);  // chunks in order
      }
      // an ordinary store: the word stays in this XCD's L2 for its readers
      if (lane == 0) gstore(lg + u, (tag16 << 16) | f32_to_bf16_bits(acc));
    }
    // wave 0 writes the x tile in stage_rows_lds's layout: item (segment
    // c * 16 + l / 4, quarter l % 4); each lane forms its segment's sum in A
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < S::NC; ++c) {
        const uint4 v = xv[c];
        uint4 o = v;
        if (QMODE == ZMOE_Q_AFFINE) {
          o.x = (v.x & 0xFFFFu) | (v.z << 16);
          o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
          o.z = (v.y & 0xFFFFu) | (v.w << 16);
          o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
        }
        *reinterpret_cast<uint4*>(xs + ((lane & 3) * S::S_H + c * 16 + (lane >> 2)) * 4) = o;
      }
    }
  }
  mark(1);

  // ---------------- T: routing ----------------
  // Every wave polls the logits, computes the softmax and writes the unique
  // keys (bf16 value order, then lower index first) to its own LDS copy;
  // thread t ranks expert t / Q against its wave's copy, so no workgroup
  // barrier sits between the logits and the ranks.
  const int Epad = E <= 64 ? 64 : (E <= 128 ? 128 : 256);
  uint32_t* keys = reinterpret_cast<uint32_t*>(smem + lay.keys) + wave * Epad;
  uint64_t* keys64 = reinterpret_cast<uint64_t*>(smem + lay.keys) + wave * Epad;  // sigmoid router (E <= 128)
  float* aux = reinterpret_cast<float*>(smem + lay.aux) + wave * 128;
  {
    RowVals<P> row;
    for (unsigned n = 0;; ++n) {
      uint32_t wd[P];
      xcd_load_row<P>(lg, E, wd);
      bool ok = true;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        ok = ok && (wd[i] >> 16) == tag16;
        row.v[i] = lane + 64 * i < E ? bf16_bits_to_f32(wd[i] & 0xFFFFu) : -INFINITY;
      }
      if (__all(ok)) break;
      if (n > spin) {
        if (lane == 0) timeout();
        dead = true;
        break;
      }
    }
    mark(3);
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
    if constexpr (SIG) {
      // unique 64-bit keys (score order key << 32 | ~e: value descending,
      // then lower index), the ranking decode1.hip's grouped sigmoid path
      // uses; the sigmoids beside them
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        const float sg = sigmoid_abs(v[i]);
        if (e < Epad) {
          keys64[e] = e < E ? (static_cast<uint64_t>(order_key(sg + bv[i])) << 32 |
                               (0xFFFFFFFFu - static_cast<uint32_t>(e)))
                            : 0ull;
          aux[e] = sg;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        if (e < Epad) keys[e] = e < E ? ((order_key(v[i]) & 0xFFFF0000u) | (0xFFFFu - static_cast<uint32_t>(e))) : 0u;
      }
    }
  }
  wave_lds_sync();
  if constexpr (SIG) {
    int i, r;
    uint64_t kl;
    if (Epad == 64) r = rank_in_row64<64>(keys64, i, kl);
    else r = rank_in_row64<128>(keys64, i, kl);
    if (r >= 0 && i < E && r < K) {
      L.route.sel[r] = i;
      L.route.saux[r] = aux[i];
    }
  } else {
    int i, r;
    uint32_t ki;
    if (Epad == 64) r = rank_in_row<64>(keys, i, ki);
    else if (Epad == 128) r = rank_in_row<128>(keys, i, ki);
    else r = rank_in_row<256>(keys, i, ki);
    if (r >= 0 && i < E && r < K) {
      const uint32_t ok = ki >> 16;
      const uint32_t u16 = (ok & 0x8000u) ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
      L.route.sel[r] = i;
      L.route.sval[r] = __uint_as_float(u16 << 16);
    }
  }
  mark(4);
  lds_barrier();
  mark(5);

  // ---------------- A: gate/up + SwiGLU of unit xcd ----------------
  // this XCD's unit: the expert of rank ux, or the shared expert (unit K).
  // Clamped: after a wait gave up, the waves may have ranked different
  // (stale) logits, and then no thread need have written rank ux.
  const int ue = ux < K ? min(max(__builtin_amdgcn_readfirstlane(L.route.sel[ux]), 0), E - 1) : -1;
  const uint32_t* uw[3];
  const void* us[3];
  const void* ub[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    uw[m] = ue >= 0 ? mw[m] + ue * wst[m] : hw[m];
    us[m] = ue >= 0 ? static_cast<const void*>(static_cast<const char*>(ms[m]) + ue * sst[m]) : hs[m];
    ub[m] = ue >= 0 ? (mb[m] ? static_cast<const void*>(static_cast<const char*>(mb[m]) + ue * sst[m]) : nullptr) : hb[m];
  }
  // down-projection items: lane group rs (of RPID) takes row h0 + g * RPID +
  // rs, lane li of it segments t * LI + li
  const int dw = wave - (kFWaves - S::DW);  // index among the down waves, < 0: none
  const bool dwave = dw >= 0;
  const int h0 = hpart * S::HR + gi * S::RW + (dwave ? dw : 0) * S::DRW;
  const int rsD = lane / S::LI, liD = lane % S::LI;
  constexpr int64_t wprD = I_ / 8;
  const int pprD = (QMODE == ZMOE_Q_AFFINE) ? (S::S_I >> gshift) : S::S_I;
  uint4 wd[S::ND];
  RawParam rd[S::ND];
  auto load_d = [&]() {
#pragma unroll
    for (int j = 0; j < S::ND; ++j) {
      const int g = j / S::TD, t = j % S::TD;
      const int row = h0 + min(g * S::RPID + rsD, S::DRW - 1);
      const int sgm = t * S::LI + liD;
      wd[j] = gload(reinterpret_cast<const uint4*>(uw[2] + row * wprD + sgm * 4));
      rd[j] = seg_param_load<QMODE>(us[2], ub[2], row * pprD + ((QMODE == ZMOE_Q_AFFINE) ? (sgm >> gshift) : sgm));
    }
  };
  // The gate/up rows are loaded first and alone; each wave loads its
  // down-projection items once its gate/up rows have arrived, so the act
  // rows are not queued behind down-projection bytes.
  constexpr int64_t wpr = kXH / 8;
  const int ppr = (QMODE == ZMOE_Q_AFFINE) ? (S::S_H >> gshift) : S::S_H;
  const int pi = (QMODE == ZMOE_Q_AFFINE) ? (lane >> gshift) : lane;
  const int a_r0 = q * S::RA;  // gate/up rows [a_r0, a_r0 + RA)
  uint4 wg[S::RA], wu[S::RA];
  RawParam rg[S::RA], ru[S::RA];
#pragma unroll
  for (int j = 0; j < S::RA; ++j) {
    const int r = min(a_r0 + j, I_ - 1);  // past the last row: repeat it
    wg[j] = gload(reinterpret_cast<const uint4*>(uw[0] + r * wpr + lane * 4));
    wu[j] = gload(reinterpret_cast<const uint4*>(uw[1] + r * wpr + lane * 4));
    rg[j] = seg_param_load<QMODE>(us[0], ub[0], r * ppr + pi);
    ru[j] = seg_param_load<QMODE>(us[1], ub[1], r * ppr + pi);
  }
  mark(13);
  // gate weights of the ranked winners (wave 0, lane r = winner r), for the
  // combine, and the routing outputs of workgroup 0
  if (wave == 0) {
    const float val = lane < K ? (sig ? L.route.saux[lane] : L.route.sval[lane]) : 0.0f;
    float w;
    if constexpr (SIG) {
      // the sigmoids normalised in selection order, scaled (decode1.hip
      // sig_weights, route_row's weights)
      const float sum = ordered_lane_sum(val, K);
      w = val / sum;
      if (rscale != 1.0f) w = w * rscale;
    } else if (rkind == kRouteSoftmaxProbs) {
      const float sb = round_bf16(ordered_lane_sum(val, K));
      w = norm ? div_to_bf16(val, sb) : val;
    } else {
      // moe.topk_gating_softmax renorm path (moe.py:1239-1396)
      const float m = readlane_f(val, 0);
      const float ex = expf(val - m);
      const float sum = ordered_lane_sum(ex, K);
      w = ex / sum;
      if (wbf) w = round_bf16(w);
    }
    if (lane < K) {
      L.route.w[lane] = w;
      if (writer) {
        if (out_idx) gstore(out_idx + lane, static_cast<uint32_t>(L.route.sel[lane]));
        if (out_w) gstore(out_w + lane, w);
      }
    }
  }
  uint32_t actw;
  {
    const uint4 x0 = *reinterpret_cast<const uint4*>(xs + ((0 * S::S_H) + lane) * 4);
    const uint4 x1 = *reinterpret_cast<const uint4*>(xs + ((1 * S::S_H) + lane) * 4);
    const uint4 x2 = *reinterpret_cast<const uint4*>(xs + ((2 * S::S_H) + lane) * 4);
    const uint4 x3 = *reinterpret_cast<const uint4*>(xs + ((3 * S::S_H) + lane) * 4);
    // sum of the lane's x segment, in stage_rows_lds's order
    float xsum = 0.0f;
    if (QMODE == ZMOE_Q_AFFINE) {
      const uint4 xq[4] = {x0, x1, x2, x3};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint4 o = xq[w];
        xsum += bf16_bits_to_f32(o.x & 0xFFFFu) + bf16_bits_to_f32(o.y & 0xFFFFu);
        xsum += bf16_bits_to_f32(o.z & 0xFFFFu) + bf16_bits_to_f32(o.w & 0xFFFFu);
        xsum += bf16_bits_to_f32(o.x >> 16) + bf16_bits_to_f32(o.y >> 16);
        xsum += bf16_bits_to_f32(o.z >> 16) + bf16_bits_to_f32(o.w >> 16);
      }
    }
    float gsel = 0.0f, usel = 0.0f;
#pragma unroll
    for (int j = 0; j < S::RA; ++j) {
      float sg, cg, su, cu2;
      seg_param_decode<QMODE>(rg[j], sg, cg);
      seg_param_decode<QMODE>(ru[j], su, cu2);
      const float gv = wave_sum(seg_accum<QMODE>(0.0f, sg, cg, seg_dot<QMODE>(wg[j], x0, x1, x2, x3, ak), xsum));
      const float uv = wave_sum(seg_accum<QMODE>(0.0f, su, cu2, seg_dot<QMODE>(wu[j], x0, x1, x2, x3, ak), xsum));
      if (lane == j) {
        gsel = gv;
        usel = uv;
      }
    }
    actw = (tag16 << 16) | (wg_dead() ? kBf16NaN : swiglu_bf16(round_bf16(gsel), round_bf16(usel)));
  }
  mark(6);
  // the act words leave before the down-projection loads of the same wave
  // (LFM2 shape: act row staged 0.6 us earlier)
  if (lane < S::RA && a_r0 + lane < I_) gstore(act + static_cast<int64_t>(xcd) * act_stride + a_r0 + lane, actw);
  if (dwave) load_d();
  mark(7);

  // ---------------- D: the unit's act row from L2, down projection ----------------
  // stage the act row in LDS in stage_rows_lds's layout: item i = (segment
  // i / 4, quarter i % 4), 8 tagged words, polled until every tag is current
  {
    constexpr int NI = S::S_I * 4;
    static_assert(NI <= kFThreads, "one staged item per thread");
    if (threadIdx.x < NI) {
      const int i = threadIdx.x;
      const uint32_t* src = act + static_cast<int64_t>(xcd) * act_stride + i * 8;
      const uint32_t want = tag16 << 16;
      auto current = [&](const uint4& c) {
        return ((c.x & 0xFFFF0000u) == want) && ((c.y & 0xFFFF0000u) == want) && ((c.z & 0xFFFF0000u) == want) &&
               ((c.w & 0xFFFF0000u) == want);
      };
      uint4 w0, w1;
      for (unsigned spins = 0;; ++spins) {
        xcd_load_2x128(src, w0, w1);
        if ((current(w0) && current(w1)) || dead) break;
        if (spins > spin) {
          timeout();
          dead = true;
          break;
        }
      }
      auto pair = [](uint32_t lo, uint32_t hi) { return (lo & 0xFFFFu) | (hi << 16); };
      const uint4 v = make_uint4(pair(w0.x, w0.y), pair(w0.z, w0.w), pair(w1.x, w1.y), pair(w1.z, w1.w));
      uint4 o = v;
      if (QMODE == ZMOE_Q_AFFINE) {
        o.x = (v.x & 0xFFFFu) | (v.z << 16);
        o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
        o.z = (v.y & 0xFFFFu) | (v.w << 16);
        o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
      }
      *reinterpret_cast<uint4*>(as + ((i & 3) * S::S_I + (i >> 2)) * 4) = o;
    }
    if (QMODE == ZMOE_Q_AFFINE) {
      lds_barrier();
      if (threadIdx.x < S::S_I) {
        const int sg = threadIdx.x;
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint4 o = *reinterpret_cast<const uint4*>(as + (w * S::S_I + sg) * 4);
          acc += bf16_bits_to_f32(o.x & 0xFFFFu) + bf16_bits_to_f32(o.y & 0xFFFFu);
          acc += bf16_bits_to_f32(o.z & 0xFFFFu) + bf16_bits_to_f32(o.w & 0xFFFFu);
          acc += bf16_bits_to_f32(o.x >> 16) + bf16_bits_to_f32(o.y >> 16);
          acc += bf16_bits_to_f32(o.z >> 16) + bf16_bits_to_f32(o.w >> 16);
        }
        asx[sg] = acc;
      }
    }
  }
  mark(8);
  lds_barrier();
  mark(9);
  if (dwave) {
    float ysum[S::ND];
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < S::ND; ++j) {
      const int t = j % S::TD;
      const int sgm = t * S::LI + liD;
      float sdj, cdj;
      seg_param_decode<QMODE>(rd[j], sdj, cdj);
      const float xsum = (QMODE == ZMOE_Q_AFFINE) ? asx[sgm] : 0.0f;
      acc = seg_accum<QMODE>(t == 0 ? 0.0f : acc, sdj, cdj, seg_dot_lds<QMODE>(wd[j], as, S::S_I, 0, sgm, ak), xsum);
      ysum[j] = (t == S::TD - 1) ? wave_sum_width<S::LI>(acc) : 0.0f;
    }
    mark(11);
#pragma unroll
    for (int j = 0; j < S::ND; ++j) {
      const int g = j / S::TD, t = j % S::TD;
      const int hl = g * S::RPID + rsD;
      if (t == S::TD - 1 && liD == 0 && hl < S::DRW)
        dev_store(xy + static_cast<int64_t>(xcd) * kXH + h0 + hl,
                  (tag16 << 16) | (wg_dead() ? kBf16NaN : f32_to_bf16_bits(ysum[j])));
    }
  }
  mark(10);

  // ---------------- C: k-ordered combine of the chunk, on one XCD ----------------
  // chunk = the output rows of the workgroups with index gi on the XCDs of
  // part hpart (one per unit); the one of unit gi % UX combines them, each
  // down wave its own DRW rows: lane k * DRW + r polls unit k's value of row
  // h0 + r, stored by XCD k * R + hpart.
  if (ux == gi % S::UX && dwave) {
    const int k = lane / S::DRW, r = lane % S::DRW;
    const bool mine = k < S::UX;
    const uint32_t* src = xy + static_cast<int64_t>((mine ? k : 0) * R + hpart) * kXH + h0 + r;
    uint32_t v = 0;
    for (unsigned spins = 0;; ++spins) {
      v = dev_load(src);
      if (__all(!mine || (v >> 16) == tag16) || dead) break;
      if (spins > spin) {
        if (lane == 0) timeout();
        break;
      }
    }
    float* yw = yl + wave * kWave;
    if (mine) yw[r * S::UX + k] = bf16_bits_to_f32(v & 0xFFFFu);
    wave_lds_sync();
    if (lane < S::DRW) {
      const float* yr = yw + lane * S::UX;
      const float* wk = L.route.w;
      float o = round_bf16(combine_one(cmode, K, [&](int kk) { return yr[kk]; }, [&](int kk) { return wk[kk]; }));
      if (K < S::UX) o = add_nofma(o, yr[K]);
      if (wg_dead()) o = kPoison;
      gstore(out + h0 + lane, static_cast<uint16_t>(f32_to_bf16_bits(o)));
    }
  }
  mark(12);
  if (threadIdx.x == 0) dev_store(sync + kEpochWord + blockIdx.x, epoch + 1);
  if (trace) {
    // the down-projection and combine stamps (10-12) come from the first
    // down wave, the others from thread 0
    const bool t0 = threadIdx.x == 0, td = dw == 0 && lane == 0;
#pragma unroll
    for (int i = 0; i < kTraceSlots; ++i) {
      const bool dslot = i == 10 || i == 11 || i == 12;
      if (tsr[i] && (dslot ? td : t0)) gstore(trace + blockIdx.x * kTraceSlots + i, tsr[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static bool d1x_enabled() {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("ZMOE_DECODE1X");
    on = (e && e[0] == '0') ? 0 : 1;
  }
  return on == 1;
}

// XCDs per unit of a layer with Uall units: 8 units: 1; 4 units: 2; 5 to 7
// units: 1 (the other XCDs idle); else 0.
static int d1x_share(int Uall) {
  if (Uall == kNX / 2) return 2;
  return (Uall >= 5 && Uall <= kNX) ? 1 : 0;
}

// Shapes with a compiled kernel (expert intermediate, XCDs per unit, units,
// router): Qwen3-30B-A3B (768, 1, 8), OLMoE (1024, 1, 8), LFM2-8B-A1B (1792,
// 2, 4), ranked softmax or top-k logits; GLM-4.7-Flash-like (1536, 1, 5: 4
// routed + 1 shared), sigmoid router.
static bool d1x_inter_ok(int I, int R, int UX, bool sig) {
  if (R == 1 && UX == kNX) return !sig && (I == 768 || I == 1024);
  if (R == 2 && UX == 4) return !sig && I == 1792;
  return R == 1 && UX == 5 && I == 1536 && sig;
}

size_t xcd_rpart_bytes(const zmoe_layer_desc* d) { return static_cast<size_t>(kNX + 1) * d->n_experts * 4; }
size_t xcd_xy_bytes(const zmoe_layer_desc* d) { return static_cast<size_t>(kNX) * d->hidden * 4; }

__global__ void k_xcc_probe(unsigned* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = static_cast<unsigned>(xcc_id());
}

// Whether the workgroups of a G-workgroup launch are dealt to the 8 XCDs in
// turn (workgroup g on XCD (s + g) % 8 for some s) on the current device:
// probed once per device with a small kernel whose result is copied back
// (scratch: G words of device memory).  While a stream is being captured
// nothing can be copied back, so an unprobed device counts as "no" (the layer
// then runs k_moe_decode1) until a call outside capture.
static int g_xcd_rr[64];

bool xcd_round_robin(hipStream_t st, unsigned* scratch, int G) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (g_xcd_rr[dev]) return g_xcd_rr[dev] == 1;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  hipLaunchKernelGGL(k_xcc_probe, dim3(G), dim3(kFThreads), 0, st, scratch);
  std::vector<unsigned> h(G, ~0u);
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(h.data(), scratch, static_cast<size_t>(G) * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    g_xcd_rr[dev] = 2;
    return false;
  }
  bool ok = true;
  for (int g = 0; g < G; ++g) ok = ok && h[g] == (h[0] + static_cast<unsigned>(g)) % kNX;
  g_xcd_rr[dev] = ok ? 1 : 2;
  return ok;
}

static size_t d1x_lds_bytes(int I) {
  const size_t need = d1x_layout(I).total;
  // at least 96 KiB: one workgroup per CU, so the 32 workgroups of an XCD
  // sit on its 32 CUs
  return need > 96 * 1024 ? need : 96 * 1024;
}

static bool d1x_shape_ok(const zmoe_layer_desc* d, int G) {
  if (!d1x_enabled() || G != kXG) return false;
  const int Uall = d->top_k + (d->shared_inter > 0 ? 1 : 0);
  const int R = d1x_share(Uall);
  if (R == 0 || d->top_k > kMaxTopK) return false;
  if (d->shared_inter > 0 && d->shared_inter != d->inter) return false;
  const bool rank_route = d->router_kind == ZMOE_ROUTER_SOFTMAX_PROBS ||
                          (d->router_kind == ZMOE_ROUTER_TOPK_LOGITS && d->router_bias == nullptr && d->norm_topk_prob);
  // the sigmoid router without a group limit, ranked over 64-bit keys (E <= 128)
  const bool sig_route = d->router_kind == ZMOE_ROUTER_SIGMOID_GROUPED && d->router_bias != nullptr &&
                         (d->n_group <= 1 || d->topk_group >= d->n_group) && d->n_experts <= 128;
  if (!(rank_route || sig_route) || d->n_experts > kD1RankMaxE || d->n_experts > kXWX) return false;
  if (d->hidden != kXH || !d1x_inter_ok(d->inter, R, Uall, sig_route)) return false;
  return d1x_lds_bytes(d->inter) <= 160 * 1024;
}

template <int QMODE, int P, int I_, int R, int UX, bool SIG>
static int launch_d1x_t(hipStream_t st, const D1XArgs& a) {
  static bool prepared = false;
  const void* fn = reinterpret_cast<const void*>(&k_moe_decode1x<QMODE, P, I_, R, UX, SIG>);
  const size_t lds = d1x_lds_bytes(I_);
  if (!prepared) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    prepared = true;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kFThreads, lds) != hipSuccess || occ < 1)
    return fail(ZMOE_EUNSUPPORTED, "[moe_layer] XCD-partitioned kernel cannot be resident on every CU");
  hipLaunchKernelGGL((k_moe_decode1x<QMODE, P, I_, R, UX, SIG>), dim3(kXG), dim3(kFThreads), lds, st, a);
  return check_launch("moe_layer(XCD-partitioned one-token launch)");
}

template <int QMODE, int I_, int R, int UX, bool SIG>
static int launch_d1x_p(hipStream_t st, const D1XArgs& a) {
  switch (route_slots(a.E)) {
    case 1: return launch_d1x_t<QMODE, 1, I_, R, UX, SIG>(st, a);
    case 2: return launch_d1x_t<QMODE, 2, I_, R, UX, SIG>(st, a);
    default:
      if constexpr (SIG) return fail(ZMOE_EUNSUPPORTED, "[moe_layer] XCD-partitioned sigmoid routing: E <= 128");
      else return launch_d1x_t<QMODE, 4, I_, R, UX, SIG>(st, a);
  }
}

template <int QMODE>
static int launch_d1x_q(hipStream_t st, const D1XArgs& a, int I) {
  if (I == 1792) return launch_d1x_p<QMODE, 1792, 2, 4, false>(st, a);
  if (I == 1536) return launch_d1x_p<QMODE, 1536, 1, 5, true>(st, a);
  return I == 768 ? launch_d1x_p<QMODE, 768, 1, kNX, false>(st, a) : launch_d1x_p<QMODE, 1024, 1, kNX, false>(st, a);
}

int try_decode1x(hipStream_t st, const zmoe_layer_desc* d, const FusedParams& fp, int grid) {
  if (!d1x_shape_ok(d, grid) || fp.xy == nullptr) return -1;
  if (!xcd_round_robin(st, fp.xy, grid)) return -1;
  D1XArgs a{};
  a.x = fp.x;
  a.out = fp.out;
  a.wr = fp.wr;
  for (int m = 0; m < 3; ++m) {
    a.w[m] = fp.w[m];
    a.s[m] = fp.s[m];
    a.b[m] = fp.b[m];
    a.shw[m] = fp.w[3 + m];
    a.shs[m] = fp.s[3 + m];
    a.shb[m] = fp.b[3 + m];
    const int64_t N = (m == 2) ? d->hidden : d->inter, Kin = (m == 2) ? d->inter : d->hidden;
    const int64_t groups = (d->quant_mode == ZMOE_Q_AFFINE) ? Kin / d->group_size : Kin / 32;
    a.wst[m] = N * (Kin / 8);
    a.sst[m] = N * groups * ((d->quant_mode == ZMOE_Q_AFFINE) ? 2 : 1);
  }
  a.sync = fp.sync;
  a.lg = reinterpret_cast<uint32_t*>(fp.rpart);
  a.act = fp.act;
  a.xy = fp.xy;
  a.out_idx = fp.out_idx;
  a.out_w = fp.out_w;
  a.trace = fp.trace;
  a.err_host = fp.err_host;
  a.spin = d->spin_limit > 0 ? static_cast<unsigned>(d->spin_limit) : kXSpinLimit;
  a.E = fp.E;
  a.K = fp.K;
  a.gshift = fp.gshift;
  a.combine_mode = fp.combine_mode;
  a.act_stride = fp.act_stride;
  a.route_kind = fp.route.kind;
  a.norm = fp.route.norm;
  a.w_bf16 = fp.route.w_bf16;
  a.rbias = fp.route.bias;
  a.rscale = fp.route.scale;
  if (d->quant_mode == ZMOE_Q_AFFINE) return launch_d1x_q<ZMOE_Q_AFFINE>(st, a, d->inter);
  return launch_d1x_q<ZMOE_Q_MXFP4>(st, a, d->inter);
}

}  // namespace zmoe
