// Single-launch MoE decode layer (the fused path of zmoe_moe_layer).
//
// One persistent grid of G = (#CUs) workgroups x 8 waves, every workgroup
// resident at once, runs the whole block:
//
//   R  router projection: the E x (H/512) (row, 1 KiB chunk) units are
//      spread over all waves; partial dots go to the workspace; meanwhile
//      x is staged in LDS.
//   T  routing: every workgroup waits for the partials, reduces them in a
//      fixed order and routes each token (wave b <-> token b) -- redundantly,
//      which is cheaper than another grid-wide exchange -- then gives the
//      selected experts (plus the shared expert) unit slots.
//   A  gate/up + SwiGLU: rows of the units are spread over all waves; act
//      rows go to the workspace.  The waves' first batch of down-projection
//      weight loads is issued together with the gate/up loads.
//   D  down projection: each workgroup waits for the act rows; each wave
//      owns output rows h for all units, so the k-ordered combine and the
//      shared-expert add happen in-workgroup and each output is written once.
//
// Cross-workgroup data carries its own readiness: every router partial and
// every act element is stored together with the launch's generation tag in
// one device-scope atomic word (f32 | tag<<32, bf16 | tag<<16), and readers
// poll until every tag they need is current.  There is no grid barrier: a
// reader waits exactly for the data it consumes, and writers never wait for
// their stores.  Each element is written once per launch and launches on a
// stream do not overlap, so a current tag proves the value.  The tag is
// 1 + the number of launches this workgroup completed on the workspace (kept
// in the workspace, one word per workgroup; every workgroup runs every
// launch, so all agree).  Every wait is bounded (on timeout: sticky error
// word, continue), so the grid always drains.
//
// Code size matters here: the kernel runs each phase once per wave, so it is
// written with rolled loops (per-token accumulators live in LDS) to stay
// within the instruction cache; one-token decode at H = 2048 has a
// register-resident fast path.  The arithmetic is the multi-kernel path's
// (same dot products, reduction trees, routing code and combine): results
// are bit-identical to it.
#include "zmoe_fused.h"

namespace zmoe {

struct UnitPtr {
  const uint32_t* w;
  const void* s;
  const void* b;
};

// Weights of unit u for matrix m (0 gate, 1 up, 2 down): routed expert
// ulist[u] or, for u == nunits, the shared expert.
template <int QMODE>
__device__ __forceinline__ UnitPtr unit_ptr(const FusedParams& p, const FusedLds& L, int u, int m) {
  UnitPtr r;
  if (u < L.nunits) {
    const int64_t e = L.ulist[u];
    const int64_t N = (m == 2) ? p.H : p.I;
    const int64_t Kin = (m == 2) ? p.I : p.H;
    const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? ((Kin >> 5) >> p.gshift) : (Kin >> 5);
    r.w = p.w[m] + e * N * (Kin >> 3);
    r.s = static_cast<const char*>(p.s[m]) + e * N * ppr * ((QMODE == ZMOE_Q_AFFINE) ? 2 : 1);
    r.b = (QMODE == ZMOE_Q_AFFINE) ? static_cast<const void*>(static_cast<const char*>(p.b[m]) + e * N * ppr * 2)
                                   : nullptr;
  } else {
    r.w = p.w[3 + m];
    r.s = p.s[3 + m];
    r.b = p.b[3 + m];
  }
  return r;
}

template <int QMODE, int P>
__global__ __launch_bounds__(kFThreads) void k_moe_decode(FusedParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  FusedLds& L = *reinterpret_cast<FusedLds*>(smem);
  wg_dead_clear();
  unsigned char* big = smem + ((sizeof(FusedLds) + 15) & ~static_cast<size_t>(15));

  const int wave = threadIdx.x / kWave;
  const int lane = __lane_id();
  const int G = gridDim.x;
  const int W = G * kFWaves;
  const int gw = blockIdx.x * kFWaves + wave;
  const int B = p.B;
  const int E = p.E;
  const int NC = p.H >> 9;
  const int S_H = p.H >> 5, S_I = p.I >> 5;
  const AffineK ak = affine_k();
  const bool has_shared = p.Is > 0;
  trace_mark(p, 0);
  if (p.trace && threadIdx.x == 0) gstore(p.trace + blockIdx.x * kTraceSlots + 13, static_cast<unsigned long long>(clock64()));
  // launches this workgroup completed before (written by itself only)
  const unsigned epoch = dev_load(p.sync + kEpochWord + blockIdx.x);
  const unsigned tag = epoch + 1u;
  const unsigned tag16 = tag & 0xFFFFu;

  // phase R..A LDS: x tile, x sums, grouped-router scratch, accumulators
  uint32_t* xs = reinterpret_cast<uint32_t*>(big);
  float* sx = reinterpret_cast<float*>(xs + static_cast<size_t>(B) * lds_row_words(S_H));
  float* rv = sx + static_cast<size_t>(B) * S_H;    // [B][E]
  float* accA = rv + static_cast<size_t>(B) * E;    // [waves][2][B][64]

  // ---------------- phase R: router partials ----------------
  for (int u = gw; u < E * NC; u += W) {
    const int e = u / NC, c = u - e * NC;
    const uint4 wv = gload(reinterpret_cast<const uint4*>(p.wr + static_cast<int64_t>(e) * p.H + c * 512 + lane * 8));
    for (int b = 0; b < B; ++b) {
      const uint4 xv = gload(reinterpret_cast<const uint4*>(p.x + static_cast<int64_t>(b) * p.H + c * 512 + lane * 8));
      float a = 0.0f;
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.x), __builtin_bit_cast(bf16x2_t, xv.x), a, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.y), __builtin_bit_cast(bf16x2_t, xv.y), a, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.z), __builtin_bit_cast(bf16x2_t, xv.z), a, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.w), __builtin_bit_cast(bf16x2_t, xv.w), a, false);
      a = wave_sum(a);
      if (lane == 0)
        dev_store(p.rpart + (static_cast<int64_t>(b) * E + e) * NC + c,
                  (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(a));
    }
  }
  stage_rows_lds<QMODE, false>(p, p.x, p.H, B, S_H, xs, sx, 0u, p.by_S4H, p.by_SH);
  trace_mark(p, 1);
  lds_barrier();
  trace_mark(p, 2);

  // ---------------- phase T: routing (wave b <-> token b) ----------------
  if (wave < B) {
    const int b = wave;
    const RowVals<P> row = poll_logits<P>(p, p.rpart + static_cast<int64_t>(b) * E * NC, NC, tag);
    trace_mark(p, 3);
    route_row<P>(p.route, row, *(ZMOE_LDS RouteLds*)(&L.route[b]), (ZMOE_LDS float*)(rv + static_cast<size_t>(b) * E));
    trace_mark(p, 4);
    if (blockIdx.x == 0 && lane < p.K) {
      if (p.out_idx) gstore(p.out_idx + b * p.K + lane, static_cast<uint32_t>(L.route[b].sel[lane]));
      if (p.out_w) gstore(p.out_w + b * p.K + lane, L.route[b].w[lane]);
    }
  }
  const int K = p.K;
  const int npairs = B * K;
  if (B == 1) {
    // one token: unit r is the r-th selected expert (each expert once)
    if (wave == 0) {
      if (lane < K) {
        L.ulist[lane] = L.route[0].sel[lane];
        L.ucount[lane] = 1;
        L.upairs[lane][0] = lane;
      }
      if (lane == 0) {
        L.nunits = K;
        if (has_shared) {
          L.ucount[K] = 1;
          L.upairs[K][0] = K;
        }
      }
    }
    __syncthreads();
  } else {
    for (int e = threadIdx.x; e < E; e += blockDim.x) L.slot_of[e] = -1;
    __syncthreads();
    if (threadIdx.x < npairs) L.slot_of[L.route[threadIdx.x / K].sel[threadIdx.x % K]] = 0;
    __syncthreads();
    if (wave == 0) {  // unit slots in expert order
      int base = 0;
      for (int e0 = 0; e0 < E; e0 += kWave) {
        const int e = e0 + lane;
        const bool f = e < E && L.slot_of[e] == 0;
        const uint64_t m = __ballot(f);
        if (f) {
          const int pos = base + __popcll(m & lanes_below_mask(lane));
          L.slot_of[e] = pos;
          L.ulist[pos] = e;
          L.ucount[pos] = 0;
        }
        base += __popcll(m);
      }
      if (lane == 0) {
        L.nunits = base;
        if (has_shared) L.ucount[base] = B;
      }
    }
    __syncthreads();
    if (threadIdx.x < npairs) {
      const int q = threadIdx.x;
      const int u = L.slot_of[L.route[q / K].sel[q % K]];
      L.upairs[u][atomicAdd(&L.ucount[u], 1)] = q;
    }
    if (has_shared && threadIdx.x < B) L.upairs[L.nunits][threadIdx.x] = npairs + threadIdx.x;
    __syncthreads();
  }
  const int U = L.nunits;
  const int Uall = U + (has_shared ? 1 : 0);
  trace_mark(p, 5);

  // ---------------- phase D setup ----------------
  // The first batch of down-projection weight loads is issued during phase A,
  // once the wave's gate/up data has arrived.
  // This wave owns output rows [h0, h0 + nrows); slot = (row, unit) with the
  // unit fastest; RPID slots per load instruction, lane group rsD.
  const int LI = p.LI, RPID = kWave / LI;
  const int rsD = lane / LI, liD = lane & (LI - 1);
  const int TD = S_I / LI;
  const int rows_per_wave = (p.H + W - 1) / W;
  const int h0 = gw * rows_per_wave;
  const int nrows = max(0, min(p.H, h0 + rows_per_wave) - h0);
  const int slots = nrows * Uall;
  const int n_groups = (slots + RPID - 1) / RPID;
  const int n_itemsD = n_groups * TD;
  const int64_t wprD = p.I >> 3;
  const int64_t pprD = (QMODE == ZMOE_Q_AFFINE) ? (S_I >> p.gshift) : S_I;
  // per-lane slot cursor (row hl, unit uu) and segment cursor (wave-uniform)
  int d_hl = rsD / max(Uall, 1), d_u = rsD - d_hl * Uall, d_t = 0, d_g = 0;
  uint4 wd[kChunkD];
  RawParam rd[kChunkD];
  int jhl[kChunkD], ju[kChunkD], jt[kChunkD], jvalid[kChunkD];
  // Loads are unconditional, so the waits of phase A can count them: items
  // past the end repeat the previous item's addresses (a cache hit), or read
  // x if the wave has no down work.
  bool d_issued = false;
  auto load_down_batch = [&](int base) {
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(p.x);
    const void* sp = p.x;
    const void* bp = p.x;
    int64_t poff = 0;
#pragma unroll
    for (int j = 0; j < kChunkD; ++j) {
      jhl[j] = min(d_hl, nrows - 1);
      ju[j] = d_u;
      jt[j] = d_t;
      jvalid[j] = d_g * RPID + rsD < slots;
      if (base + j < n_itemsD) {
        const UnitPtr pd = unit_ptr<QMODE>(p, L, d_u, 2);
        const int s = d_t * LI + liD;
        const int64_t row = h0 + jhl[j];
        wp = pd.w + row * wprD + s * 4;
        sp = pd.s;
        bp = pd.b;
        poff = row * pprD + ((QMODE == ZMOE_Q_AFFINE) ? (s >> p.gshift) : s);
        if (++d_t == TD) {  // next slot-group: advance this lane's slot by RPID
          d_t = 0;
          ++d_g;
          d_u += RPID;
          while (d_u >= Uall) {
            d_u -= Uall;
            ++d_hl;
          }
          d_u = (d_hl >= nrows) ? 0 : d_u;  // past the end: any valid unit (result unused)
        }
      }
      wd[j] = gload(reinterpret_cast<const uint4*>(wp));
      rd[j] = seg_param_load<QMODE>(sp, bp, poff);
    }
    d_issued = true;
  };

  // ---------------- phase A: gate/up + SwiGLU ----------------
  if (B == 1 && S_H == kWave) {
    // One token, H = 2048: lane l owns x segment l of every row, so the x
    // segment and the per-row accumulators stay in registers; loads are
    // issued unconditionally (past the end they repeat the previous item's
    // addresses, a cache hit) so each item waits only for its own data.
    const int rg_total = Uall * p.I;
    const int per = (rg_total + W - 1) / W;
    const int g0 = min(rg_total, gw * per), g1 = min(rg_total, g0 + per);
    const uint4 x0 = *reinterpret_cast<const uint4*>(xs + ((0 * 4 + 0) * S_H + lane) * 4);
    const uint4 x1 = *reinterpret_cast<const uint4*>(xs + ((0 * 4 + 1) * S_H + lane) * 4);
    const uint4 x2 = *reinterpret_cast<const uint4*>(xs + ((0 * 4 + 2) * S_H + lane) * 4);
    const uint4 x3 = *reinterpret_cast<const uint4*>(xs + ((0 * 4 + 3) * S_H + lane) * 4);
    const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[lane] : 0.0f;
    const int64_t wpr = p.H >> 3;
    const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S_H >> p.gshift) : S_H;
    const int pi = (QMODE == ZMOE_Q_AFFINE) ? (lane >> p.gshift) : lane;
    int cu_unit = g0 / p.I;
    int cu_row = g0 - cu_unit * p.I;
    for (int base = g0; base < g1; base += kChunkA) {
      uint4 wg[kChunkA], wu[kChunkA];
      RawParam rg[kChunkA], ru[kChunkA];
      int jrow[kChunkA], jpair[kChunkA];
      const uint32_t *gwp = nullptr, *uwp = nullptr;
      const void *gsp = nullptr, *gbp = nullptr, *usp = nullptr, *ubp = nullptr;
      int64_t poff = 0;
#pragma unroll
      for (int j = 0; j < kChunkA; ++j) {
        if (j == 0 || base + j < g1) {
          const UnitPtr pg = unit_ptr<QMODE>(p, L, cu_unit, 0);
          const UnitPtr pu = unit_ptr<QMODE>(p, L, cu_unit, 1);
          gwp = pg.w + cu_row * wpr + lane * 4;
          uwp = pu.w + cu_row * wpr + lane * 4;
          gsp = pg.s;
          gbp = pg.b;
          usp = pu.s;
          ubp = pu.b;
          poff = cu_row * ppr + pi;
          jrow[j] = cu_row;
          jpair[j] = L.upairs[cu_unit][0];
          if (++cu_row == p.I) {
            cu_row = 0;
            ++cu_unit;
          }
        } else {
          jrow[j] = jrow[j - 1];
          jpair[j] = jpair[j - 1];
        }
        wg[j] = gload(reinterpret_cast<const uint4*>(gwp));
        wu[j] = gload(reinterpret_cast<const uint4*>(uwp));
        rg[j] = seg_param_load<QMODE>(gsp, gbp, poff);
        ru[j] = seg_param_load<QMODE>(usp, ubp, poff);
      }
      float gv[kChunkA], uv[kChunkA];
#pragma unroll
      for (int j = 0; j < kChunkA; ++j) {
        float sg, cg, su, cu;
        seg_param_decode<QMODE>(rg[j], sg, cg);
        seg_param_decode<QMODE>(ru[j], su, cu);
        gv[j] = wave_sum(seg_accum<QMODE>(0.0f, sg, cg, seg_dot<QMODE>(wg[j], x0, x1, x2, x3, ak), xsum));
        uv[j] = wave_sum(seg_accum<QMODE>(0.0f, su, cu, seg_dot<QMODE>(wu[j], x0, x1, x2, x3, ak), xsum));
      }
      if (base == g0) trace_mark(p, 6);
      // lane j finalises item j (every lane holds every item's sums)
      float gsel = gv[0], usel = uv[0];
      int rsel = jrow[0], psel = jpair[0];
#pragma unroll
      for (int j = 1; j < kChunkA; ++j) {
        if (lane == j) {
          gsel = gv[j];
          usel = uv[j];
          rsel = jrow[j];
          psel = jpair[j];
        }
      }
      if (lane < kChunkA && base + lane < g1)
        dev_store(p.act + static_cast<int64_t>(psel) * p.act_stride + rsel,
                  (tag16 << 16) | (wg_dead() ? kBf16NaN : swiglu_bf16(round_bf16(gsel), round_bf16(usel))));
      // gate/up data is in and the act rows are on their way: start the down
      // stream (issued earlier it would compete with this phase's loads and
      // hold the stores back)
      if (base == g0) load_down_batch(0);
    }
  } else {
    const int LH = p.LH, RPI = kWave / LH;
    const int rs = lane / LH, li = lane & (LH - 1);
    const int T = S_H / LH;
    const int rgu = p.I / RPI;  // row-groups per unit (Is == I)
    const int rg_total = Uall * rgu;
    const int per = (rg_total + W - 1) / W;
    const int g0 = min(rg_total, gw * per), g1 = min(rg_total, g0 + per);
    const int n_items = (g1 - g0) * T;
    const int64_t wpr = p.H >> 3;
    const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S_H >> p.gshift) : S_H;
    float* ag = accA + (static_cast<size_t>(wave) * 2 * B) * kWave + lane;  // [tk] stride 64
    float* au = ag + static_cast<size_t>(B) * kWave;
    // wave-uniform cursor over (unit, row-group, segment)
    int cu_unit = g0 / max(rgu, 1);
    int cu_rg = g0 - cu_unit * rgu;
    int cu_t = 0;
    for (int base = 0; base < n_items; base += kChunkA) {
      uint4 wg[kChunkA], wu[kChunkA];
      RawParam rg[kChunkA], ru[kChunkA];
      int iu[kChunkA], irow[kChunkA], it_[kChunkA];
#pragma unroll
      for (int j = 0; j < kChunkA; ++j) {
        iu[j] = cu_unit;
        irow[j] = cu_rg * RPI + rs;
        it_[j] = cu_t;
        if (base + j < n_items) {
          const int s = cu_t * LH + li;
          const UnitPtr pg = unit_ptr<QMODE>(p, L, cu_unit, 0);
          const UnitPtr pu = unit_ptr<QMODE>(p, L, cu_unit, 1);
          const int64_t row = irow[j];
          wg[j] = gload(reinterpret_cast<const uint4*>(pg.w + row * wpr + s * 4));
          wu[j] = gload(reinterpret_cast<const uint4*>(pu.w + row * wpr + s * 4));
          const int pi = (QMODE == ZMOE_Q_AFFINE) ? (s >> p.gshift) : s;
          rg[j] = seg_param_load<QMODE>(pg.s, pg.b, row * ppr + pi);
          ru[j] = seg_param_load<QMODE>(pu.s, pu.b, row * ppr + pi);
          if (++cu_t == T) {
            cu_t = 0;
            if (++cu_rg == rgu) {
              cu_rg = 0;
              ++cu_unit;
            }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kChunkA; ++j) {
        if (base + j < n_items) {
          const int u = iu[j], t = it_[j];
          const int s = t * LH + li;
          const int nt = L.ucount[u];
          float sgj, cgj, suj, cuj;
          seg_param_decode<QMODE>(rg[j], sgj, cgj);
          seg_param_decode<QMODE>(ru[j], suj, cuj);
          for (int tk = 0; tk < nt; ++tk) {
            const int q = L.upairs[u][tk];
            const int b = (u < U) ? q / K : q - npairs;
            const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[b * S_H + s] : 0.0f;
            const float g_prev = t == 0 ? 0.0f : ag[tk * kWave];
            const float u_prev = t == 0 ? 0.0f : au[tk * kWave];
            ag[tk * kWave] = seg_accum<QMODE>(g_prev, sgj, cgj, seg_dot_lds<QMODE>(wg[j], xs, S_H, b, s, ak), xsum);
            au[tk * kWave] = seg_accum<QMODE>(u_prev, suj, cuj, seg_dot_lds<QMODE>(wu[j], xs, S_H, b, s, ak), xsum);
          }
          if (base == 0 && j == 0) trace_mark(p, 6);
          if (t == T - 1) {  // row-group complete: reduce, SwiGLU, store act
            for (int tk = 0; tk < nt; ++tk) {
              const float gv = lanes_sum(ag[tk * kWave], LH);
              const float uv = lanes_sum(au[tk * kWave], LH);
              if (li == 0)
                dev_store(p.act + static_cast<int64_t>(L.upairs[u][tk]) * p.act_stride + irow[j],
                          (tag16 << 16) | (wg_dead() ? kBf16NaN : swiglu_bf16(round_bf16(gv), round_bf16(uv))));
            }
          }
        }
      }
    }
  }
  trace_mark(p, 7);

  if (!d_issued) load_down_batch(0);
  trace_mark(p, 8);
  lds_barrier();  // the workgroup is done with the phase A tiles (aliased below)
  trace_mark(p, 9);

  // ---------------- phase D: down projection ----------------
  const int P0 = npairs;
  const int Ptot = npairs + (has_shared ? B : 0);
  uint32_t* as = reinterpret_cast<uint32_t*>(big);
  float* asx = reinterpret_cast<float*>(as + static_cast<size_t>(Ptot) * lds_row_words(S_I));
  float* ybuf = asx + static_cast<size_t>(Ptot) * S_I;                         // [wg rows][Ptot]
  float* accD = ybuf + static_cast<size_t>(kFWaves) * rows_per_wave * Ptot;   // [waves][B][64]
  stage_rows_lds<QMODE, true>(p, p.act, p.act_stride, Ptot, S_I, as, asx, tag16, p.by_S4I, p.by_SI);
  lds_barrier();
  trace_mark(p, 10);
  float* ad = accD + static_cast<size_t>(wave) * B * kWave + lane;
  for (int base = 0; base < n_itemsD; base += kChunkD) {
    if (base > 0) load_down_batch(base);
#pragma unroll
    for (int j = 0; j < kChunkD; ++j) {
      if (base + j < n_itemsD) {
        const int u = ju[j], t = jt[j], hl = jhl[j];
        const int s = t * LI + liD;
        const int nt = L.ucount[u];
        float sdj, cdj;
        seg_param_decode<QMODE>(rd[j], sdj, cdj);
        for (int tk = 0; tk < nt; ++tk) {
          const int q = L.upairs[u][tk];
          const float xsum = (QMODE == ZMOE_Q_AFFINE) ? asx[q * S_I + s] : 0.0f;
          const float prev = t == 0 ? 0.0f : ad[tk * kWave];
          ad[tk * kWave] = seg_accum<QMODE>(prev, sdj, cdj, seg_dot_lds<QMODE>(wd[j], as, S_I, q, s, ak), xsum);
        }
        if (t == TD - 1) {
          for (int tk = 0; tk < nt; ++tk) {
            const float y = lanes_sum(ad[tk * kWave], LI);
            if (liD == 0 && jvalid[j]) ybuf[(wave * rows_per_wave + hl) * Ptot + L.upairs[u][tk]] = round_bf16(y);
          }
        }
      }
    }
  }
  lds_barrier();
  trace_mark(p, 11);

  // ---------------- combine (+ shared expert) ----------------
  const int wg_row0 = blockIdx.x * kFWaves * rows_per_wave;
  const int wg_rows = kFWaves * rows_per_wave;
  for (int b = 0; b < B; ++b) {
    const float* wk = L.route[b].w;
    for (int r = threadIdx.x; r < wg_rows; r += blockDim.x) {
      const int h = wg_row0 + r;
      if (h >= p.H) continue;
      const float* yr = ybuf + r * Ptot + b * K;
      float o = round_bf16(combine_one(p.combine_mode, K, [&](int k) { return yr[k]; }, [&](int k) { return wk[k]; }));
      if (has_shared) o = add_nofma(o, ybuf[r * Ptot + P0 + b]);
      if (wg_dead()) o = kPoison;
      gstore(p.out + static_cast<int64_t>(b) * p.H + h, static_cast<uint16_t>(f32_to_bf16_bits(o)));
    }
  }
  trace_mark(p, 12);
  if (threadIdx.x == 0) dev_store(p.sync + kEpochWord + blockIdx.x, epoch + 1);
  if (p.trace && threadIdx.x == 0) gstore(p.trace + blockIdx.x * kTraceSlots + 14, static_cast<unsigned long long>(clock64()));
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int g_num_cu = 0;

static int num_cus() {
  if (g_num_cu == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      g_num_cu = prop.multiProcessorCount;
    if (g_num_cu <= 0) g_num_cu = 1;
  }
  return g_num_cu;
}

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

size_t fused_lds_bytes(const zmoe_layer_desc* d, int B) {
  const int S_H = d->hidden / 32, S_I = d->inter / 32;
  const int Ptot = B * d->top_k + (d->shared_inter > 0 ? B : 0);
  const int G = num_cus();
  const int rows_per_wave = (d->hidden + G * kFWaves - 1) / (G * kFWaves);
  const size_t front = static_cast<size_t>(B) * (lds_row_words(S_H) * 4 + S_H * 4) + static_cast<size_t>(B) * d->n_experts * 4 +
                       static_cast<size_t>(kFWaves) * 2 * B * kWave * 4;
  const size_t back = static_cast<size_t>(Ptot) * (lds_row_words(S_I) * 4 + S_I * 4) + static_cast<size_t>(kFWaves) * rows_per_wave * Ptot * 4 +
                      static_cast<size_t>(kFWaves) * B * kWave * 4;
  return ((sizeof(FusedLds) + 15) & ~static_cast<size_t>(15)) + (front > back ? front : back);
}

// Which batches take a single-launch kernel.  One token always (the kernel
// sequence's launches dominate: Qwen3 13.0 vs 22.7 us, LFM2 19.2 vs 23.8,
// GLM 19.1 vs 34.6, DeepSeek-V3 76.4 vs 82.9).  From two tokens on the
// kernel sequence streams the experts at a higher rate than the batched
// single-launch kernel gains on launches (Qwen3 B=2/4/8: 26.3/34.4/47.5 us
// vs 30.5/43.0/63.5; LFM2 B=2: 29.7 vs 43.2), except for layers with a
// shared expert, whose own kernels the sequence adds (GLM B=2/4: 31.5/46.3
// vs 42.2/54.1 us; even at B=8) -- so batches of 2..kFusedSharedMaxB tokens
// take k_moe_decodeb there.  (1 MI355X, 48 or 8 rotated layer copies.)
constexpr int kFusedSharedMaxB = 4;

bool fused_supported(const zmoe_layer_desc* d, int B) {
  if (num_cus() > kMaxGrid) return false;
  if (B >= 2)
    return B <= kFusedSharedMaxB && d->shared_inter > 0 && decodeb_supported(d, B, num_cus());
  if (B < 1 || B > kFMaxB) return false;
  if (num_cus() > kMaxGrid) return false;
  if (d->hidden % 512 != 0 || d->hidden / 512 > kMaxNC) return false;
  if (B * d->top_k > kFThreads) return false;
  if (d->shared_inter > 0 && d->shared_inter != d->inter) return false;
  if (d->n_experts > 1024 || d->top_k > kMaxTopK) return false;
  if (fused_lds_bytes(d, B) > 160 * 1024) return false;
  return true;
}

// workspace: state block | rpart | act | trace
static size_t off_rpart() { return kSyncBlockBytes; }
static size_t off_act(const zmoe_layer_desc* d, int B) {
  size_t rpart = static_cast<size_t>(B) * d->n_experts * (d->hidden / 512) * 8;
  if (B == 1 && xcd_rpart_bytes(d) > rpart) rpart = xcd_rpart_bytes(d);  // one XCD-local copy per XCD
  return align256(off_rpart() + rpart);
}
static size_t off_flags(const zmoe_layer_desc* d, int B) {
  const int stride = d->inter > d->shared_inter ? d->inter : d->shared_inter;
  size_t Ptot = static_cast<size_t>(B) * d->top_k + (d->shared_inter > 0 ? B : 0);
  if (B == 1 && Ptot < 8) Ptot = 8;  // the XCD-partitioned one-token kernel: one act row per XCD
  return align256(off_act(d, B) + Ptot * stride * 4);
}
static size_t off_trace(const zmoe_layer_desc* d, int B) {
  return align256(off_flags(d, B) + 4096 + static_cast<size_t>(num_cus()) * 4);
}

static size_t off_xy(const zmoe_layer_desc* d, int B) {
  return align256(off_trace(d, B) + static_cast<size_t>(num_cus()) * kTraceSlots * 8);
}

// tagged expert outputs of the XCD-partitioned one-token kernel
static size_t xy_bytes(const zmoe_layer_desc* d, int B) { return B == 1 ? xcd_xy_bytes(d) : 0; }

size_t fused_workspace_bytes(const zmoe_layer_desc* d, int B) { return off_xy(d, B) + xy_bytes(d, B); }

size_t fused_trace_info(const zmoe_layer_desc* d, int B, int* n_blocks, int* n_slots) {
  *n_blocks = num_cus();
  *n_slots = kTraceSlots;
  return off_trace(d, B);
}

template <int QMODE, int P>
static int launch_fused_t(hipStream_t st, const FusedParams& fp, size_t lds) {
  static bool prepared = false;
  int occ = 0;
  const void* fn = reinterpret_cast<const void*>(&k_moe_decode<QMODE, P>);
  if (!prepared) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    prepared = true;
  }
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kFThreads, lds) != hipSuccess || occ < 1) {
    return fail(ZMOE_EUNSUPPORTED, "[moe_layer] single-launch kernel cannot be resident on every CU");
  }
  hipLaunchKernelGGL((k_moe_decode<QMODE, P>), dim3(num_cus()), dim3(kFThreads), lds, st, fp);
  return check_launch("moe_layer(single launch)");
}

template <int QMODE>
static int launch_fused_q(hipStream_t st, const FusedParams& fp, size_t lds) {
  switch (route_slots(fp.E)) {
    case 1: return launch_fused_t<QMODE, 1>(st, fp, lds);
    case 2: return launch_fused_t<QMODE, 2>(st, fp, lds);
    case 4: return launch_fused_t<QMODE, 4>(st, fp, lds);
    case 8: return launch_fused_t<QMODE, 8>(st, fp, lds);
    default: return launch_fused_t<QMODE, 16>(st, fp, lds);
  }
}

int launch_fused(hipStream_t st, const zmoe_layer_desc* d, const void* x, int B, void* out, uint32_t* out_idx,
                 float* out_w, void* workspace) {
  FusedParams fp{};
  fp.H = d->hidden;
  fp.E = d->n_experts;
  fp.K = d->top_k;
  fp.I = d->inter;
  fp.Is = d->shared_inter;
  fp.B = B;
  int gs = 0;
  for (int v = d->group_size / 32; v > 1; v >>= 1) ++gs;
  fp.gshift = d->quant_mode == ZMOE_Q_AFFINE ? gs : 0;
  fp.combine_mode = d->combine_mode;
  const bool grouped = d->router_kind == ZMOE_ROUTER_SIGMOID_GROUPED;
  fp.route.kind = d->router_kind;
  fp.route.E = d->n_experts;
  fp.route.k = d->top_k;
  fp.route.norm = d->norm_topk_prob;
  fp.route.n_group = grouped ? d->n_group : 1;
  fp.route.topk_group = grouped ? d->topk_group : 1;
  fp.route.scale = grouped ? d->routed_scaling_factor : 1.0f;
  fp.route.bias = d->router_bias;
  fp.route.w_bf16 = 1;
  fp.LH = gcd_int(d->hidden / 32, kWave);
  fp.LI = gcd_int(d->inter / 32, kWave);
  fp.x = static_cast<const uint16_t*>(x);
  fp.out = static_cast<uint16_t*>(out);
  fp.wr = static_cast<const uint16_t*>(d->router_w);
  const uint32_t* ws[6] = {d->gate_w, d->up_w, d->down_w, d->sh_gate_w, d->sh_up_w, d->sh_down_w};
  const void* ss[6] = {d->gate_s, d->up_s, d->down_s, d->sh_gate_s, d->sh_up_s, d->sh_down_s};
  const void* bs[6] = {d->gate_b, d->up_b, d->down_b, d->sh_gate_b, d->sh_up_b, d->sh_down_b};
  for (int i = 0; i < 6; ++i) {
    fp.w[i] = ws[i];
    fp.s[i] = ss[i];
    fp.b[i] = bs[i];
  }
  char* base = static_cast<char*>(workspace);
  fp.sync = reinterpret_cast<unsigned*>(base);
  fp.rpart = reinterpret_cast<unsigned long long*>(base + off_rpart());
  fp.act = reinterpret_cast<uint32_t*>(base + off_act(d, B));
  fp.aflag = reinterpret_cast<unsigned*>(base + off_flags(d, B));
  fp.act_stride = d->inter > d->shared_inter ? d->inter : d->shared_inter;
  fp.out_idx = out_idx;
  fp.out_w = out_w;
  fp.trace = (d->flags & ZMOE_LAYER_TRACE) ? reinterpret_cast<unsigned long long*>(base + off_trace(d, B)) : nullptr;
  fp.err_host = d->error_flag_host;
  fp.spin = d->spin_limit > 0 ? static_cast<unsigned>(d->spin_limit) : kSpinLimit;
  fp.xy = xy_bytes(d, B) > 0 ? reinterpret_cast<uint32_t*>(base + off_xy(d, B)) : nullptr;
  fp.by_S4H = make_fastdiv(static_cast<uint32_t>(d->hidden / 8));
  fp.by_SH = make_fastdiv(static_cast<uint32_t>(d->hidden / 32));
  fp.by_S4I = make_fastdiv(static_cast<uint32_t>(d->inter / 8));
  fp.by_SI = make_fastdiv(static_cast<uint32_t>(d->inter / 32));
  if (B == 1 && decode1_supported(d, num_cus())) return launch_decode1(st, d, fp, num_cus());
  if (B >= 2 && decodeb_supported(d, B, num_cus())) return launch_decodeb(st, d, fp, num_cus());
  const size_t lds = fused_lds_bytes(d, B);
  if (d->quant_mode == ZMOE_Q_AFFINE) return launch_fused_q<ZMOE_Q_AFFINE>(st, fp, lds);
  return launch_fused_q<ZMOE_Q_MXFP4>(st, fp, lds);
}

}  // namespace zmoe
