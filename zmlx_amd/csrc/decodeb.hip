// Batched MoE decode layer in a single launch (2 <= B <= 16 tokens, hidden
// 2048; the path of zmoe_moe_layer for small decode batches,
// moe_mlp.py:787-1072 patched_call).
//
// Same workspace, tagged exchange, arrival counters and arithmetic as the
// one-token kernel (decode1.hip), so results are bit-identical to the kernel
// sequence.  Differences for B tokens:
//
//   R  router partials of every token from one load of each router chunk.
//   T  wave w routes tokens w, w + 8 (route_row); the selected experts form
//      units (ascending expert order); the (token, k) pairs of unit u get
//      consecutive act slots pstart[u] + i, so a unit's act rows are one
//      contiguous block.
//   A  gate/up rows (unit, row) are spread over all waves in contiguous
//      ranges and streamed with double-buffered batches of loads; each row's
//      weights are dequantised once and dotted with every token of the unit
//      (x of all tokens staged in LDS).
//   D  each wave owns output row h of every unit.  The act slots are staged
//      in LDS in passes of whole units that fit (two passes at B = 16 for
//      Qwen3's shape); the row's y values of all slots stay in LDS until the
//      k-ordered combine of every token at the end.
#include "zmoe_fused.h"

namespace zmoe {

constexpr int kDBMaxB = 16;
constexpr int kDBDispatchMaxB = 8;
constexpr int kDBMaxUnits = kDBMaxB * 8 + 1;   // B * K (K <= 8) + shared
constexpr int kDBMaxSlots = kDBMaxB * 8 + kDBMaxB;
constexpr int kDBMaxPass = 16;
constexpr int kDBA = 4;  // gate/up items per batch
constexpr int kDBMaxTD = 8;  // down-projection segments per lane (I / 32 / lanes per row), at most
// act arrival counters: same block layout as the one-token kernel's
constexpr int kDBCtrs = 32;
constexpr int kDBCtrStride = 32;
constexpr int kDBCtrEpoch = kDBCtrs * kDBCtrStride;

struct DBLds {
  unsigned dead, pad_[3];  // word 0 of every single-launch kernel's LDS (wg_dead_word)
  RouteLds route[kDBMaxB];
  int slot_of[1024];            // expert -> unit (or -1)
  int ulist[kDBMaxUnits];
  int ucount[kDBMaxUnits + 1];
  unsigned umask[kDBMaxUnits];   // tokens of unit u
  int pstart[kDBMaxUnits + 1];  // first act slot of unit u
  int ptok[kDBMaxSlots];        // act slot -> token
  int pslot[kDBMaxSlots];       // pair q (b*K + k; npairs + b shared) -> act slot
  int pass_u[kDBMaxPass + 1];   // unit boundaries of the down-projection passes
  float astage[kFWaves][kDBMaxB * 4];  // per wave: act values of one gate/up batch
  int nunits, npass;
  const uint32_t* w[3][kDBMaxUnits];
  const void* s[3][kDBMaxUnits];
  const void* b[3][kDBMaxUnits];
};

struct DBLayout {
  size_t big, xs_sx, as_sx, ybuf, grow, total;
};

// LDS: the DBLds block, then one region used first for the x tile (B rows)
// and later for the act tile (PB slots), then the y values [waves][slots] and
// the grouped-router scratch.
__host__ __device__ inline DBLayout db_layout(int B, int I, int E, int PB) {
  DBLayout o;
  const int S_H = 64, S_I = I / 32;
  size_t off = (sizeof(DBLds) + 15) & ~static_cast<size_t>(15);
  o.big = off;
  const size_t xbytes = static_cast<size_t>(B) * lds_row_words(S_H) * 4;
  o.xs_sx = off + xbytes;
  const size_t x_total = xbytes + static_cast<size_t>(B) * S_H * 4;
  const size_t abytes = static_cast<size_t>(PB) * lds_row_words(S_I) * 4;
  o.as_sx = off + abytes;
  const size_t a_total = abytes + static_cast<size_t>(PB) * S_I * 4;
  off += ((x_total > a_total ? x_total : a_total) + 15) & ~static_cast<size_t>(15);
  o.ybuf = off;
  off += static_cast<size_t>(kFWaves) * kDBMaxSlots * 4;
  o.grow = off;
  off += static_cast<size_t>(kFWaves) * E * 4;
  o.total = off;
  return o;
}

__device__ __forceinline__ void db_set_unit(const FusedParams& p, DBLds& L, int u, int m, int e) {
  if (e >= 0) {
    L.w[m][u] = p.w[m] + static_cast<int64_t>(e) * p.d1.wst[m];
    L.s[m][u] = static_cast<const char*>(p.s[m]) + static_cast<int64_t>(e) * p.d1.sst[m];
    L.b[m][u] = p.b[m] ? static_cast<const void*>(static_cast<const char*>(p.b[m]) + static_cast<int64_t>(e) * p.d1.sst[m])
                       : nullptr;
  } else {
    L.w[m][u] = p.w[3 + m];
    L.s[m][u] = p.s[3 + m];
    L.b[m][u] = p.b[3 + m];
  }
}

// poll_logits for two token rows at once (the second only if `two`).
template <int P>
__device__ __forceinline__ void poll_logits2(const FusedParams& p, const unsigned long long* rp0,
                                             const unsigned long long* rp1, bool two, int NC, unsigned tag,
                                             RowVals<P> (&rows)[2]) {
  const int lane = __lane_id();
  unsigned n = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned long long* rp = h == 0 ? rp0 : rp1;
      const bool act = h == 0 || two;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = lane + 64 * i;
        if (act && e < p.E) {
          unsigned long long part[kMaxNC];
#pragma unroll
          for (int c = 0; c < kMaxNC; ++c)
            if (c < NC) part[c] = dev_load(rp + e * NC + c);
          float a = 0.0f;
#pragma unroll
          for (int c = 0; c < kMaxNC; ++c) {
            if (c < NC) {
              ok = ok && static_cast<unsigned>(part[c] >> 32) == tag;
              a += __uint_as_float(static_cast<uint32_t>(part[c]));
            }
          }
          rows[h].v[i] = round_bf16(a);
        } else {
          rows[h].v[i] = -INFINITY;
        }
      }
    }
    if (__all(ok)) break;
    if (++n > p.spin) {
      if (lane == 0) wait_timeout(p);
      break;
    }
  }
}

template <int QMODE, int P, int TDM>
__global__ __launch_bounds__(kFThreads) void k_moe_decodeb(FusedParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  DBLds& L = *reinterpret_cast<DBLds*>(smem);
  wg_dead_clear();

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = __lane_id();
  const int G = gridDim.x;
  const int W = G * kFWaves;
  const int gw = blockIdx.x * kFWaves + wave;
  const int B = p.B, E = p.E, K = p.K, H = p.H, I = p.I;
  const int NC = H >> 9;
  const int S_H = H >> 5, S_I = I >> 5;
  const AffineK ak = affine_k();
  const bool has_shared = p.Is > 0;
  const D1Plan& pl = p.d1;
  const int PB = pl.PB;
  const DBLayout lay = db_layout(B, I, E, PB);
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem + lay.big);
  float* sx = reinterpret_cast<float*>(smem + lay.xs_sx);
  uint32_t* as = reinterpret_cast<uint32_t*>(smem + lay.big);
  float* asx = reinterpret_cast<float*>(smem + lay.as_sx);
  float* grow = reinterpret_cast<float*>(smem + lay.grow) + wave * E;

  trace_mark(p, 0);
  const unsigned epoch = dev_load(p.sync + kEpochWord + blockIdx.x);
  const unsigned tag = epoch + 1u;
  const unsigned tag16 = tag & 0xFFFFu;
  const unsigned ctag = dev_load(p.aflag + kDBCtrEpoch + blockIdx.x) + 1u;

  // ---------------- R: router partials of every token ----------------
  // unit (e, c, token group of 4): every wave of the grid takes part at B = 16
  {
    const int TG = (B + 3) >> 2;
    const int NU = E * NC * TG;
    for (int u = wave * G + blockIdx.x; u < NU; u += W) {
      const int ec = u / TG, tg = u - ec * TG;
      const int e = static_cast<int>(fdiv(static_cast<uint32_t>(ec), pl.by_NC)), c = ec - e * NC;
      const uint4 wv = gload(reinterpret_cast<const uint4*>(p.wr + static_cast<int64_t>(e) * H + c * 512 + lane * 8));
      uint4 xv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = tg * 4 + i;
        if (b < B) xv[i] = gload(reinterpret_cast<const uint4*>(p.x + static_cast<int64_t>(b) * H + c * 512 + lane * 8));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = tg * 4 + i;
        if (b < B) {
          float a = 0.0f;
          a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.x), __builtin_bit_cast(bf16x2_t, xv[i].x), a, false);
          a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.y), __builtin_bit_cast(bf16x2_t, xv[i].y), a, false);
          a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.z), __builtin_bit_cast(bf16x2_t, xv[i].z), a, false);
          a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.w), __builtin_bit_cast(bf16x2_t, xv[i].w), a, false);
          a = wave_sum(a);
          if (lane == 0)
            dev_store(p.rpart + (static_cast<int64_t>(b) * E + e) * NC + c,
                      (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(a));
        }
      }
    }
  }
  stage_rows_lds<QMODE, false, 4>(p, p.x, H, B, S_H, xs, sx, 0u, p.by_S4H, p.by_SH);
  for (int e = threadIdx.x; e < E; e += kFThreads) L.slot_of[e] = -1;
  trace_mark(p, 1);
  lds_barrier();
  trace_mark(p, 2);

  // ---------------- T: routing, units, act slots ----------------
  if (wave < B) {
    // wave w routes tokens w and w + 8; the second row's partials are polled
    // together with the first's
    const int b1 = wave + kFWaves;
    RowVals<P> rows[2];
    poll_logits2<P>(p, p.rpart + static_cast<int64_t>(wave) * E * NC, p.rpart + static_cast<int64_t>(b1) * E * NC,
                    b1 < B, NC, tag, rows);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int b = wave + h * kFWaves;
      if (b < B) {
        route_row<P>(p.route, rows[h], *(ZMOE_LDS RouteLds*)(&L.route[b]), (ZMOE_LDS float*)grow);
        if (blockIdx.x == 0 && lane < K) {
          if (p.out_idx) gstore(p.out_idx + b * K + lane, static_cast<uint32_t>(L.route[b].sel[lane]));
          if (p.out_w) gstore(p.out_w + b * K + lane, L.route[b].w[lane]);
        }
      }
    }
  }
  trace_mark(p, 3);
  const int npairs = B * K;
  lds_barrier();
  if (threadIdx.x < npairs) L.slot_of[L.route[threadIdx.x / K].sel[threadIdx.x % K]] = 0;
  lds_barrier();
  if (wave == 0) {  // units in ascending expert order
    int base = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
      const int e = e0 + lane;
      const bool f = e < E && L.slot_of[e] == 0;
      const uint64_t m = __ballot(f);
      if (f) {
        const int pos = base + __popcll(m & lanes_below_mask(lane));
        L.slot_of[e] = pos;
        L.ulist[pos] = e;
        L.umask[pos] = 0u;
      }
      base += __popcll(m);
    }
    if (lane == 0) {
      L.nunits = base;
      L.ucount[base] = has_shared ? B : 0;
    }
  }
  lds_barrier();
  // Tokens of each unit as a bitmask (atomicOr is order-free), so a pair's
  // place among its unit's slots -- tokens in ascending order -- is the same
  // in every workgroup.
  int my_u = -1, my_tk = 0;
  if (threadIdx.x < npairs) {
    my_u = L.slot_of[L.route[threadIdx.x / K].sel[threadIdx.x % K]];
    atomicOr(&L.umask[my_u], 1u << (threadIdx.x / K));
  }
  lds_barrier();
  if (threadIdx.x < npairs) my_tk = __popc(L.umask[my_u] & ((1u << (threadIdx.x / K)) - 1u));
  for (int u = threadIdx.x; u < L.nunits; u += kFThreads) L.ucount[u] = __popc(L.umask[u]);
  lds_barrier();
  const int U = L.nunits;
  const int Uall = U + (has_shared ? 1 : 0);
  if (wave == 0) {
    // exclusive prefix sum of the unit counts, 64 units per round
    int carry = 0;
    for (int u0 = 0; u0 < Uall; u0 += kWave) {
      const int u = u0 + lane;
      const int c = u < Uall ? L.ucount[u] : 0;
      int incl = c;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      if (u < Uall) L.pstart[u] = carry + incl - c;
      carry += __shfl(incl, kWave - 1);
    }
    if (lane == 0) L.pstart[Uall] = carry;
  }
  for (int t = threadIdx.x; t < Uall * 3; t += kFThreads) {
    const int u = t / 3, m = t - u * 3;
    db_set_unit(p, L, u, m, u < U ? L.ulist[u] : -1);
  }
  lds_barrier();
  if (threadIdx.x < npairs) {
    const int slot = L.pstart[my_u] + my_tk;
    L.pslot[threadIdx.x] = slot;
    L.ptok[slot] = threadIdx.x / K;
  }
  if (has_shared && threadIdx.x < B) {
    const int slot = L.pstart[U] + threadIdx.x;
    L.pslot[npairs + threadIdx.x] = slot;
    L.ptok[slot] = threadIdx.x;
  }
  lds_barrier();
  trace_mark(p, 5);

  // ---------------- D setup ----------------
  // The workgroup owns output rows [hb, hb + nrw).  Item = (unit, sub-block
  // of RPID rows): lane group rg takes row sb * RPID + rg, LI lanes per row,
  // TD (<= TDM) segments per lane, all loaded at once; every lane of an
  // item serves the same unit, so the token loop is uniform and the act
  // reads are LDS broadcasts.  Items go round-robin to the workgroup's
  // waves, the next item's loads in flight while one is computed.
  const int LI = 1 << pl.lLI, RPID = kWave >> pl.lLI;
  const int rg = lane >> pl.lLI, liD = lane & (LI - 1);
  const int TD = pl.TD;
  const int hb = blockIdx.x * kFWaves;
  const int nrw = max(0, min(H - hb, kFWaves));
  const int nsb = kFWaves / RPID;  // sub-blocks per unit (1 or 2)
  const int64_t wprD = I >> 3;
  const int64_t pprD = (QMODE == ZMOE_Q_AFFINE) ? (S_I >> p.gshift) : S_I;
  int d_u0 = 0, d_nitems = 0;  // this pass: first unit, this wave's items
  auto d_pass_begin = [&](int u0, int u1) {
    d_u0 = u0;
    const int items = (u1 - u0) * nsb;
    d_nitems = (nrw > 0 && items > wave) ? (items - wave + kFWaves - 1) / kFWaves : 0;
  };
  struct ItemD {
    uint4 w[TDM];
    RawParam r[TDM];
    int u, rowl;
  };
  constexpr int kNB = TDM <= 4 ? 2 : 1;  // items in flight per wave (as registers allow)
  ItemD dbuf[kNB];
  auto load_down = [&](int ii, ItemD& it) {
    const int item = wave + kFWaves * min(ii, max(d_nitems - 1, 0));
    const int u = d_u0 + item / nsb, sb = item - (item / nsb) * nsb;
    it.u = u;
    it.rowl = sb * RPID + rg;
    const int64_t row = hb + min(it.rowl, max(nrw - 1, 0));
    const bool ok = d_nitems > 0;
    const uint32_t* wbase = ok ? L.w[2][u] + row * wprD : reinterpret_cast<const uint32_t*>(p.x);
#pragma unroll
    for (int t = 0; t < TDM; ++t) {
      if (t < TD) {
        const int s = t * LI + liD;
        it.w[t] = gload(reinterpret_cast<const uint4*>(wbase + (ok ? s * 4 : 0)));
        it.r[t] = ok ? seg_param_load<QMODE>(L.s[2][u], L.b[2][u],
                                             row * pprD + ((QMODE == ZMOE_Q_AFFINE) ? (s >> p.gshift) : s))
                     : seg_param_load<QMODE>(p.x, p.x, 0);
      }
    }
  };

  // ---------------- A: gate/up + SwiGLU ----------------
  {
    // Batch = 4 consecutive rows of one unit; batch i of this wave is batch
    // number gw + i * W, so every wave gets rows of every unit and the
    // per-token work is balanced.  A batch's act values collect in the
    // wave's LDS stage and leave as one store instruction (16 contiguous
    // bytes per token).
    const int RA = Uall * I;
    const int NBA = RA >> 2;
    const int nb = gw < NBA ? static_cast<int>(fdiv(static_cast<uint32_t>(NBA - gw + W - 1), pl.by_W)) : 0;
    const int64_t wpr = H >> 3;
    const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S_H >> p.gshift) : S_H;
    const int pi = (QMODE == ZMOE_Q_AFFINE) ? (lane >> p.gshift) : lane;
    float* astage = L.astage[wave];
    struct BatchA {
      uint4 wg[kDBA], wu[kDBA];
      RawParam rg[kDBA], ru[kDBA];
      int row0, unit;
    };
    BatchA ba[2];
    auto load_a = [&](int i, BatchA& bt) {
      const int g4 = (gw + min(i, nb - 1) * W) * kDBA;  // past the end: repeat the last batch
      const int cu = static_cast<int>(fdiv(static_cast<uint32_t>(g4), pl.by_I));
      const int r0 = g4 - cu * I;
      bt.row0 = r0;
      bt.unit = cu;
      const uint32_t* gp = L.w[0][cu] + r0 * wpr + lane * 4;
      const uint32_t* up = L.w[1][cu] + r0 * wpr + lane * 4;
#pragma unroll
      for (int j = 0; j < kDBA; ++j) {
        bt.wg[j] = gload(reinterpret_cast<const uint4*>(gp + j * wpr));
        bt.wu[j] = gload(reinterpret_cast<const uint4*>(up + j * wpr));
        bt.rg[j] = seg_param_load<QMODE>(L.s[0][cu], L.b[0][cu], (r0 + j) * ppr + pi);
        bt.ru[j] = seg_param_load<QMODE>(L.s[1][cu], L.b[1][cu], (r0 + j) * ppr + pi);
      }
    };
    auto compute_a = [&](const BatchA& bt) {
      const int u = bt.unit;
      const int p0 = L.pstart[u], nt = L.pstart[u + 1] - p0;
#pragma unroll
      for (int j = 0; j < kDBA; ++j) {
        float sg, cg, su, cu2;
        seg_param_decode<QMODE>(bt.rg[j], sg, cg);
        seg_param_decode<QMODE>(bt.ru[j], su, cu2);
        uint32_t dg[16], du[16];
        seg_dequant<QMODE>(bt.wg[j], dg, ak);
        seg_dequant<QMODE>(bt.wu[j], du, ak);
        for (int tk = 0; tk < nt; ++tk) {  // wave-uniform
          const int b = L.ptok[p0 + tk];
          const uint32_t* xrow = xs + b * lds_row_words(S_H);
          const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[b * S_H + lane] : 0.0f;
          const float gv = wave_sum(seg_accum<QMODE>(0.0f, sg, cg, seg_dot_dq(dg, xrow, S_H, lane), xsum));
          const float uv = wave_sum(seg_accum<QMODE>(0.0f, su, cu2, seg_dot_dq(du, xrow, S_H, lane), xsum));
          if (lane == 0) astage[tk * kDBA + j] = __uint_as_float(swiglu_bf16(round_bf16(gv), round_bf16(uv)));
        }
      }
      wave_lds_sync();
      if (lane < nt * kDBA) {
        const int tk = lane >> 2, j = lane & 3;
        dev_store(p.act + static_cast<int64_t>(p0 + tk) * p.act_stride + bt.row0 + j,
                  (tag16 << 16) | (wg_dead() ? kBf16NaN : __float_as_uint(astage[lane])));
      }
      wave_lds_sync();
    };
    if (nb > 0) load_a(0, ba[0]);
    // down-projection passes (whole units whose act slots fit the LDS tile),
    // worked out while the first gate/up loads are in flight
    if (threadIdx.x == 0) {
      int np = 0, u0 = 0;
      L.pass_u[0] = 0;
      for (int u = 0; u < Uall; ++u) {
        if (L.pstart[u + 1] - L.pstart[u0] > PB) {
          L.pass_u[++np] = u;
          u0 = u;
        }
      }
      L.pass_u[++np] = Uall;
      L.npass = np;
    }
    for (int i = 0; i < nb; i += 2) {
      if (i + 1 < nb) load_a(i + 1, ba[1]);
      compute_a(ba[0]);
      if (i + 1 < nb) {
        if (i + 2 < nb) load_a(i + 2, ba[0]);
        compute_a(ba[1]);
      }
      if (i == 0) trace_mark(p, 6);
    }
  }
  trace_mark(p, 7);

  // every act store of the grid is done once every workgroup has arrived
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  trace_mark(p, 13);
  const int npass = L.npass;
  d_pass_begin(L.pass_u[0], L.pass_u[1]);
  if (threadIdx.x == 0)
    (void)__hip_atomic_fetch_add((ZMOE_GLOBAL unsigned*)(p.aflag + (blockIdx.x % kDBCtrs) * kDBCtrStride), 1u,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the first down items stream in during the exchange; wave 0 polls first
  // (its loads return in order, so polls issued behind them would wait)
  if (wave != 0) {
#pragma unroll
    for (int j = 0; j < kNB; ++j) load_down(j, dbuf[j]);
  } else {
    const int c = lane;
    const unsigned share = c < kDBCtrs ? G / kDBCtrs + (c < G % kDBCtrs ? 1u : 0u) : 0u;
    const unsigned target = ctag * share;
    unsigned spins = 0;
    for (;;) {
      const bool ok = c >= kDBCtrs || static_cast<int>(dev_load(p.aflag + c * kDBCtrStride) - target) >= 0;
      if (__all(ok)) break;
      if (++spins > p.spin) {
        if (lane == 0) wait_timeout(p);
        break;
      }
    }
    trace_mark(p, 14);
#pragma unroll
    for (int j = 0; j < kNB; ++j) load_down(j, dbuf[j]);
  }
  lds_barrier();
  trace_mark(p, 8);

  // ---------------- D: down projection, pass by pass ----------------
  float* ybw = reinterpret_cast<float*>(smem + lay.ybuf);  // [row][slot]
  auto compute_down = [&](int s0, const ItemD& it) {
    const int u = it.u;
    const int p0 = L.pstart[u] - s0, nt = L.pstart[u + 1] - L.pstart[u];
    float sd[TDM], cd[TDM];
#pragma unroll
    for (int t = 0; t < TDM; ++t)
      if (t < TD) seg_param_decode<QMODE>(it.r[t], sd[t], cd[t]);
    for (int tk0 = 0; tk0 < nt; tk0 += 4) {  // wave-uniform: token groups of 4
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < TDM; ++t) {
        if (t < TD) {
          const int s = t * LI + liD;
          uint32_t dq[16];
          seg_dequant<QMODE>(it.w[t], dq, ak);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (tk0 + i < nt) {
              const int r = p0 + tk0 + i;
              const float xsum = (QMODE == ZMOE_Q_AFFINE) ? asx[r * S_I + s] : 0.0f;
              acc[i] = seg_accum<QMODE>(acc[i], sd[t], cd[t], seg_dot_dq(dq, as + r * lds_row_words(S_I), S_I, s), xsum);
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (tk0 + i < nt) {
          const float y = lanes_sum(acc[i], LI);
          if (liD == 0 && it.rowl < nrw) ybw[it.rowl * kDBMaxSlots + L.pstart[u] + tk0 + i] = round_bf16(y);
        }
      }
    }
  };
  for (int ps = 0; ps < npass; ++ps) {
    const int u0 = L.pass_u[ps], u1 = L.pass_u[ps + 1];
    const int s0 = L.pstart[u0], ns = L.pstart[u1] - s0;
    if (ps > 0) {
      lds_barrier();  // the previous pass is done with the tile
      d_pass_begin(u0, u1);
#pragma unroll
      for (int j = 0; j < kNB; ++j) load_down(j, dbuf[j]);
    }
    stage_rows_lds<QMODE, true, 4>(p, p.act + static_cast<int64_t>(s0) * p.act_stride, p.act_stride, ns, S_I, as, asx,
                                tag16, p.by_S4I, p.by_SI);
    lds_barrier();
    if (ps == 0) trace_mark(p, 10);
    for (int ii = 0; ii < d_nitems; ii += kNB) {
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        if (ii + j < d_nitems) {  // wave-uniform
          compute_down(s0, dbuf[j]);
          if (ii + j + kNB < d_nitems) load_down(ii + j + kNB, dbuf[j]);
        }
      }
    }
  }
  lds_barrier();
  trace_mark(p, 11);

  // ---------------- combine (+ shared expert): wave w -> row hb + w, lane b -> token b ----------------
  if (wave < nrw && lane < B) {
    const int b = lane;
    const float* yr = ybw + wave * kDBMaxSlots;
    const float* wk = L.route[b].w;
    float o = round_bf16(combine_one(p.combine_mode, K, [&](int k) { return yr[L.pslot[b * K + k]]; },
                                     [&](int k) { return wk[k]; }));
    if (has_shared) o = add_nofma(o, yr[L.pslot[npairs + b]]);
    if (wg_dead()) o = kPoison;
    gstore(p.out + static_cast<int64_t>(b) * H + hb + wave, static_cast<uint16_t>(f32_to_bf16_bits(o)));
  }
  trace_mark(p, 12);
  if (threadIdx.x == 0) {
    dev_store(p.sync + kEpochWord + blockIdx.x, epoch + 1);
    dev_store(p.aflag + kDBCtrEpoch + blockIdx.x, ctag);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int db_pass_slots(const zmoe_layer_desc* d, int B) {
  // largest act tile (slots) whose layout fits 160 KiB of LDS
  const size_t per = static_cast<size_t>(lds_row_words(d->inter / 32)) * 4 + static_cast<size_t>(d->inter / 32) * 4;
  int pb = static_cast<int>((160 * 1024) / per);
  while (pb > 0 && db_layout(B, d->inter, d->n_experts, pb).total > 160 * 1024) --pb;
  return pb;
}

bool decodeb_supported(const zmoe_layer_desc* d, int B, int grid) {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("ZMOE_DECODEB");
    on = (e && e[0] == '0') ? 0 : 1;
  }
  if (!on) return false;
  // dispatched up to kDBDispatchMaxB tokens (the kernel sequence is faster
  // above that); ZMOE_DECODEB_MAXB raises the limit up to kDBMaxB
  static int maxb = -1;
  if (maxb < 0) {
    const char* e = getenv("ZMOE_DECODEB_MAXB");
    maxb = e ? atoi(e) : kDBDispatchMaxB;
    maxb = maxb < 2 ? 2 : (maxb > kDBMaxB ? kDBMaxB : maxb);
  }
  if (B < 2 || B > maxb || d->hidden != 2048 || d->top_k > 8) return false;
  if (d->n_experts > 1024) return false;
  if (d->shared_inter > 0 && d->shared_inter != d->inter) return false;
  if (d->inter % 32 != 0) return false;
  if ((d->inter / 32) / gcd_int(d->inter / 32, kWave) > kDBMaxTD) return false;
  if (d->inter % 4 != 0) return false;
  // a unit has at most B slots: one must fit a pass; one output row per wave
  return db_pass_slots(d, B) >= B && grid * kFWaves >= d->hidden && grid <= 1024;
}

template <int QMODE, int P, int TDM>
static int launch_db_t(hipStream_t st, const FusedParams& fp, size_t lds, int grid) {
  static bool prepared = false;
  const void* fn = reinterpret_cast<const void*>(&k_moe_decodeb<QMODE, P, TDM>);
  if (!prepared) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    prepared = true;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kFThreads, lds) != hipSuccess || occ < 1)
    return fail(ZMOE_EUNSUPPORTED, "[moe_layer] batched decode kernel cannot be resident on every CU");
  hipLaunchKernelGGL((k_moe_decodeb<QMODE, P, TDM>), dim3(grid), dim3(kFThreads), lds, st, fp);
  return check_launch("moe_layer(batched single launch)");
}

template <int QMODE, int TDM>
static int launch_db_q(hipStream_t st, const FusedParams& fp, size_t lds, int grid) {
  switch (route_slots(fp.E)) {
    case 1: return launch_db_t<QMODE, 1, TDM>(st, fp, lds, grid);
    case 2: return launch_db_t<QMODE, 2, TDM>(st, fp, lds, grid);
    case 4: return launch_db_t<QMODE, 4, TDM>(st, fp, lds, grid);
    case 8: return launch_db_t<QMODE, 8, TDM>(st, fp, lds, grid);
    default: return launch_db_t<QMODE, 16, TDM>(st, fp, lds, grid);
  }
}

int launch_decodeb(hipStream_t st, const zmoe_layer_desc* d, const FusedParams& fp_in, int grid) {
  FusedParams fp = fp_in;
  D1Plan& pl = fp.d1;
  const int W = grid * kFWaves;
  const int H = d->hidden, I = d->inter, S_I = I / 32;
  pl.rpw = (H + W - 1) / W;
  const int LI = gcd_int(S_I, kWave);
  pl.lLI = 0;
  while ((1 << pl.lLI) < LI) ++pl.lLI;
  pl.lLH = 6;
  pl.TA = 1;
  pl.TD = S_I / LI;
  pl.PB = db_pass_slots(d, fp.B);
  pl.by_NC = make_fastdiv(static_cast<uint32_t>(H / 512));
  pl.by_W = make_fastdiv(static_cast<uint32_t>(W));
  pl.by_I = make_fastdiv(static_cast<uint32_t>(I));
  for (int m = 0; m < 3; ++m) {
    const int64_t N = (m == 2) ? H : I, Kin = (m == 2) ? I : H;
    const int64_t groups = (d->quant_mode == ZMOE_Q_AFFINE) ? Kin / d->group_size : Kin / 32;
    pl.wst[m] = N * (Kin / 8);
    pl.sst[m] = N * groups * ((d->quant_mode == ZMOE_Q_AFFINE) ? 2 : 1);
  }
  const size_t lds = db_layout(fp.B, I, d->n_experts, pl.PB).total;
  const bool small = pl.TD <= 4;
  if (d->quant_mode == ZMOE_Q_AFFINE)
    return small ? launch_db_q<ZMOE_Q_AFFINE, 4>(st, fp, lds, grid) : launch_db_q<ZMOE_Q_AFFINE, 8>(st, fp, lds, grid);
  return small ? launch_db_q<ZMOE_Q_MXFP4, 4>(st, fp, lds, grid) : launch_db_q<ZMOE_Q_MXFP4, 8>(st, fp, lds, grid);
}

}  // namespace zmoe
