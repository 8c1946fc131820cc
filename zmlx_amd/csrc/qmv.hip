// Gather + quantized GEMV kernels (decode-shaped: few activation rows per
// selected expert).  Entry points: zmoe_gather_qmm_swiglu, zmoe_gather_qmm.
//
// Work decomposition (wave64, weights streamed once with 16-byte loads):
//   * a row of K packed 4-bit weights is S = K/32 segments of 16 bytes;
//   * L = gcd(S, 64) lanes share a row, so one wave-wide load instruction
//     covers 64/L rows x L segments = 1 KiB of contiguous-per-row bytes;
//   * lane (rs, li) owns segments li, li+L, ... of its rows, accumulates in
//     fp32 and the L lanes of a row are reduced with cross-lane adds;
//   * the activation rows are staged once per workgroup in LDS in the
//     pair-permuted layout the dot2 dequant trick needs (zmoe_common.h).
#include "zmoe_common.h"
#include "zmoe_grouped.h"
#include "zmoe_host.h"

#include <type_traits>
#include <utility>

namespace zmoe {

constexpr int kQmvThreads = 256;
constexpr int kQmvWaves = kQmvThreads / kWave;

// Stage activation row `xrow` (bf16 [32*S]) as token t of the LDS tile.
//   xs[((t*4 + j)*S + s)*4 + d] : bf16 pair d of word j of segment s
//   sx[t*S + s]                 : fp32 sum of the segment's 32 values (affine)
template <int QMODE>
__device__ void stage_x_row(const uint16_t* __restrict__ xrow, int S, uint32_t* xs, float* sx, int t) {
  for (int i = threadIdx.x; i < S * 4; i += blockDim.x) {
    const int s = i >> 2, j = i & 3;
    const uint4 v = *reinterpret_cast<const uint4*>(xrow + s * 32 + j * 8);
    uint4 o;
    if (QMODE == ZMOE_Q_AFFINE) {
      // elements e0..e7 -> pairs (e0,e4) (e1,e5) (e2,e6) (e3,e7)
      o.x = (v.x & 0xFFFFu) | (v.z << 16);
      o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
      o.z = (v.y & 0xFFFFu) | (v.w << 16);
      o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
    } else {
      o = v;  // natural pairs (e0,e1) (e2,e3) ...
    }
    *reinterpret_cast<uint4*>(xs + ((t * 4 + j) * S + s) * 4) = o;
  }
  if (QMODE == ZMOE_Q_AFFINE) {
    for (int s = threadIdx.x; s < S; s += blockDim.x) {
      float acc = 0.0f;
      const uint4* p = reinterpret_cast<const uint4*>(xrow + s * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint4 v = p[q];
        acc += bf16_bits_to_f32(v.x & 0xFFFFu) + bf16_bits_to_f32(v.x >> 16);
        acc += bf16_bits_to_f32(v.y & 0xFFFFu) + bf16_bits_to_f32(v.y >> 16);
        acc += bf16_bits_to_f32(v.z & 0xFFFFu) + bf16_bits_to_f32(v.z >> 16);
        acc += bf16_bits_to_f32(v.w & 0xFFFFu) + bf16_bits_to_f32(v.w >> 16);
      }
      sx[t * S + s] = acc;
    }
  }
}

// Per-(row, segment) quantisation parameters.
struct SegParam {
  float s;  // scale
  float c;  // affine: bias - 128*scale (multiplies the segment's x sum)
};

template <int QMODE>
__device__ __forceinline__ SegParam load_param(const void* __restrict__ scales, const void* __restrict__ biases,
                                               int64_t idx) {
  SegParam p;
  if (QMODE == ZMOE_Q_AFFINE) {
    const float s = bf16_bits_to_f32(static_cast<const uint16_t*>(scales)[idx]);
    const float b = bf16_bits_to_f32(static_cast<const uint16_t*>(biases)[idx]);
    p.s = s;
    p.c = b - 128.0f * s;
  } else {
    p.s = e8m0_to_f32(static_cast<const uint8_t*>(scales)[idx]);
    p.c = 0.0f;
  }
  return p;
}

// One wave computes J*(64/L) rows of one (or, with SWIGLU, two) quantized
// matrices against NT staged activation rows.  Results land in lanes with
// (lane % L) == 0.
template <int L, int J, int NT, int QMODE, bool SWIGLU>
__device__ __forceinline__ void wave_qmv(const uint32_t* __restrict__ Wg, const void* __restrict__ Sg,
                                         const void* __restrict__ Bg, const uint32_t* __restrict__ Wu,
                                         const void* __restrict__ Su, const void* __restrict__ Bu, int N,
                                         int K, int gshift, int row0, int ntok, const uint32_t* xs,
                                         const float* sx, float (&rg)[J][NT], float (&ru)[J][NT]) {
  constexpr int RPI = kWave / L;
  const int lane = threadIdx.x & (kWave - 1);
  const int rs = lane / L, li = lane % L;
  const int S = K >> 5;
  const int T = S / L;
  const int64_t wpr = K >> 3;                                        // words per row
  const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S >> gshift) : S;  // params per row
  const AffineK ak = affine_k();

  int64_t rowoff[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    int r = row0 + j * RPI + rs;
    rowoff[j] = r < N ? r : N - 1;  // clamp: lanes past N load a valid row, result discarded
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      rg[j][t] = 0.0f;
      ru[j][t] = 0.0f;
    }
  }

  for (int t = 0; t < T; ++t) {
    const int s = t * L + li;
    const int g = (QMODE == ZMOE_Q_AFFINE) ? (s >> gshift) : s;
    uint4 wg[J], wu[J];
    SegParam pg[J], pu[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      wg[j] = *reinterpret_cast<const uint4*>(Wg + rowoff[j] * wpr + s * 4);
      if (SWIGLU) wu[j] = *reinterpret_cast<const uint4*>(Wu + rowoff[j] * wpr + s * 4);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      pg[j] = load_param<QMODE>(Sg, Bg, rowoff[j] * ppr + g);
      if (SWIGLU) pu[j] = load_param<QMODE>(Su, Bu, rowoff[j] * ppr + g);
    }
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      if (tok < ntok) {
        const uint4 x0 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 0) * S + s) * 4);
        const uint4 x1 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 1) * S + s) * 4);
        const uint4 x2 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 2) * S + s) * 4);
        const uint4 x3 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 3) * S + s) * 4);
        const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[tok * S + s] : 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const float vg = seg_dot<QMODE>(wg[j], x0, x1, x2, x3, ak);
          rg[j][tok] = seg_accum<QMODE>(rg[j][tok], pg[j].s, pg[j].c, vg, xsum);
          if (SWIGLU) {
            const float vu = seg_dot<QMODE>(wu[j], x0, x1, x2, x3, ak);
            ru[j][tok] = seg_accum<QMODE>(ru[j][tok], pu[j].s, pu[j].c, vu, xsum);
          }
        }
      }
    }
  }

#pragma unroll
  for (int j = 0; j < J; ++j) {
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      rg[j][tok] = wave_sum_width<L>(rg[j][tok]);
      if (SWIGLU) ru[j][tok] = wave_sum_width<L>(ru[j][tok]);
    }
  }
}

template <int L, int J, int NT, int QMODE, bool SWIGLU>
__global__ __launch_bounds__(kQmvThreads) void k_gather_qmv(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ Wg, const void* __restrict__ Sg,
    const void* __restrict__ Bg, const uint32_t* __restrict__ Wu, const void* __restrict__ Su,
    const void* __restrict__ Bu, const uint32_t* __restrict__ lhs, const uint32_t* __restrict__ rhs, int lhs_div,
    int M, int N, int K, int gshift, uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) uint32_t smem[];
  const int S = K >> 5;
  uint32_t* xs = smem;
  float* sx = reinterpret_cast<float*>(smem + NT * S * 16);

  const int64_t p = blockIdx.y;
  const int m0 = blockIdx.z * NT;
  const int ntok = min(NT, M - m0);
  // Without index arrays (internal callers): x row p / lhs_div, expert 0.
  const int64_t xl = lhs ? static_cast<int64_t>(lhs[p]) : p / lhs_div;
  const int64_t e = rhs ? static_cast<int64_t>(rhs[p]) : 0;

  for (int t = 0; t < ntok; ++t) stage_x_row<QMODE>(x + (xl * M + m0 + t) * K, S, xs, sx, t);
  __syncthreads();

  constexpr int RPW = J * (kWave / L);  // rows per wave
  const int wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kQmvWaves + wave) * RPW;
  if (row0 >= N) return;

  const int64_t wstride = static_cast<int64_t>(N) * (K >> 3);
  const int64_t pstride = static_cast<int64_t>(N) * ((QMODE == ZMOE_Q_AFFINE) ? (S >> gshift) : S);
  const int pbytes = (QMODE == ZMOE_Q_AFFINE) ? 2 : 1;
  const uint32_t* wg = Wg + e * wstride;
  const void* sg = static_cast<const char*>(Sg) + e * pstride * pbytes;
  const void* bg = (QMODE == ZMOE_Q_AFFINE) ? static_cast<const void*>(static_cast<const char*>(Bg) + e * pstride * 2) : nullptr;
  const uint32_t* wu = SWIGLU ? Wu + e * wstride : nullptr;
  const void* su = SWIGLU ? static_cast<const void*>(static_cast<const char*>(Su) + e * pstride * pbytes) : nullptr;
  const void* bu = (SWIGLU && QMODE == ZMOE_Q_AFFINE) ? static_cast<const void*>(static_cast<const char*>(Bu) + e * pstride * 2) : nullptr;

  float rg[J][NT], ru[J][NT];
  wave_qmv<L, J, NT, QMODE, SWIGLU>(wg, sg, bg, wu, su, bu, N, K, gshift, row0, ntok, xs, sx, rg, ru);

  const int lane = threadIdx.x & (kWave - 1);
  if ((lane % L) == 0) {
    const int rs = lane / L;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int r = row0 + j * (kWave / L) + rs;
      if (r < N) {
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
          if (tok < ntok) {
            uint32_t v;
            if (SWIGLU) {
              v = swiglu_bf16(round_bf16(rg[j][tok]), round_bf16(ru[j][tok]));
            } else {
              v = f32_to_bf16_bits(rg[j][tok]);
            }
            out[(p * M + m0 + tok) * N + r] = static_cast<uint16_t>(v);
          }
        }
      }
    }
  }
}

template <int L, int J, int NT, int QMODE, bool SWIGLU>
static int launch_qmv_t(hipStream_t st, const void* x, const uint32_t* wg, const void* sg, const void* bg,
                        const uint32_t* wu, const void* su, const void* bu, const uint32_t* lhs,
                        const uint32_t* rhs, int lhs_div, int64_t n_pairs, int M, int N, int K, int gshift,
                        void* out) {
  constexpr int RPW = J * (kWave / L);
  const int S = K >> 5;
  dim3 grid((N + kQmvWaves * RPW - 1) / (kQmvWaves * RPW), static_cast<unsigned>(n_pairs), (M + NT - 1) / NT);
  const size_t lds = static_cast<size_t>(NT) * S * 64 + static_cast<size_t>(NT) * S * 4;
  hipLaunchKernelGGL((k_gather_qmv<L, J, NT, QMODE, SWIGLU>), grid, dim3(kQmvThreads), lds, st,
                     static_cast<const uint16_t*>(x), wg, sg, bg, wu, su, bu, lhs, rhs, lhs_div, M, N, K, gshift,
                     static_cast<uint16_t*>(out));
  return check_launch(SWIGLU ? "gather_qmm_swiglu" : "gather_qmm");
}

template <int NT, int QMODE, bool SWIGLU>
static int launch_qmv_l(hipStream_t st, int L, const void* x, const uint32_t* wg, const void* sg,
                        const void* bg, const uint32_t* wu, const void* su, const void* bu,
                        const uint32_t* lhs, const uint32_t* rhs, int lhs_div, int64_t n_pairs, int M, int N,
                        int K, int gshift, void* out) {
  switch (L) {
    case 64:
      return launch_qmv_t<64, 4, NT, QMODE, SWIGLU>(st, x, wg, sg, bg, wu, su, bu, lhs, rhs, lhs_div, n_pairs, M, N, K, gshift, out);
    case 32:
      return launch_qmv_t<32, 2, NT, QMODE, SWIGLU>(st, x, wg, sg, bg, wu, su, bu, lhs, rhs, lhs_div, n_pairs, M, N, K, gshift, out);
    case 16:
      return launch_qmv_t<16, 2, NT, QMODE, SWIGLU>(st, x, wg, sg, bg, wu, su, bu, lhs, rhs, lhs_div, n_pairs, M, N, K, gshift, out);
    case 8:
      return launch_qmv_t<8, 2, NT, QMODE, SWIGLU>(st, x, wg, sg, bg, wu, su, bu, lhs, rhs, lhs_div, n_pairs, M, N, K, gshift, out);
    default:
      return fail(ZMOE_EUNSUPPORTED, "[gather_qmm] unsupported lane split");
  }
}

// ---------------------------------------------------------------------------
// Expert-major GEMV over the expert-sorted (token, k) pairs: block (row tile,
// chunk c) takes the chunk's expert e and its up to NT sorted rows, stages
// those activation rows in LDS, and streams e's weight rows once for all of
// them (wave_qmv, the same arithmetic as k_gather_qmv).  Results go to the
// rows' pair positions (scatter) or their sorted positions.
// ---------------------------------------------------------------------------
constexpr int kGemvRows = 128;  // weight rows per workgroup of the expert-major GEMV
constexpr int kGqDepth = 4;     // items in the expert-major GEMV's load ring

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Quantisation parameters loaded raw and decoded at use (decoding right
// after the load would make its wait immediate); decode_raw_q gives
// load_param's values.
struct RawQ {
  uint32_t s, b;
};
template <int QMODE>
__device__ __forceinline__ RawQ load_raw_q(const void* __restrict__ scales, const void* __restrict__ biases,
                                           int64_t idx) {
  RawQ r;
  if (QMODE == ZMOE_Q_AFFINE) {
    r.s = static_cast<const uint16_t*>(scales)[idx];
    r.b = static_cast<const uint16_t*>(biases)[idx];
  } else {
    r.s = static_cast<const uint8_t*>(scales)[idx];
    r.b = 0;
  }
  return r;
}
template <int QMODE>
__device__ __forceinline__ SegParam decode_raw_q(RawQ r) {
  SegParam p;
  if (QMODE == ZMOE_Q_AFFINE) {
    const float s = bf16_bits_to_f32(r.s);
    const float b = bf16_bits_to_f32(r.b);
    p.s = s;
    p.c = b - 128.0f * s;
  } else {
    p.s = e8m0_to_f32(r.s);
    p.c = 0.0f;
  }
  return p;
}

template <int L, int J, int NT, int QMODE, bool SWIGLU>
__global__ __launch_bounds__(kQmvThreads) void k_grouped_qmv(GroupedArgs g, int gshift, int tiles) {
  extern __shared__ __align__(16) uint32_t smem[];
  const int K = g.K, N = g.N;
  const int S = K >> 5;
  uint32_t* xs = smem;
  float* sx = reinterpret_cast<float*>(smem + NT * S * 16);
  const int c = blockIdx.y;
  if (c >= g.offsets[g.E + 1]) return;  // whole workgroup: past the chunk list
  const int ce = g.blocks[c];
  const int64_t e = ce & 2047;
  const int r_begin = g.offsets[e] + (ce >> 11) * NT;
  const int ntok = min(NT, g.offsets[e + 1] - r_begin);
  for (int t = 0; t < ntok; ++t) {
    const int src = g.sorted[r_begin + t];
    const int64_t arow = g.a_div > 0 ? src / g.a_div : src;
    stage_x_row<QMODE>(g.a + arow * g.lda, S, xs, sx, t);
  }
  __syncthreads();
  const int wave = threadIdx.x / kWave;
  const int64_t wstride = static_cast<int64_t>(N) * (K >> 3);
  const int64_t pstride = static_cast<int64_t>(N) * ((QMODE == ZMOE_Q_AFFINE) ? (S >> gshift) : S);
  const int pbytes = (QMODE == ZMOE_Q_AFFINE) ? 2 : 1;
  const uint32_t* wg = g.w0 + e * wstride;
  const void* sg = static_cast<const char*>(g.s0) + e * pstride * pbytes;
  const void* bg = (QMODE == ZMOE_Q_AFFINE) ? static_cast<const void*>(static_cast<const char*>(g.b0) + e * pstride * 2)
                                            : nullptr;
  const uint32_t* wu = SWIGLU ? g.w1 + e * wstride : nullptr;
  const void* su = SWIGLU ? static_cast<const void*>(static_cast<const char*>(g.s1) + e * pstride * pbytes) : nullptr;
  const void* bu_ = (SWIGLU && QMODE == ZMOE_Q_AFFINE)
                       ? static_cast<const void*>(static_cast<const char*>(g.b1) + e * pstride * 2)
                       : nullptr;
  // The block covers `tiles` consecutive row tiles (about kGemvRows rows) with
  // one staging of the chunk's rows: the index loads and the staging are paid
  // once for all of them.  A wave's work is a flat list of items (row tile
  // tt, segment step t), T = S / L steps per row; the loads of the next
  // kGqDepth - 1 items are in flight while one is computed (loads are
  // unconditional, the item index clamped at the end, so the wait counts
  // stay exact).  Per row the arithmetic is wave_qmv's: segment steps
  // accumulated in order, then the L-lane sum.
  static_assert(J == 1, "one row group per wave and tile");
  constexpr int RPW = kWave / L;
  constexpr int D = kGqDepth;
  const int lane = threadIdx.x & (kWave - 1);
  const int rs = lane / L, li = lane % L;
  const int T = S / L;
  const int64_t wpr = K >> 3;
  const int64_t ppr = (QMODE == ZMOE_Q_AFFINE) ? (S >> gshift) : S;
  const AffineK ak = affine_k();
  int64_t orow[NT];
#pragma unroll
  for (int tok = 0; tok < NT; ++tok)
    orow[tok] = tok < ntok ? (g.scatter ? static_cast<int64_t>(g.sorted[r_begin + tok]) : r_begin + tok) : 0;
  // tiles of this block that hold rows for this wave
  const int tile0 = blockIdx.x * tiles;
  int ntl = 0;
  while (ntl < tiles && ((tile0 + ntl) * kQmvWaves + wave) * RPW < N) ++ntl;
  const int nitems = ntl * T;
  if (nitems == 0) return;
  uint4 bw[D], bu[D];
  RawQ pgr[D], pur[D];
  auto load_item = [&](int i, auto qc) {
    constexpr int q = decltype(qc)::value;
    const int it = min(i, nitems - 1);
    const int tt = it / T, t = it - tt * T;
    const int r = ((tile0 + tt) * kQmvWaves + wave) * RPW + rs;
    const int64_t row = r < N ? r : N - 1;
    const int sg_ = t * L + li;
    const int gi = (QMODE == ZMOE_Q_AFFINE) ? (sg_ >> gshift) : sg_;
    bw[q] = *reinterpret_cast<const uint4*>(wg + row * wpr + sg_ * 4);
    if (SWIGLU) bu[q] = *reinterpret_cast<const uint4*>(wu + row * wpr + sg_ * 4);
    pgr[q] = load_raw_q<QMODE>(sg, bg, row * ppr + gi);
    if (SWIGLU) pur[q] = load_raw_q<QMODE>(su, bu_, row * ppr + gi);
  };
  float rg[NT], ru[NT];
#pragma unroll
  for (int tok = 0; tok < NT; ++tok) rg[tok] = ru[tok] = 0.0f;
  auto compute_item = [&](int i, auto qc) {
    constexpr int q = decltype(qc)::value;
    const int tt = i / T, t = i - tt * T;
    const int sg_ = t * L + li;
    const SegParam pg = decode_raw_q<QMODE>(pgr[q]);
    SegParam pu{0.0f, 0.0f};
    if (SWIGLU) pu = decode_raw_q<QMODE>(pur[q]);
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      if (tok < ntok) {
        const uint4 x0 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 0) * S + sg_) * 4);
        const uint4 x1 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 1) * S + sg_) * 4);
        const uint4 x2 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 2) * S + sg_) * 4);
        const uint4 x3 = *reinterpret_cast<const uint4*>(xs + ((tok * 4 + 3) * S + sg_) * 4);
        const float xsum = (QMODE == ZMOE_Q_AFFINE) ? sx[tok * S + sg_] : 0.0f;
        rg[tok] = seg_accum<QMODE>(rg[tok], pg.s, pg.c, seg_dot<QMODE>(bw[q], x0, x1, x2, x3, ak), xsum);
        if (SWIGLU) ru[tok] = seg_accum<QMODE>(ru[tok], pu.s, pu.c, seg_dot<QMODE>(bu[q], x0, x1, x2, x3, ak), xsum);
      }
    }
    if (t == T - 1) {
      const int r = ((tile0 + tt) * kQmvWaves + wave) * RPW + rs;
#pragma unroll
      for (int tok = 0; tok < NT; ++tok) {
        const float vg = wave_sum_width<L>(rg[tok]);
        const float vu = SWIGLU ? wave_sum_width<L>(ru[tok]) : 0.0f;
        if (li == 0 && r < N && tok < ntok) {
          const uint32_t v = SWIGLU ? swiglu_bf16(round_bf16(vg), round_bf16(vu)) : f32_to_bf16_bits(vg);
          g.out[orow[tok] * g.ldo + r] = static_cast<uint16_t>(v);
        }
        rg[tok] = ru[tok] = 0.0f;
      }
    }
  };
  // ring slot q holds item i with i % D == q
  static_for<D - 1>([&](auto q) { load_item(decltype(q)::value, q); });
  for (int i = 0; i < nitems; i += D) {
    static_for<D>([&](auto q) {
      constexpr int Q = decltype(q)::value;
      load_item(i + Q + D - 1, std::integral_constant<int, (Q + D - 1) % D>{});
      if (i + Q < nitems) compute_item(i + Q, q);
    });
  }
}

template <int L, int J, int QMODE, bool SWIGLU>
static int launch_grouped_qmv_t(hipStream_t st, const GroupedArgs& g, int n_experts, int gshift) {
  constexpr int NT = kGroupedGemvRows;
  constexpr int RPW = J * (kWave / L);
  const int S = g.K >> 5;
  const int tiles = kGemvRows / (kQmvWaves * RPW) > 0 ? kGemvRows / (kQmvWaves * RPW) : 1;
  const int rows_per_block = kQmvWaves * RPW * tiles;
  dim3 grid((g.N + rows_per_block - 1) / rows_per_block, static_cast<unsigned>(grouped_gemv_max_chunks(g.M, n_experts)));
  const size_t lds = static_cast<size_t>(NT) * S * 64 + static_cast<size_t>(NT) * S * 4;
  hipLaunchKernelGGL((k_grouped_qmv<L, J, NT, QMODE, SWIGLU>), grid, dim3(kQmvThreads), lds, st, g, gshift, tiles);
  return check_launch(SWIGLU ? "grouped gather_qmm_swiglu (gemv)" : "grouped gather_qmm (gemv)");
}

template <int QMODE, bool SWIGLU>
static int launch_grouped_qmv_l(hipStream_t st, const GroupedArgs& g, int n_experts, int gshift) {
  switch (gcd_int(g.K >> 5, kWave)) {
    case 64:
      return launch_grouped_qmv_t<64, 1, QMODE, SWIGLU>(st, g, n_experts, gshift);
    case 32:
      return launch_grouped_qmv_t<32, 1, QMODE, SWIGLU>(st, g, n_experts, gshift);
    case 16:
      return launch_grouped_qmv_t<16, 1, QMODE, SWIGLU>(st, g, n_experts, gshift);
    case 8:
      return launch_grouped_qmv_t<8, 1, QMODE, SWIGLU>(st, g, n_experts, gshift);
    default:
      return fail(ZMOE_EUNSUPPORTED, "[gather_qmm] unsupported lane split");
  }
}

int launch_grouped_qmv(hipStream_t st, const GroupedArgs& g, int n_experts, int quant_mode, bool swiglu) {
  if (g.M == 0) return ZMOE_OK;
  ZMOE_REQUIRE(g.K % 256 == 0, ZMOE_EINVAL_SHAPE, "[gather_qmm] K must be a multiple of 256.");
  int gshift = 0;
  if (quant_mode == ZMOE_Q_AFFINE)
    for (int v = g.gs / 32; v > 1; v >>= 1) ++gshift;
  if (quant_mode == ZMOE_Q_AFFINE)
    return swiglu ? launch_grouped_qmv_l<ZMOE_Q_AFFINE, true>(st, g, n_experts, gshift)
                  : launch_grouped_qmv_l<ZMOE_Q_AFFINE, false>(st, g, n_experts, gshift);
  return swiglu ? launch_grouped_qmv_l<ZMOE_Q_MXFP4, true>(st, g, n_experts, gshift)
                : launch_grouped_qmv_l<ZMOE_Q_MXFP4, false>(st, g, n_experts, gshift);
}

// Shared argument validation of the two gather-QMM entry points.  Messages
// follow the reference's wording where one exists (patch:578-581, 714-743).
static int validate_qmm(const char* op, const void* x, int64_t x_batch, const uint32_t* w, const void* s,
                        const void* b, const uint32_t* lhs, const uint32_t* rhs, int64_t n_pairs, int M,
                        int N, int K, int E, int group_size, int bits, int quant_mode, const void* out,
                        int* gshift) {
  const std::string tag = std::string("[") + op + "] ";
  ZMOE_REQUIRE(quant_mode == ZMOE_Q_AFFINE || quant_mode == ZMOE_Q_MXFP4, ZMOE_EUNSUPPORTED,
               tag + "Only affine and mxfp4 quantization modes are supported.");
  ZMOE_REQUIRE(bits == 4, ZMOE_EUNSUPPORTED, tag + "Only bits == 4 is supported.");
  if (quant_mode == ZMOE_Q_AFFINE) {
    ZMOE_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128, ZMOE_EUNSUPPORTED,
                 tag + "group_size must be 32, 64 or 128 for affine mode.");
    ZMOE_REQUIRE(b != nullptr, ZMOE_EINVAL_SHAPE, tag + "affine mode requires biases.");
  } else {
    ZMOE_REQUIRE(group_size == 32, ZMOE_EUNSUPPORTED, tag + "mxfp4 requires group_size == 32.");
  }
  ZMOE_REQUIRE(M >= 1 && N >= 1 && K >= 1 && E >= 1 && n_pairs >= 0 && x_batch >= 1, ZMOE_EINVAL_SHAPE,
               tag + "sizes must be positive.");
  ZMOE_REQUIRE(K % 256 == 0, ZMOE_EINVAL_SHAPE, tag + "K must be a multiple of 256.");
  ZMOE_REQUIRE(n_pairs <= 65535, ZMOE_EINVAL_SHAPE, tag + "at most 65535 (lhs, rhs) pairs per call.");
  ZMOE_REQUIRE((M + 3) / 4 <= 65535, ZMOE_EINVAL_SHAPE, tag + "M too large.");
  ZMOE_REQUIRE(n_pairs == 0 || (x && w && s && lhs && rhs && out), ZMOE_EINVAL_SHAPE, tag + "null pointer.");
  ZMOE_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
               ZMOE_EINVAL_SHAPE, tag + "x and weights must be 16-byte aligned.");
  int gs = 0;
  for (int v = group_size / 32; v > 1; v >>= 1) ++gs;
  *gshift = gs;
  return ZMOE_OK;
}

int dispatch_qmv(bool swiglu, void* stream, const void* x, const uint32_t* wg, const void* sg, const void* bg,
                 const uint32_t* wu, const void* su, const void* bu, const uint32_t* lhs, const uint32_t* rhs,
                 int lhs_div, int64_t n_pairs, int M, int N, int K, int quant_mode, int gshift, void* out) {
  if (n_pairs == 0) return ZMOE_OK;
  hipStream_t st = as_stream(stream);
  const int L = gcd_int(K >> 5, kWave);
  const bool one = (M == 1);
  const bool aff = (quant_mode == ZMOE_Q_AFFINE);
#define ZMOE_QMV_CASE(NT, QM, SW) \
  return launch_qmv_l<NT, QM, SW>(st, L, x, wg, sg, bg, wu, su, bu, lhs, rhs, lhs_div, n_pairs, M, N, K, gshift, out)
  if (swiglu) {
    if (aff) {
      if (one) ZMOE_QMV_CASE(1, ZMOE_Q_AFFINE, true);
      ZMOE_QMV_CASE(4, ZMOE_Q_AFFINE, true);
    }
    if (one) ZMOE_QMV_CASE(1, ZMOE_Q_MXFP4, true);
    ZMOE_QMV_CASE(4, ZMOE_Q_MXFP4, true);
  }
  if (aff) {
    if (one) ZMOE_QMV_CASE(1, ZMOE_Q_AFFINE, false);
    ZMOE_QMV_CASE(4, ZMOE_Q_AFFINE, false);
  }
  if (one) ZMOE_QMV_CASE(1, ZMOE_Q_MXFP4, false);
  ZMOE_QMV_CASE(4, ZMOE_Q_MXFP4, false);
#undef ZMOE_QMV_CASE
}

}  // namespace zmoe

using namespace zmoe;

extern "C" int zmoe_gather_qmm_swiglu(void* stream, const void* x, int64_t x_batch, const uint32_t* gate_w,
                                      const void* gate_s, const void* gate_b, const uint32_t* up_w,
                                      const void* up_s, const void* up_b, const uint32_t* lhs_indices,
                                      const uint32_t* rhs_indices, int64_t n_pairs, int M, int N, int K, int E,
                                      int group_size, int bits, int quant_mode, void* out) {
  int gshift = 0;
  int rc = validate_qmm("gather_qmm_swiglu", x, x_batch, gate_w, gate_s, gate_b, lhs_indices, rhs_indices,
                        n_pairs, M, N, K, E, group_size, bits, quant_mode, out, &gshift);
  if (rc) return rc;
  ZMOE_REQUIRE(n_pairs == 0 || (up_w && up_s && (quant_mode != ZMOE_Q_AFFINE || up_b)), ZMOE_EINVAL_SHAPE,
               "[gather_qmm_swiglu] null up-projection pointer.");
  ZMOE_REQUIRE((reinterpret_cast<uintptr_t>(up_w) & 15) == 0, ZMOE_EINVAL_SHAPE,
               "[gather_qmm_swiglu] weights must be 16-byte aligned.");
  return dispatch_qmv(true, stream, x, gate_w, gate_s, gate_b, up_w, up_s, up_b, lhs_indices, rhs_indices, 1,
                      n_pairs, M, N, K, quant_mode, gshift, out);
}

extern "C" int zmoe_gather_qmm(void* stream, const void* x, int64_t x_batch, const uint32_t* w, const void* scales,
                               const void* biases, const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                               int64_t n_pairs, int M, int N, int K, int E, int group_size, int bits,
                               int quant_mode, void* out) {
  int gshift = 0;
  int rc = validate_qmm("gather_qmm", x, x_batch, w, scales, biases, lhs_indices, rhs_indices, n_pairs, M, N, K,
                        E, group_size, bits, quant_mode, out, &gshift);
  if (rc) return rc;
  return dispatch_qmv(false, stream, x, w, scales, biases, nullptr, nullptr, nullptr, lhs_indices, rhs_indices, 1,
                      n_pairs, M, N, K, quant_mode, gshift, out);
}
