// Router kernels: dense router projection and the top-k gating variants.
// One wave owns one token row for the top-k kernels; the selection order is
// "higher value first, lower expert index on ties" (zmoe_wave.h).
#include "zmoe_common.h"
#include "zmoe_host.h"
#include "zmoe_route.h"

namespace zmoe {

constexpr int kRouterMaxE = 1024;
constexpr int kRouterMaxK = kMaxTopK;

// ---------------------------------------------------------------------------
// Dense router projection: logits[b, e] = x[b, :] . w[e, :]
// ---------------------------------------------------------------------------
// TOK tokens per block: 2 for decode batches up to 32 (more workgroups,
// shorter wave-sum chains), 4 above (each token group re-reads the router
// matrix, so larger batches take fewer groups)
constexpr int kLogitTokMax = 4;
constexpr int kLogitRows = 1;  // rows per wave (short dependent chains: one row of wave sums per wave)
constexpr int kLogitXv = 4;  // 16-byte x loads per thread per staging batch
// PRE: 512-element chunks of a row loaded together (4 at hidden <= 2048, else 8)
template <int TOK, int PRE>
__global__ __launch_bounds__(256) void k_dense_logits(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      int B, int E, int H, int out_f32, void* __restrict__ out) {
  extern __shared__ __align__(16) uint32_t xsm[];  // TOK * H bf16
  const int b0 = blockIdx.y * TOK;
  const int nt = min(TOK, B - b0);
  const int hw = H >> 1;  // dwords per row
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int e0 = (blockIdx.x * 4 + wave) * kLogitRows;
  const int nch = (H + 511) / 512;  // chunks of 512 elements (8 per lane)
  // The router rows are cold in HBM: every chunk of a batch is loaded before
  // any is used (and the first batch before the x staging), so a wave waits
  // for one HBM round trip per batch instead of one per chunk.  Addresses are
  // clamped and the lanes past H zeroed after the load, so the loads carry no
  // branch.
  uint4 wv[PRE][kLogitRows];
  auto load_batch = [&](int cb) {
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
      const int h = (cb + j) * 512 + lane * 8;
      const int hc = min(h, H - 8);
#pragma unroll
      for (int r = 0; r < kLogitRows; ++r) {
        const int e = min(e0 + r, E - 1);
        const uint4 v = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(e) * H + hc);
        wv[j][r] = h < H ? v : make_uint4(0, 0, 0, 0);
      }
    }
  };
  load_batch(0);
  {
    // x staged with 16-byte loads, a batch of kLogitXv per thread in flight
    // before its LDS stores
    const uint4* xg = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(b0) * H);
    uint4* xs = reinterpret_cast<uint4*>(xsm);
    const int nv = nt * (H >> 3);
    for (int i0 = 0; i0 < nv; i0 += kLogitXv * 256) {
      uint4 v[kLogitXv];
#pragma unroll
      for (int j = 0; j < kLogitXv; ++j) v[j] = xg[min(i0 + j * 256 + static_cast<int>(threadIdx.x), nv - 1)];
#pragma unroll
      for (int j = 0; j < kLogitXv; ++j)
        if (i0 + j * 256 + static_cast<int>(threadIdx.x) < nv) xs[i0 + j * 256 + threadIdx.x] = v[j];
    }
  }
  __syncthreads();
  if (e0 >= E) return;
  float acc[kLogitRows][TOK];
#pragma unroll
  for (int r = 0; r < kLogitRows; ++r)
#pragma unroll
    for (int t = 0; t < TOK; ++t) acc[r][t] = 0.0f;

  // each chunk's dot is reduced across the wave, then chunks are added in
  // order -- the same order as the fused decode kernels, so both produce
  // identical logits.
  for (int cb = 0; cb < nch; cb += PRE) {
    if (cb > 0) load_batch(cb);
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
      if (cb + j >= nch) break;
      const int h = (cb + j) * 512 + lane * 8;
      const bool valid = h < H;
#pragma unroll
      for (int t = 0; t < TOK; ++t) {
        if (t < nt) {
          const uint4 xv = valid ? *reinterpret_cast<const uint4*>(xsm + t * hw + (h >> 1)) : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < kLogitRows; ++r) {
            float a = 0.0f;
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[j][r].x), __builtin_bit_cast(bf16x2_t, xv.x), a, false);
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[j][r].y), __builtin_bit_cast(bf16x2_t, xv.y), a, false);
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[j][r].z), __builtin_bit_cast(bf16x2_t, xv.z), a, false);
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv[j][r].w), __builtin_bit_cast(bf16x2_t, xv.w), a, false);
            acc[r][t] += wave_sum(a);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kLogitRows; ++r) {
#pragma unroll
    for (int t = 0; t < TOK; ++t) {
      const float v = acc[r][t];
      if (lane == 0 && t < nt && e0 + r < E) {
        const int64_t o = static_cast<int64_t>(b0 + t) * E + e0 + r;
        if (out_f32)
          static_cast<float*>(out)[o] = v;
        else
          static_cast<uint16_t*>(out)[o] = static_cast<uint16_t>(f32_to_bf16_bits(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Top-k gating kernels: one wave per token row (4 rows per block); the row is
// staged in wave-private LDS and routed by route_row (zmoe_route.h), the same
// code the single-launch layer kernel runs.
// ---------------------------------------------------------------------------
struct RouterBlockLds {
  float grow[4][kRouterMaxE];
  RouteLds r[4];
};

__global__ __launch_bounds__(256) void k_route_rows(const void* __restrict__ logits, int dtype, int B, RouteArgs a,
                                                    int out_bf16, void* __restrict__ out_w,
                                                    uint32_t* __restrict__ out_idx) {
  __shared__ RouterBlockLds S;
  const int wave = threadIdx.x / kWave;
  const int row = blockIdx.x * 4 + wave;
  if (row >= B) return;  // wave-private LDS only: no block barriers
  const int lane = __lane_id();
  const int64_t base = static_cast<int64_t>(row) * a.E;
  route_row_any(
      a,
      [&](int e) {
        return (dtype == ZMOE_DT_F32) ? static_cast<const float*>(logits)[base + e]
                                      : bf16_bits_to_f32(static_cast<const uint16_t*>(logits)[base + e]);
      },
      *(ZMOE_LDS RouteLds*)(&S.r[wave]), (ZMOE_LDS float*)(S.grow[wave]));
  if (lane < a.k) {
    const int64_t o = static_cast<int64_t>(row) * a.k + lane;
    const float w = S.r[wave].w[lane];
    if (out_bf16)
      static_cast<uint16_t*>(out_w)[o] = static_cast<uint16_t>(f32_to_bf16_bits(w));
    else
      static_cast<float*>(out_w)[o] = w;
    out_idx[o] = static_cast<uint32_t>(S.r[wave].sel[lane]);
  }
}

static int launch_route(hipStream_t st, const void* logits, int dtype, int B, const RouteArgs& a, int out_bf16,
                        void* out_w, uint32_t* out_idx, const char* what) {
  hipLaunchKernelGGL(k_route_rows, dim3((B + 3) / 4), dim3(256), 0, st, logits, dtype, B, a, out_bf16, out_w,
                     out_idx);
  return check_launch(what);
}

static RouteArgs make_args(int kind, int E, int k, int norm, const float* bias, int n_group, int topk_group,
                           float scale, int w_bf16) {
  RouteArgs a;
  a.kind = kind;
  a.E = E;
  a.k = k;
  a.norm = norm;
  a.bias = bias;
  a.n_group = n_group;
  a.topk_group = topk_group;
  a.scale = scale;
  a.w_bf16 = w_bf16;
  return a;
}

static int check_router(const char* op, int B, int E, int k) {
  const std::string tag = std::string("[") + op + "] ";
  ZMOE_REQUIRE(B >= 0 && E >= 1 && E <= kRouterMaxE, ZMOE_EINVAL_SHAPE, tag + "need 1 <= E <= 1024.");
  ZMOE_REQUIRE(k >= 1, ZMOE_EINVAL_SHAPE, tag + "k must be > 0");
  ZMOE_REQUIRE(k <= E, ZMOE_EINVAL_SHAPE, tag + "k=" + std::to_string(k) + " exceeds last dimension D=" + std::to_string(E));
  ZMOE_REQUIRE(k <= kRouterMaxK, ZMOE_EUNSUPPORTED, tag + "k must be <= 16.");
  return ZMOE_OK;
}

// Internal launchers for the layer composition (arguments pre-validated).
int launch_topk_gating(hipStream_t st, const void* logits, int in_dtype, int B, int E, int k, const float* bias,
                       int norm, int out_bf16, void* out_w, uint32_t* out_idx) {
  return launch_route(st, logits, in_dtype, B, make_args(kRouteTopkLogits, E, k, norm, bias, 1, 1, 1.0f, out_bf16),
                      out_bf16, out_w, out_idx, "topk_gating_softmax");
}

int launch_deepseek_router(hipStream_t st, const void* logits, int in_dtype, const float* bias, int B, int E, int k,
                           int n_group, int topk_group, float scaling, float* out_w, uint32_t* out_idx) {
  return launch_route(st, logits, in_dtype, B,
                      make_args(kRouteSigmoidGrouped, E, k, 1, bias, n_group, topk_group, scaling, 0), 0, out_w,
                      out_idx, "deepseek_router_topk_sigmoid");
}

}  // namespace zmoe

using namespace zmoe;

extern "C" int zmoe_dense_logits(void* stream, const void* x, const void* w, int B, int E, int H, int out_dtype,
                                 void* out) {
  ZMOE_REQUIRE(B >= 0 && E >= 1 && H >= 8 && H % 8 == 0, ZMOE_EINVAL_SHAPE, "[dense_logits] need H % 8 == 0.");
  ZMOE_REQUIRE(out_dtype == ZMOE_DT_BF16 || out_dtype == ZMOE_DT_F32, ZMOE_EINVAL_DTYPE,
               "[dense_logits] out dtype must be bf16 or f32.");
  ZMOE_REQUIRE(static_cast<int64_t>(kLogitTokMax) * H * 2 <= 64 * 1024, ZMOE_EUNSUPPORTED, "[dense_logits] H too large.");
  if (B == 0) return ZMOE_OK;
  ZMOE_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
               ZMOE_EINVAL_SHAPE, "[dense_logits] x and w must be 16-byte aligned.");
  const int tok = B <= 32 ? 2 : kLogitTokMax;
  dim3 grid((E + 4 * kLogitRows - 1) / (4 * kLogitRows), (B + tok - 1) / tok);
  auto fn = tok == 2 ? (H <= 2048 ? k_dense_logits<2, 4> : k_dense_logits<2, 8>)
                     : (H <= 2048 ? k_dense_logits<kLogitTokMax, 4> : k_dense_logits<kLogitTokMax, 8>);
  hipLaunchKernelGGL(fn, grid, dim3(256), static_cast<size_t>(tok) * H * 2, as_stream(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), B, E, H,
                     out_dtype == ZMOE_DT_F32 ? 1 : 0, out);
  return check_launch("dense_logits");
}

// ---------------------------------------------------------------------------
// Router projection for prefill batches on MFMA: a workgroup of 8 waves owns
// a 16-token x 16-expert tile (256 workgroups at 512 tokens x 128 experts, so
// every CU streams its share); wave w of 8 takes the k range
// [w*H/8, (w+1)*H/8) with v_mfma_f32_16x16x32_bf16 (bf16 products exact, fp32
// accumulation) and the 8 partial tiles are added in wave order through LDS.
// Used by the layer for batches on the grouped path, where no single-launch
// kernel has to reproduce its logits bit for bit.
// ---------------------------------------------------------------------------
typedef __bf16 lg_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float lg_f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kLgSteps = 4;  // k-steps of 32 per load batch
constexpr int kLgWaves = 8;  // waves per tile, each a k range
constexpr int kLgPieces = 32;  // 8-element pieces of one wave's k range (hidden 2048) with group sums

// With xsum (affine grouped GEMMs), the workgroups of the first expert tile
// also write the fp32 sums of every gs-group of their 16 token rows,
// xsum[b][H / gs], from the x values they hold: each lane's 8 consecutive
// values are summed as k_row_group_sums sums an 8-element piece, the pieces
// of a group are then added in k order, so the sums are bit-identical to
// k_row_group_sums'.
__global__ __launch_bounds__(512) void k_logits_mfma(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     int B, int E, int H, int out_f32, void* __restrict__ out,
                                                     float* __restrict__ xsum, int gs) {
  __shared__ float red[kLgWaves - 1][kWave][5];
  __shared__ float piece[kLgWaves][16][kLgPieces + 1];  // 8-element sums: [wave][token][piece]
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int q = lane >> 4, col = lane & 15;  // k quarter (8 of every 32 k), row in the tile
  const int b0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
  const int64_t xr = min(b0 + col, B - 1), wr = min(e0 + col, E - 1);
  const int kq = H / kLgWaves;  // k per wave
  const uint16_t* xp = x + xr * H + wave * kq + q * 8;
  const uint16_t* wp = w + wr * H + wave * kq + q * 8;
  const int nch = kq / (32 * kLgSteps);  // load batches per wave (even)
  const bool sums = xsum != nullptr && blockIdx.y == 0;
  lg_f32x4_t acc = {};
  // two register buffers in ping-pong, loads issued unconditionally (the
  // batch index clamped) so the compiler's wait counts stay exact
  uint4 xa[kLgSteps], wa[kLgSteps], xb[kLgSteps], wb[kLgSteps];
  auto load = [&](uint4* xv, uint4* wv, int c) {
#pragma unroll
    for (int i = 0; i < kLgSteps; ++i) {
      xv[i] = gload(reinterpret_cast<const uint4*>(xp + (c * kLgSteps + i) * 32));
      wv[i] = gload(reinterpret_cast<const uint4*>(wp + (c * kLgSteps + i) * 32));
    }
  };
  auto mfma = [&](const uint4* xv, const uint4* wv, int c) {
#pragma unroll
    for (int i = 0; i < kLgSteps; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(lg_bf16x8_t, xv[i]),
                                                    __builtin_bit_cast(lg_bf16x8_t, wv[i]), acc, 0, 0, 0);
    if (sums) {
      // piece (c * kLgSteps + i) * 4 + q of this wave's k range: elements
      // wave * kq + (c * kLgSteps + i) * 32 + q * 8 .. + 7 of token col
#pragma unroll
      for (int i = 0; i < kLgSteps; ++i) {
        const uint4 v = xv[i];
        const float t = (((bf16_bits_to_f32(v.x & 0xFFFFu) + bf16_bits_to_f32(v.x >> 16)) +
                          (bf16_bits_to_f32(v.y & 0xFFFFu) + bf16_bits_to_f32(v.y >> 16))) +
                         (bf16_bits_to_f32(v.z & 0xFFFFu) + bf16_bits_to_f32(v.z >> 16))) +
                        (bf16_bits_to_f32(v.w & 0xFFFFu) + bf16_bits_to_f32(v.w >> 16));
        piece[wave][col][(c * kLgSteps + i) * 4 + q] = t;
      }
    }
  };
  load(xa, wa, 0);
  for (int c = 0; c < nch; c += 2) {
    load(xb, wb, c + 1);
    mfma(xa, wa, c);
    load(xa, wa, min(c + 2, nch - 1));
    mfma(xb, wb, c + 1);
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave - 1][lane][i] = acc[i];
  }
  __syncthreads();
  if (sums) {
    // this wave's kq / gs groups of the 16 tokens, pieces added in k order
    const int ppg = gs / 8, gpw = kq / gs;
    for (int it = lane; it < 16 * gpw; it += kWave) {
      const int tok = it & 15, gg = it >> 4;
      float sv = 0.0f;
      for (int j = 0; j < ppg; ++j) sv += piece[wave][tok][gg * ppg + j];
      if (b0 + tok < B) xsum[static_cast<int64_t>(b0 + tok) * (H / gs) + wave * gpw + gg] = sv;
    }
  }
  if (wave != 0) return;
  // element i of the 16x16 tile: token row 4*q + i, expert column col
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = acc[i];
#pragma unroll
    for (int r = 0; r < kLgWaves - 1; ++r) v += red[r][lane][i];
    const int b = b0 + q * 4 + i, e = e0 + col;
    if (b < B && e < E) {
      const int64_t o = static_cast<int64_t>(b) * E + e;
      if (out_f32)
        static_cast<float*>(out)[o] = v;
      else
        static_cast<uint16_t*>(out)[o] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
  }
}

int zmoe::launch_logits_mfma(hipStream_t st, const void* x, const void* w, int B, int E, int H, int out_dtype,
                             void* out, float* xsum, int gs) {
  ZMOE_REQUIRE(H % (2 * kLgWaves * kLgSteps * 32) == 0, ZMOE_EINVAL_SHAPE,
               "[dense_logits] hidden must be a multiple of 2048.");
  ZMOE_REQUIRE(xsum == nullptr || ((gs == 32 || gs == 64 || gs == 128) && H / kLgWaves <= kLgPieces * 8),
               ZMOE_EINVAL_SHAPE, "[dense_logits] group sums: gs 32, 64 or 128 and hidden at most 2048.");
  if (B == 0) return ZMOE_OK;
  hipLaunchKernelGGL(k_logits_mfma, dim3((B + 15) / 16, (E + 15) / 16), dim3(kLgWaves * kWave), 0, st,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), B, E, H,
                     out_dtype == ZMOE_DT_F32 ? 1 : 0, out, xsum, gs);
  return check_launch("dense_logits (mfma)");
}

extern "C" int zmoe_router_softmax_topk(void* stream, const void* logits, int B, int E, int k, int norm_topk_prob,
                                        void* out_w, uint32_t* out_idx) {
  int rc = check_router("router_softmax_topk", B, E, k);
  if (rc) return rc;
  if (B == 0) return ZMOE_OK;
  return launch_route(as_stream(stream), logits, ZMOE_DT_BF16, B,
                      make_args(kRouteSoftmaxProbs, E, k, norm_topk_prob ? 1 : 0, nullptr, 1, 1, 1.0f, 1), 1, out_w,
                      out_idx, "router_softmax_topk");
}

extern "C" int zmoe_topk_gating_softmax(void* stream, const void* logits, int in_dtype, int B, int E, int k,
                                        const float* expert_bias, int norm_topk_prob, float* out_w,
                                        uint32_t* out_idx) {
  int rc = check_router("topk_gating_softmax", B, E, k);
  if (rc) return rc;
  ZMOE_REQUIRE(in_dtype == ZMOE_DT_BF16 || in_dtype == ZMOE_DT_F32, ZMOE_EINVAL_DTYPE,
               "[topk_gating_softmax] logits must be bf16 or f32.");
  if (B == 0) return ZMOE_OK;
  return launch_topk_gating(as_stream(stream), logits, in_dtype, B, E, k, expert_bias, norm_topk_prob ? 1 : 0, 0,
                            out_w, out_idx);
}

extern "C" int zmoe_deepseek_router_topk_sigmoid(void* stream, const float* logits, const float* bias, int B, int E,
                                                 int k, int n_group, int topk_group, float routed_scaling_factor,
                                                 float* out_w, uint32_t* out_idx) {
  int rc = check_router("deepseek_router_topk_sigmoid", B, E, k);
  if (rc) return rc;
  ZMOE_REQUIRE(n_group > 0, ZMOE_EINVAL_SHAPE, "[deepseek_router_topk_sigmoid] n_group must be > 0");
  ZMOE_REQUIRE(topk_group > 0 && topk_group <= n_group, ZMOE_EINVAL_SHAPE,
               "[deepseek_router_topk_sigmoid] invalid topk_group");
  ZMOE_REQUIRE(E % n_group == 0, ZMOE_EINVAL_SHAPE, "[deepseek_router_topk_sigmoid] n_group must divide D");
  ZMOE_REQUIRE(n_group <= kWave, ZMOE_EUNSUPPORTED, "[deepseek_router_topk_sigmoid] n_group must be <= 64");
  ZMOE_REQUIRE(bias != nullptr, ZMOE_EINVAL_SHAPE, "[deepseek_router_topk_sigmoid] bias must have shape (D,)");
  if (B == 0) return ZMOE_OK;
  return launch_deepseek_router(as_stream(stream), logits, ZMOE_DT_F32, bias, B, E, k, n_group, topk_group,
                                routed_scaling_factor, out_w, out_idx);
}
