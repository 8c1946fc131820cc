// Pieces of the one-token kernels (decode1.hip: k_moe_decode1; decode1x.hip:
// the XCD-partitioned k_moe_decode1x): the workgroup's LDS header with the
// routing results and the per-unit pointer table, and the parallel ranking
// that selects the routed experts.
#pragma once

#include "zmoe_fused.h"

#include <cstddef>

namespace zmoe {

constexpr int kD1MaxUnits = kMaxTopK + 1;
constexpr int kD1A = 4;  // gate/up items per batch
constexpr int kD1D = 4;  // down items per batch
constexpr int kD1RankMaxE = 256;  // parallel ranking for E <= this


struct D1Lds {
  unsigned dead, pad_[3];  // word 0 of every single-launch kernel's LDS (wg_dead_word)
  RouteLds route;
  // packed (bf16 order key << 16 | 0xFFFF - e); the grouped sigmoid
  // router's 64-bit keys use all of it
  uint32_t keys[2 * kD1RankMaxE];
  const uint32_t* w[3][kD1MaxUnits];  // matrix (gate, up, down) x unit
  const void* s[3][kD1MaxUnits];
  const void* b[3][kD1MaxUnits];
};
static_assert(offsetof(D1Lds, keys) % 16 == 0, "keys are read as 16-byte vectors");

// Unit u's pointers for matrix m (0 gate, 1 up, 2 down): routed expert e, or
// the shared expert for e < 0.
__device__ __forceinline__ void set_unit_e(const FusedParams& p, D1Lds& L, int u, int m, int e) {
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

// Rank of key i (number of larger keys; keys are unique) over an EPAD-entry
// row, Q = 512/EPAD adjacent threads per key, each counting one slice.
// Returns the rank in thread q == 0 of each group (-1 elsewhere).
template <int EPAD>
__device__ __forceinline__ int rank_in_row(const uint32_t* keys, int& i, uint32_t& ki) {
  constexpr int Q = kFThreads / EPAD;
  constexpr int PER = EPAD / Q;
  static_assert(Q >= 2 && Q <= 8 && PER % 4 == 0, "rank slices");
  i = threadIdx.x / Q;
  const int q = threadIdx.x % Q;
  ki = keys[i];
  uint4 kk[PER / 4];
#pragma unroll
  for (int c = 0; c < PER / 4; ++c) kk[c] = *reinterpret_cast<const uint4*>(&keys[q * PER + 4 * c]);
  int c0 = 0, c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
  for (int c = 0; c < PER / 4; ++c) {
    c0 += kk[c].x > ki ? 1 : 0;
    c1 += kk[c].y > ki ? 1 : 0;
    c2 += kk[c].z > ki ? 1 : 0;
    c3 += kk[c].w > ki ? 1 : 0;
  }
  int cnt = (c0 + c1) + (c2 + c3);
  cnt += __builtin_amdgcn_update_dpp(0, cnt, kDppQuadSwap1, 0xF, 0xF, false);
  if (Q >= 4) cnt += __builtin_amdgcn_update_dpp(0, cnt, kDppQuadSwap2, 0xF, 0xF, false);
  if (Q >= 8) cnt += __builtin_amdgcn_update_dpp(0, cnt, kDppHalfMirror, 0xF, 0xF, false);
  return q == 0 ? cnt : -1;
}

// Rank of 64-bit key i (number of larger keys; keys are unique) over an
// EPAD-entry row, Q = 512/EPAD adjacent threads per key, each counting one
// slice in chunks of up to 16 keys.  Returns the rank in thread q == 0 of each
// group (-1 elsewhere).
template <int EPAD>
__device__ __forceinline__ int rank_in_row64(const uint64_t* keys, int& i, uint64_t& ki) {
  constexpr int Q = kFThreads / EPAD;
  constexpr int PER = EPAD / Q;
  constexpr int CH = PER < 16 ? PER : 16;  // keys per chunk
  static_assert(Q >= 2 && Q <= 8 && PER % CH == 0 && CH % 2 == 0, "rank slices");
  i = threadIdx.x / Q;
  const int q = threadIdx.x % Q;
  ki = keys[i];
  int cnt = 0;
  for (int c = 0; c < PER; c += CH) {
    uint4 kk[CH / 2];
#pragma unroll
    for (int m = 0; m < CH / 2; ++m) kk[m] = *reinterpret_cast<const uint4*>(&keys[q * PER + c + 2 * m]);
#pragma unroll
    for (int m = 0; m < CH / 2; ++m) {
      cnt += ((static_cast<uint64_t>(kk[m].y) << 32 | kk[m].x) > ki) ? 1 : 0;
      cnt += ((static_cast<uint64_t>(kk[m].w) << 32 | kk[m].z) > ki) ? 1 : 0;
    }
  }
  cnt += __builtin_amdgcn_update_dpp(0, cnt, kDppQuadSwap1, 0xF, 0xF, false);
  if (Q >= 4) cnt += __builtin_amdgcn_update_dpp(0, cnt, kDppQuadSwap2, 0xF, 0xF, false);
  if (Q >= 8) cnt += __builtin_amdgcn_update_dpp(0, cnt, kDppHalfMirror, 0xF, 0xF, false);
  return q == 0 ? cnt : -1;
}

// Gate weights of the ranked winners (wave 0; lane r < K holds winner r),
// then the routing outputs of workgroup 0.
__device__ __forceinline__ void rank_weights(const FusedParams& p, D1Lds& L, int K) {
  const int lane = __lane_id();
  const float val = lane < K ? L.route.sval[lane] : 0.0f;
  float w;
  if (p.route.kind == kRouteSoftmaxProbs) {
    const float sb = round_bf16(ordered_lane_sum(val, K));
    w = p.route.norm ? div_to_bf16(val, sb) : val;
  } else {
    // moe.topk_gating_softmax renorm path (moe.py:1239-1396)
    const float m = readlane_f(val, 0);
    const float ex = expf(val - m);
    const float sum = ordered_lane_sum(ex, K);
    w = ex / sum;
    if (p.route.w_bf16) w = round_bf16(w);
  }
  if (lane < K) {
    L.route.w[lane] = w;
    if (blockIdx.x == 0) {
      if (p.out_idx) gstore(p.out_idx + lane, static_cast<uint32_t>(L.route.sel[lane]));
      if (p.out_w) gstore(p.out_w + lane, w);
    }
  }
}

}  // namespace zmoe
