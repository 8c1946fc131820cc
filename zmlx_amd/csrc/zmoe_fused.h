// Pieces shared by the single-launch decode kernels (layer_fused.hip, the
// general small-batch kernel, and decode1.hip, the one-token kernel): launch
// shape, kernel parameters, the workspace's tagged cross-workgroup data, and
// the loaders and dot-product helpers both kernels use so that their
// arithmetic is identical.
#pragma once

#include "zmoe_combine.h"
#include "zmoe_common.h"
#include "zmoe_host.h"
#include "zmoe_route.h"

namespace zmoe {

constexpr int kFThreads = 512;
constexpr int kFWaves = kFThreads / kWave;
constexpr int kFMaxB = 8;                 // tokens per call on the fused path
constexpr int kFMaxUnits = kFMaxB * kMaxTopK + 1;
constexpr int kChunkA = 4;                // (row-group, segment) items per batch, phase A
constexpr int kChunkD = 4;                // (slot-group, segment) items per batch, phase D
constexpr unsigned kSpinLimit = 1u << 18;  // default polls before a wait gives up
constexpr int kTraceSlots = 24;
// words of the workspace's leading state block
constexpr int kErrWord = static_cast<int>(kSyncErrorByte / 4);
constexpr int kEpochWord = 64;  // + workgroup: launches completed
constexpr int kMaxGrid = static_cast<int>(kSyncBlockBytes / 4) - kEpochWord;
constexpr int kMaxNC = 16;                // router chunks of 512 (H <= 8192)

// Launch constants of the one-token kernel's work assignment (host-made).
struct D1Plan {
  int Uall;          // routed units + shared unit
  int rpw;           // output rows per wave (phase D)
  int perA;          // (unit, row-group) items per wave (phase A)
  int lLH, lLI;      // log2 of the lanes per row, K_in = H / K_in = I
  int TA, TD;        // segments per lane, phase A / phase D
  int rgu;           // row-groups per unit (phase A)
  int PB;             // act slots per down-projection pass (batched kernel)
  int shpre;          // one-token kernel, general H: the shared expert's gate/up rows before the routing wait
  FastDiv by_rgu, by_Uall, by_NC, by_W, by_I;
  int64_t wst[3], sst[3];  // per-expert strides: packed words, scale (= bias) bytes
};

struct FusedParams {
  int H, E, K, I, Is, B;
  int gshift, combine_mode;
  RouteArgs route;
  int LH, LI;            // lanes per row for K_in = H / K_in = I (= Is)
  const uint16_t* x;
  uint16_t* out;
  const uint16_t* wr;
  const uint32_t* w[6];  // gate, up, down, sh_gate, sh_up, sh_down
  const void* s[6];
  const void* b[6];
  unsigned* sync;        // state block (words kErrWord, kEpochWord + g)
  unsigned long long* rpart;  // [B][E][NC]: f32 bits | tag << 32
  uint32_t* act;         // [B*K + B][act_stride]: bf16 bits | (tag & 0xFFFF) << 16
  unsigned* aflag;       // one-token kernel: act arrival counters and its launch counts
  int act_stride;
  uint32_t* out_idx;
  float* out_w;
  unsigned long long* trace;  // nullable: [G][kTraceSlots] realtime stamps
  uint32_t* xy;          // XCD-partitioned one-token kernel: [8][H] tagged expert outputs (bf16 | tag << 16)
  unsigned* err_host;    // nullable host-visible flag, set when a wait gives up
  unsigned spin;         // polls before a wait gives up
  FastDiv by_S4H, by_SH, by_S4I, by_SI;  // staged-row items: S*4 and S per row
  D1Plan d1;
};

struct FusedLds {
  unsigned dead, pad_[3];  // word 0 of every single-launch kernel's LDS (wg_dead_word)
  int ulist[kFMaxUnits];   // expert of each unit (slot order = expert order)
  int ucount[kFMaxUnits];
  int upairs[kFMaxUnits][kFMaxB];
  int nunits;              // routed units; the shared unit (if any) is index nunits
  int slot_of[1024];
  RouteLds route[kFMaxB];
};

__device__ __forceinline__ void trace_mark(const FusedParams& p, int slot) {
  if (p.trace && threadIdx.x == 0) gstore(p.trace + blockIdx.x * kTraceSlots + slot, static_cast<unsigned long long>(wall_clock64()));
}

// Word 0 of the dynamic LDS of every single-launch kernel (the first member
// of its LDS struct): nonzero once a wait of the workgroup gave up.  Thread 0
// clears it at the start; the data the workgroup publishes afterwards and its
// outputs are NaN while it is set, so a failed exchange never yields a
// silently wrong result.
__device__ __forceinline__ ZMOE_LDS unsigned* wg_dead_word() {
  extern __shared__ unsigned zmoe_dyn_lds[];
  return (ZMOE_LDS unsigned*)zmoe_dyn_lds;
}
__device__ __forceinline__ void wg_dead_clear() {
  if (threadIdx.x == 0) *wg_dead_word() = 0u;
}
__device__ __forceinline__ bool wg_dead() {
  return __hip_atomic_load(wg_dead_word(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u;
}
constexpr uint32_t kBf16NaN = 0x7FC0u;
constexpr float kPoison = __builtin_nanf("");

// A wait gave up: the sticky error word, the workgroup's flag, and the
// host-visible flag if there is one.
__device__ __forceinline__ void wait_timeout_at(unsigned* sync, unsigned* err_host) {
  __hip_atomic_fetch_or((ZMOE_GLOBAL unsigned*)(sync + kErrWord), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_or(wg_dead_word(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (err_host) __hip_atomic_store(err_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void wait_timeout(const FusedParams& p) { wait_timeout_at(p.sync, p.err_host); }

// Router logits of one token, lane-strided (e = lane + 64 i): the H/512
// partials of each expert, summed in chunk order once every one of them
// carries `tag`, rounded to bf16 (the gate Linear returns bf16 logits).
template <int P>
__device__ __forceinline__ RowVals<P> poll_logits(const FusedParams& p, const unsigned long long* rp, int NC,
                                                  unsigned tag, int backoff = 0) {
  const int lane = __lane_id();
  RowVals<P> row;
  unsigned n = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int e = lane + 64 * i;
      if (e < p.E) {
        unsigned long long part[kMaxNC];
#pragma unroll
        for (int c = 0; c < kMaxNC; ++c)
          if (c < NC) part[c] = dev_load(rp + e * NC + c);
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < kMaxNC; ++c) {
          if (c < NC) {
            ok = ok && static_cast<unsigned>(part[c] >> 32) == tag;
            a += __uint_as_float(static_cast<uint32_t>(part[c]));  // chunks in order
          }
        }
        row.v[i] = round_bf16(a);
      } else {
        row.v[i] = -INFINITY;
      }
    }
    if (__all(ok)) break;
    if (++n > p.spin) {
      if (lane == 0) wait_timeout(p);
      break;
    }
    if (backoff) __builtin_amdgcn_s_sleep(1);
  }
  return row;
}

// bf16 rows -> LDS tile in the layout of qmv.hip (stage_x_row):
//   xs[((r*4 + j)*S + s)*4 + d], sums sx[r*S + s] (affine).
// DEV: read the rows with device-coherent 64-bit loads (rows written by
// other workgroups in this launch).
// Words per staged row in LDS: 16 per segment plus a 128-byte pad, so that
// lane groups reading the same segment of different rows (the down
// projection reads one row per unit) fall in different LDS banks.
__host__ __device__ constexpr int lds_row_words(int S) { return 16 * S + 32; }

// bf16 rows -> LDS tile, row r at word r * lds_row_words(S):
//   xs[r*RW + (j*S + s)*4 + d], sums sx[r*S + s] (affine),
// segment s of a row holding its 16 words as (e0,e4)(e1,e5)(e2,e6)(e3,e7)
// pairs (affine; natural pairs for mxfp4), quarter j.
// DEV: rows written by other workgroups in this launch, as tagged words
// (bf16 | tag<<16).  They are read first with ordinary loads (the 32
// workgroups of an XCD then share one fetch through its L2), and every item
// whose tags are not all current is re-read with device-coherent loads until
// they are.
template <int QMODE, bool DEV, int NI = 2>
__device__ __forceinline__ void stage_rows_lds(const FusedParams& p, const void* __restrict__ src, int64_t src_stride,
                                               int nrows, int S, uint32_t* xs, float* sx, unsigned tag16,
                                               FastDiv by_S4, FastDiv by_S, int backoff = 0) {
  // (row, segment, quarter) items, NI per thread per round, all of a round's
  // loads in flight together
  const int S4 = S * 4;
  const int RW = lds_row_words(S);
  const int n = nrows * S4;
  for (int i0 = threadIdx.x; i0 < n; i0 += NI * kFThreads) {
    uint4 v[NI];
    if (DEV) {
      const uint32_t want = tag16 << 16;
      const uint32_t* q[NI];
#pragma unroll
      for (int h = 0; h < NI; ++h) {
        const int i = min(i0 + h * kFThreads, n - 1);  // past the end: repeat a valid item
        const int r = fdiv(i, by_S4), rem = i - r * S4;
        q[h] = static_cast<const uint32_t*>(src) + r * src_stride + rem * 8;
      }
      uint4 w[NI][2];
#pragma unroll
      for (int h = 0; h < NI; ++h) {
        w[h][0] = gload(reinterpret_cast<const uint4*>(q[h]));
        w[h][1] = gload(reinterpret_cast<const uint4*>(q[h]) + 1);
      }
      auto current = [&](const uint4& a) {
        return ((a.x & 0xFFFF0000u) == want) && ((a.y & 0xFFFF0000u) == want) && ((a.z & 0xFFFF0000u) == want) &&
               ((a.w & 0xFFFF0000u) == want);
      };
      unsigned spins = 0;
      for (;;) {
        bool ok = true;
#pragma unroll
        for (int h = 0; h < NI; ++h) ok = ok && current(w[h][0]) && current(w[h][1]);
        if (ok) break;
        if (++spins > p.spin) {
          wait_timeout(p);
          break;
        }
        if (backoff) __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int h = 0; h < NI; ++h) {
          unsigned long long d[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) d[k] = dev_load(reinterpret_cast<const unsigned long long*>(q[h]) + k);
          w[h][0] = make_uint4(static_cast<uint32_t>(d[0]), static_cast<uint32_t>(d[0] >> 32),
                               static_cast<uint32_t>(d[1]), static_cast<uint32_t>(d[1] >> 32));
          w[h][1] = make_uint4(static_cast<uint32_t>(d[2]), static_cast<uint32_t>(d[2] >> 32),
                               static_cast<uint32_t>(d[3]), static_cast<uint32_t>(d[3] >> 32));
        }
      }
      auto pair = [](uint32_t lo, uint32_t hi) { return (lo & 0xFFFFu) | (hi << 16); };
#pragma unroll
      for (int h = 0; h < NI; ++h)
        v[h] = make_uint4(pair(w[h][0].x, w[h][0].y), pair(w[h][0].z, w[h][0].w), pair(w[h][1].x, w[h][1].y),
                          pair(w[h][1].z, w[h][1].w));
    } else {
#pragma unroll
      for (int h = 0; h < NI; ++h) {
        const int i = i0 + h * kFThreads;
        if (i < n) {
          const int r = fdiv(i, by_S4), rem = i - r * S4;
          v[h] = gload(reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + r * src_stride + rem * 8));
        }
      }
    }
#pragma unroll
    for (int h = 0; h < NI; ++h) {
      const int i = i0 + h * kFThreads;
      if (i < n) {
        const int r = fdiv(i, by_S4), rem = i - r * S4;
        const int s = rem >> 2, j = rem & 3;
        uint4 o;
        if (QMODE == ZMOE_Q_AFFINE) {
          o.x = (v[h].x & 0xFFFFu) | (v[h].z << 16);
          o.y = (v[h].x >> 16) | (v[h].z & 0xFFFF0000u);
          o.z = (v[h].y & 0xFFFFu) | (v[h].w << 16);
          o.w = (v[h].y >> 16) | (v[h].w & 0xFFFF0000u);
        } else {
          o = v[h];
        }
        *reinterpret_cast<uint4*>(xs + r * RW + (j * S + s) * 4) = o;
      }
    }
  }
  if (QMODE == ZMOE_Q_AFFINE) {
    lds_barrier();
    for (int i = threadIdx.x; i < nrows * S; i += kFThreads) {
      const int r = fdiv(i, by_S), s = i - r * S;
      float acc = 0.0f;
      for (int w = 0; w < 4; ++w) {
        // pairs (e0,e4) (e1,e5) (e2,e6) (e3,e7) summed in natural order:
        // (e0+e1) (e2+e3) (e4+e5) (e6+e7), as stage_x_row does
        const uint4 o = *reinterpret_cast<const uint4*>(xs + r * RW + (w * S + s) * 4);
        acc += bf16_bits_to_f32(o.x & 0xFFFFu) + bf16_bits_to_f32(o.y & 0xFFFFu);
        acc += bf16_bits_to_f32(o.z & 0xFFFFu) + bf16_bits_to_f32(o.w & 0xFFFFu);
        acc += bf16_bits_to_f32(o.x >> 16) + bf16_bits_to_f32(o.y >> 16);
        acc += bf16_bits_to_f32(o.z >> 16) + bf16_bits_to_f32(o.w >> 16);
      }
      sx[r * S + s] = acc;
    }
  }
}

template <int QMODE>
__device__ __forceinline__ float seg_dot_lds(const uint4 w, const uint32_t* xs, int S, int r, int s, AffineK k) {
  const uint32_t* row = xs + r * lds_row_words(S);
  const uint4 x0 = *reinterpret_cast<const uint4*>(row + ((0 * S) + s) * 4);
  const uint4 x1 = *reinterpret_cast<const uint4*>(row + ((1 * S) + s) * 4);
  const uint4 x2 = *reinterpret_cast<const uint4*>(row + ((2 * S) + s) * 4);
  const uint4 x3 = *reinterpret_cast<const uint4*>(row + ((3 * S) + s) * 4);
  return seg_dot<QMODE>(w, x0, x1, x2, x3, k);
}

// Quantisation parameters of one (row, segment): loaded raw, decoded at use
// (decoding right after the load would make the load's wait immediate).
struct RawParam {
  uint32_t s, b;
};

template <int QMODE>
__device__ __forceinline__ RawParam seg_param_load(const void* __restrict__ scales, const void* __restrict__ biases,
                                                   int64_t idx) {
  RawParam r;
  if (QMODE == ZMOE_Q_AFFINE) {
    r.s = gload(static_cast<const uint16_t*>(scales) + idx);
    r.b = gload(static_cast<const uint16_t*>(biases) + idx);
  } else {
    r.s = gload(static_cast<const uint8_t*>(scales) + idx);
    r.b = 0;
  }
  return r;
}

template <int QMODE>
__device__ __forceinline__ void seg_param_decode(RawParam r, float& s, float& c) {
  if (QMODE == ZMOE_Q_AFFINE) {
    s = bf16_bits_to_f32(r.s);
    c = bf16_bits_to_f32(r.b) - 128.0f * s;
  } else {
    s = e8m0_to_f32(r.s);
    c = 0.0f;
  }
}

// Dequantised bf16 pairs of one 16-byte weight segment, in the order
// seg_dot consumes them (word x: pairs of nibbles (0,4) (1,5) (2,6) (3,7)).
template <int QMODE>
__device__ __forceinline__ void seg_dequant(const uint4 w, uint32_t (&d)[16], AffineK k) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (QMODE == ZMOE_Q_AFFINE) {
      d[4 * i + 0] = (ws[i] & k.m) | k.o;
      d[4 * i + 1] = ((ws[i] >> 4) & k.m) | k.o;
      d[4 * i + 2] = ((ws[i] >> 8) & k.m) | k.o;
      d[4 * i + 3] = ((ws[i] >> 12) & k.m) | k.o;
    } else {
      d[4 * i + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws[i], 1.0f, 0));
      d[4 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws[i], 1.0f, 1));
      d[4 * i + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws[i], 1.0f, 2));
      d[4 * i + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws[i], 1.0f, 3));
    }
  }
}

// seg_dot on dequantised pairs: one chain of 16 dot2 in seg_dot's order.
__device__ __forceinline__ float seg_dot_dq(const uint32_t (&d)[16], const uint32_t* xrow, int S, int s) {
  float v = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 x = *reinterpret_cast<const uint4*>(xrow + (i * S + s) * 4);
    v = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[4 * i + 0]), __builtin_bit_cast(bf16x2_t, x.x), v, false);
    v = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[4 * i + 1]), __builtin_bit_cast(bf16x2_t, x.y), v, false);
    v = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[4 * i + 2]), __builtin_bit_cast(bf16x2_t, x.z), v, false);
    v = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[4 * i + 3]), __builtin_bit_cast(bf16x2_t, x.w), v, false);
  }
  return v;
}

// One-token kernel (decode1.hip): used by launch_fused for B = 1 when it
// supports the shape (ZMOE_DECODE1=0 in the environment turns it off).
bool decode1_supported(const zmoe_layer_desc* d, int grid);
// XCD-partitioned one-token kernel (decode1.hip): tried first by
// launch_decode1 (ZMOE_DECODE1X=0 turns it off).  Workspace beyond the
// one-token kernel's: the router partials of each XCD (xcd_rpart_bytes at
// fp.rpart) and the tagged expert outputs (xcd_xy_bytes at fp.xy).
size_t xcd_rpart_bytes(const zmoe_layer_desc* d);
size_t xcd_xy_bytes(const zmoe_layer_desc* d);
// Launches it when it applies (returns its status), else returns -1.
int try_decode1x(hipStream_t st, const zmoe_layer_desc* d, const FusedParams& fp, int grid);
int launch_decode1(hipStream_t st, const zmoe_layer_desc* d, const FusedParams& fp, int grid);
// Batched kernel (decodeb.hip): 2 <= B <= 16 at hidden 2048
// (ZMOE_DECODEB=0 turns it off).
bool decodeb_supported(const zmoe_layer_desc* d, int B, int grid);
int launch_decodeb(hipStream_t st, const zmoe_layer_desc* d, const FusedParams& fp, int grid);

}  // namespace zmoe
