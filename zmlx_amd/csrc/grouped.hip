// Grouped (per-expert) quantized GEMM on MFMA: the batched / prefill path.
//
// For many tokens the (token, expert) pairs are counting-sorted by expert
// and every expert's weights are streamed once for all of its rows (the role
// of mlx_lm's SwitchGLU sort path + gather_qmm(sorted_indices=True) that the
// reference keeps for M > 1, moe_mlp.py:540-543).
//
// Tiles: a workgroup of 8 waves owns (expert e, a chunk of up to 64 of its
// sorted rows, 256 output rows n); wave w computes n0 = 256*tile + 32*w .. +31
// for both 32-row blocks of the chunk with v_mfma_f32_32x32x16_bf16, so each
// weight load feeds two blocks.  Per 64-k block the chunk's activations are
// loaded once by the whole workgroup into LDS (one 16-byte load per thread,
// double-buffered) and read from there by every wave.  Chunks come from the
// sort kernel's list, so a heavy expert spreads over many workgroups.
//
// In-register dequant keeps the decode GEMV's exact products: the weight
// operand is the bf16 number 128+q (q = the 4-bit code, exact in bf16, made
// with one v_and_or per pair) and the activation operand is x itself, so
// every product (128+q)*x is exact in fp32.  Per quantisation group g:
//   acc_g = sum x*(128+q)                       (MFMA, fresh accumulator)
//   tot  += s_g * acc_g                         (16 FMAs per lane)
// and after the K loop the affine offset sum_g (b_g - 128 s_g) * sum_g(x)
// is one more small GEMM, done on v_mfma_f32_32x32x2f32 from precomputed
// per-group activation sums.  mxfp4: the operand comes from the gfx950
// e2m1 converter (scale 1, exact) and tot += 2^(e-127) * acc_g.
//
// k mapping.  An MFMA covers 16 k: lane half h holds 8 of them.  For groups
// of >= 64 the 8 words (64 k) of a block are split as h -> words h*4..h*4+3,
// k-step j -> word h*4+j, so a lane loads 16 contiguous bytes of weights
// and 64 of activations per block.  For groups of 32 (affine g32, mxfp4)
// k-step j uses word 2j+h, so one MFMA stays inside one group.  The affine
// operand pairs nibbles (i, i+4) of a word, so the activation pairs are
// permuted to (e0,e4) (e1,e5) (e2,e6) (e3,e7) in registers (v_perm).
#include "zmoe_common.h"
#include "zmoe_grouped.h"
#include "zmoe_host.h"

#include <string>
#include <type_traits>

namespace zmoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGThreads = 256;  // 4 waves
constexpr int kGWaves = kGThreads / 64;
constexpr int kGTileN = 32 * kGWaves;  // output rows per workgroup
constexpr int kGTileM = 32;            // sorted rows per MFMA block
constexpr int kGBlocksM = 1;           // MFMA blocks per chunk
constexpr int kGChunk = kGTileM * kGBlocksM;
constexpr int kGLdsRow = 64 + 8;       // bf16 per staged activation row (64 k + pad)
constexpr int kGStage = kGChunk * 8 / kGThreads;  // 16-byte staging pieces per thread
static_assert(kGChunk == kGroupedChunk && kGStage >= 1, "chunk");


// ---------------------------------------------------------------------------
// sort (token, k) pairs by expert: one workgroup, counts in LDS
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_sort_pairs(const uint32_t* __restrict__ idx, int npairs, int E, int chunk,
                                                     int* __restrict__ offsets, int* __restrict__ sorted,
                                                     int* __restrict__ blocks) {
  __shared__ int cnt[1024];
  __shared__ int off[1025];
  __shared__ int cst[1024];  // first chunk of each expert
  __shared__ int wtot[2][16];
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int q = threadIdx.x; q < npairs; q += blockDim.x) atomicAdd(&cnt[min(static_cast<int>(idx[q]), E - 1)], 1);
  __syncthreads();
  // exclusive scans of the pair counts and the chunk counts, thread e owns
  // expert e (E <= 1024): per-wave shuffle scans, then the wave totals
  {
    const int e = threadIdx.x, lane = e & (kWave - 1), wv = e / kWave;
    const int c = e < E ? cnt[e] : 0;
    const int nc = (c + chunk - 1) / chunk;
    int ic = c, inc = nc;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int t0 = __shfl_up(ic, o), t1 = __shfl_up(inc, o);
      if (lane >= o) ic += t0, inc += t1;
    }
    if (lane == kWave - 1) wtot[0][wv] = ic, wtot[1][wv] = inc;
    __syncthreads();
    int bc = 0, bnc = 0;
    for (int w = 0; w < wv; ++w) bc += wtot[0][w], bnc += wtot[1][w];
    if (e < E) {
      off[e] = bc + ic - c;
      cst[e] = bnc + inc - nc;
    }
    if (e == E - 1) {
      off[E] = bc + ic;
      if (blocks) offsets[E + 1] = bnc + inc;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) offsets[e] = off[e];
  if (blocks) {
    // chunks of `chunk` rows of every expert, in expert order
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      const int nbe = (off[e + 1] - off[e] + chunk - 1) / chunk;
      for (int j = 0; j < nbe; ++j) blocks[cst[e] + j] = e | (j << 11);
    }
  }
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  // position inside an expert's range is arbitrary: every row is computed
  // independently of the others
  for (int q = threadIdx.x; q < npairs; q += blockDim.x) {
    const int e = min(static_cast<int>(idx[q]), E - 1);
    sorted[off[e] + atomicAdd(&cnt[e], 1)] = q;
  }
}

// out[r][g] = sum of a[r][g*gs .. g*gs+gs) in fp32 (one thread per (r, g))
__global__ void k_row_group_sums(const uint16_t* __restrict__ a, int64_t lda, int rows, int K, int gs,
                                 float* __restrict__ out) {
  const int G = K / gs;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= static_cast<int64_t>(rows) * G) return;
  const int64_t r = t / G;
  const int g = static_cast<int>(t - r * G);
  const uint16_t* p = a + r * lda + static_cast<int64_t>(g) * gs;
  float s = 0.0f;
  for (int i = 0; i < gs; i += 8) {
    const uint4 v = gload(reinterpret_cast<const uint4*>(p + i));
    s += (bf16_bits_to_f32(v.x & 0xFFFFu) + bf16_bits_to_f32(v.x >> 16)) +
         (bf16_bits_to_f32(v.y & 0xFFFFu) + bf16_bits_to_f32(v.y >> 16)) +
         (bf16_bits_to_f32(v.z & 0xFFFFu) + bf16_bits_to_f32(v.z >> 16)) +
         (bf16_bits_to_f32(v.w & 0xFFFFu) + bf16_bits_to_f32(v.w >> 16));
  }
  out[t] = s;
}

// ---------------------------------------------------------------------------
// operand construction
// ---------------------------------------------------------------------------
__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint4 v = make_uint4(a, b, c, d);
  return __builtin_bit_cast(bf16x8_t, v);
}

// 8 consecutive activations (x0..x7 as natural pairs) -> (x0,x4) (x1,x5) (x2,x6) (x3,x7)
__device__ __forceinline__ bf16x8_t act_affine(uint4 v) {
  return as_bf16x8(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                   __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
}
__device__ __forceinline__ bf16x8_t act_natural(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// one packed word (8 codes) -> the 8-element weight operand
template <int QMODE>
__device__ __forceinline__ bf16x8_t wt_operand(uint32_t w, AffineK k) {
  if (QMODE == ZMOE_Q_AFFINE) {
    const uint32_t a = (w & k.m) | k.o;
    const uint32_t b = ((w >> 4) & k.m) | k.o;
    const uint32_t c = ((w >> 8) & k.m) | k.o;
    const uint32_t d = ((w >> 12) & k.m) | k.o;
    return as_bf16x8(a, b, c, d);
  }
  const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0);
  const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1);
  const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2);
  const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3);
  return as_bf16x8(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1), __builtin_bit_cast(uint32_t, p2),
                   __builtin_bit_cast(uint32_t, p3));
}

template <int QMODE>
__device__ __forceinline__ float group_scale(const void* s, int64_t i) {
  if (QMODE == ZMOE_Q_AFFINE) return bf16_bits_to_f32(gload(static_cast<const uint16_t*>(s) + i));
  return e8m0_to_f32(gload(static_cast<const uint8_t*>(s) + i));
}

// ---------------------------------------------------------------------------
// the grouped GEMM
// ---------------------------------------------------------------------------
// Bytes of the LDS parameter cache (0 if it does not fit): per wave its 32
// rows' scales (and biases) of every group, then (affine) the chunk rows'
// group sums of the activations.
__host__ __device__ inline size_t grouped_pcache_bytes(int qmode, bool swiglu, int G) {
  const size_t per_row = (qmode == ZMOE_Q_AFFINE) ? static_cast<size_t>(G) * 2 * 2 : static_cast<size_t>(G);
  const size_t arrays = swiglu ? 2 : 1;
  size_t bytes = static_cast<size_t>(kGWaves) * 32 * per_row * arrays;
  bytes = (bytes + 15) & ~static_cast<size_t>(15);
  if (qmode == ZMOE_Q_AFFINE) bytes += static_cast<size_t>(kGChunk) * G * 4;
  return bytes;
}
constexpr size_t kGPcacheMax = 96 * 1024;

template <int QMODE, int GS, bool SWIGLU, bool PLDS, int NB>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(3, 8))) void k_grouped_qmm(GroupedArgs g) {
  __shared__ __align__(16) uint16_t alds[2][kGChunk * kGLdsRow];
  extern __shared__ __align__(16) unsigned char pcache[];
  constexpr bool G32 = GS == 32;
  constexpr int KPG = GS / 16;  // k-steps per quantisation group
  constexpr int PB = (QMODE == ZMOE_Q_AFFINE) ? 2 : 1;  // parameter bytes
  const int ntiles = (g.N + kGTileN - 1) / kGTileN;
  const int wave = threadIdx.x / kWave;
  const int lane = __lane_id();
  const int h = lane >> 5, col = lane & 31;
  const int c = blockIdx.x / ntiles;
  const int tile = blockIdx.x - c * ntiles;
  if (c >= g.offsets[g.E + 1]) return;  // whole workgroup: past the chunk list
  const int ce = g.blocks[c];
  const int e = ce & 2047;
  const int r_begin = g.offsets[e] + (ce >> 11) * kGChunk;
  const int r_end = min(r_begin + kGChunk, g.offsets[e + 1]);
  const int n0 = tile * kGTileN + wave * 32;
  const bool active = n0 < g.N;  // idle waves still take part in the barriers

  const AffineK ak = affine_k();
  const int K = g.K;
  const int nblk = K >> 6;  // 64-k blocks
  const int G = K / GS;
  const int64_t wpr = K >> 3;
  const int nb = min(n0, g.N - 32);  // this wave's first row (clamped for idle waves)
  const int n = nb + col;            // this lane's output row (B-operand column)
  const int64_t erow = static_cast<int64_t>(e) * g.N + n;
  const uint32_t* W0 = g.w0 + erow * wpr;
  const uint32_t* W1 = SWIGLU ? g.w1 + erow * wpr : nullptr;
  const int64_t prow = erow * G;  // scale/bias row

  // activation row of sorted row r (clamped to the chunk)
  auto act_row = [&](int r) -> int64_t {
    const int rr = min(r, r_end - 1);
    const int src = g.sorted ? g.sorted[rr] : rr;
    return g.lhs ? static_cast<int64_t>(g.lhs[src]) : (g.a_div > 0 ? static_cast<int64_t>(src / g.a_div) : rr);
  };
  // cooperative staging: thread t moves kGStage pieces of 16 bytes (8 k),
  // rows t / 8 + i * (threads / 8)
  const int st_row = threadIdx.x >> 3, st_q = threadIdx.x & 7;
  const uint16_t* st_src[kGStage];
#pragma unroll
  for (int i = 0; i < kGStage; ++i)
    st_src[i] = g.a + act_row(r_begin + st_row + i * (kGThreads / 8)) * g.lda + st_q * 8;

  // ---- parameter cache (PLDS): this wave's rows' scales/biases, chunk sums
  const size_t row_bytes = static_cast<size_t>(G) * PB;
  const size_t wave_bytes = 32 * row_bytes * (QMODE == ZMOE_Q_AFFINE ? 2 : 1);
  unsigned char* pw = pcache + wave * wave_bytes * (SWIGLU ? 2 : 1);  // [matrix][s, b][G][32 rows]
  float* pxs = reinterpret_cast<float*>(
      pcache + ((static_cast<size_t>(kGWaves) * wave_bytes * (SWIGLU ? 2 : 1) + 15) & ~static_cast<size_t>(15)));
  if (PLDS) {
    // each array of the wave's 32 rows is one contiguous block of 32 * G params
    const int64_t base_el = (static_cast<int64_t>(e) * g.N + nb) * G;
    const int nvec = static_cast<int>((32 * row_bytes) >> 4);  // 16-byte pieces per array
    const void* srcs[4] = {g.s0, (QMODE == ZMOE_Q_AFFINE) ? g.b0 : nullptr, g.s1, (QMODE == ZMOE_Q_AFFINE) ? g.b1 : nullptr};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bool use = (m < 2 || SWIGLU) && (QMODE == ZMOE_Q_AFFINE || (m & 1) == 0);
      if (!use) continue;
      const int slot = (QMODE == ZMOE_Q_AFFINE) ? m : (m >> 1);
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const unsigned char*>(srcs[m]) + base_el * PB);
      // stored group-major ([group][row]) so a wave's 32 lanes read 32
      // consecutive entries of one group
      unsigned char* dst = pw + slot * 32 * row_bytes;
      constexpr int per = 16 / PB;  // parameters per 16-byte piece
      for (int i = lane; i < nvec; i += kWave) {
        const uint4 v = gload(src + i);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int t = 0; t < per; ++t) {
          const int el = i * per + t, row = el / G, gi = el - row * G;
          const uint32_t word = wv[(t * PB) >> 2];
          if (PB == 2)
            reinterpret_cast<uint16_t*>(dst)[gi * 32 + row] = static_cast<uint16_t>(word >> ((t & 1) * 16));
          else
            dst[gi * 32 + row] = static_cast<uint8_t>(word >> ((t & 3) * 8));
        }
      }
    }
    if (QMODE == ZMOE_Q_AFFINE) {
      // chunk rows' group sums (G floats per row)
      for (int i = threadIdx.x; i < kGChunk * G; i += kGThreads) {
        const int r = i / G, q = i - r * G;
        pxs[q * kGChunk + r] = gload(g.asum + act_row(r_begin + r) * G + q);
      }
    }
  }
  auto pscale = [&](int m, int gi) -> float {  // scale of this lane's row, matrix m, group gi
    if (QMODE == ZMOE_Q_AFFINE) {
      const uint16_t* a = reinterpret_cast<const uint16_t*>(pw + (m * 2) * 32 * row_bytes);
      return bf16_bits_to_f32(a[gi * 32 + col]);
    }
    return e8m0_to_f32(pw[m * 32 * row_bytes + gi * 32 + col]);
  };
  auto poffset = [&](int m, int gi) -> float {  // affine: b - 128 s
    const uint16_t* sa = reinterpret_cast<const uint16_t*>(pw + (m * 2) * 32 * row_bytes);
    const uint16_t* ba = reinterpret_cast<const uint16_t*>(pw + (m * 2 + 1) * 32 * row_bytes);
    return bf16_bits_to_f32(ba[gi * 32 + col]) - 128.0f * bf16_bits_to_f32(sa[gi * 32 + col]);
  };
  // this lane's rows in the two MFMA blocks (affine offset operand, no cache)
  const float* as_row[kGBlocksM];
#pragma unroll
  for (int mb = 0; mb < kGBlocksM; ++mb)
    as_row[mb] = (QMODE == ZMOE_Q_AFFINE && !PLDS) ? g.asum + act_row(r_begin + mb * kGTileM + col) * G : nullptr;

  f32x16_t tot0[kGBlocksM], tot1[kGBlocksM], acc0[kGBlocksM], acc1[kGBlocksM];
#pragma unroll
  for (int mb = 0; mb < kGBlocksM; ++mb) tot0[mb] = tot1[mb] = acc0[mb] = acc1[mb] = f32x16_t{};
  const int nsteps = G >> 1;
  constexpr int kGpb2 = 128 / GS;  // groups completed per 2 blocks
  // Per 64-k block, one block ahead of use: this lane's weights, this
  // thread's 16 staged activation bytes, and without the cache the scales of
  // the groups the block completes and one affine-offset step's operands.
  struct KBuf {
    uint32_t w0[4], w1[4];
    uint32_t s0[2], s1[2];
    float xs[kGBlocksM];
    uint32_t os0, ob0, os1, ob1;
    uint4 st[kGStage];
  };
  auto raw_scale = [&](const void* sp, int64_t i) -> uint32_t {
    if (QMODE == ZMOE_Q_AFFINE) return gload(static_cast<const uint16_t*>(sp) + i);
    return gload(static_cast<const uint8_t*>(sp) + i);
  };
  auto load_blk = [&](int blk, KBuf& kb) {
#pragma unroll
    for (int i = 0; i < kGStage; ++i) kb.st[i] = gload(reinterpret_cast<const uint4*>(st_src[i] + blk * 64));
    if (!G32) {
      const uint4 q0 = gload(reinterpret_cast<const uint4*>(W0 + blk * 8 + h * 4));
      kb.w0[0] = q0.x, kb.w0[1] = q0.y, kb.w0[2] = q0.z, kb.w0[3] = q0.w;
      if (SWIGLU) {
        const uint4 q1 = gload(reinterpret_cast<const uint4*>(W1 + blk * 8 + h * 4));
        kb.w1[0] = q1.x, kb.w1[1] = q1.y, kb.w1[2] = q1.z, kb.w1[3] = q1.w;
      }
    } else {
      const uint4 qa = gload(reinterpret_cast<const uint4*>(W0 + blk * 8));
      const uint4 qb = gload(reinterpret_cast<const uint4*>(W0 + blk * 8 + 4));
      kb.w0[0] = h ? qa.y : qa.x, kb.w0[1] = h ? qa.w : qa.z, kb.w0[2] = h ? qb.y : qb.x, kb.w0[3] = h ? qb.w : qb.z;
      if (SWIGLU) {
        const uint4 ua = gload(reinterpret_cast<const uint4*>(W1 + blk * 8));
        const uint4 ub = gload(reinterpret_cast<const uint4*>(W1 + blk * 8 + 4));
        kb.w1[0] = h ? ua.y : ua.x, kb.w1[1] = h ? ua.w : ua.z, kb.w1[2] = h ? ub.y : ub.x, kb.w1[3] = h ? ub.w : ub.z;
      }
    }
    if (PLDS) return;
    const int first = (blk * kGpb2) >> 1;
    const int cnt = (((blk + 1) * kGpb2) >> 1) - first;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gi = min(first + i, G - 1);
      kb.s0[i] = i < cnt ? raw_scale(g.s0, prow + gi) : 0u;
      if (SWIGLU) kb.s1[i] = i < cnt ? raw_scale(g.s1, prow + gi) : 0u;
    }
    if (QMODE == ZMOE_Q_AFFINE) {
      const int gi = min(2 * blk + h, G - 1);
      const bool ok = blk < nsteps && 2 * blk + h < G;
#pragma unroll
      for (int mb = 0; mb < kGBlocksM; ++mb) kb.xs[mb] = ok ? as_row[mb][gi] : 0.0f;
      kb.os0 = ok ? gload(static_cast<const uint16_t*>(g.s0) + prow + gi) : 0u;
      kb.ob0 = ok ? gload(static_cast<const uint16_t*>(g.b0) + prow + gi) : 0u;
      if (SWIGLU) {
        kb.os1 = ok ? gload(static_cast<const uint16_t*>(g.s1) + prow + gi) : 0u;
        kb.ob1 = ok ? gload(static_cast<const uint16_t*>(g.b1) + prow + gi) : 0u;
      }
    }
  };
  // staged activations are stored already in the operand order: affine pairs
  // (x0,x4) (x1,x5) (x2,x6) (x3,x7)
  auto stage = [&](const KBuf& kb, int buf) {
#pragma unroll
    for (int i = 0; i < kGStage; ++i) {
      uint4 v = kb.st[i];
      if (QMODE == ZMOE_Q_AFFINE) v = __builtin_bit_cast(uint4, act_affine(v));
      *reinterpret_cast<uint4*>(&alds[buf][(st_row + i * (kGThreads / 8)) * kGLdsRow + st_q * 8]) = v;
    }
  };
  auto decode_scale = [&](uint32_t r) -> float {
    if (QMODE == ZMOE_Q_AFFINE) return bf16_bits_to_f32(r);
    return e8m0_to_f32(r);
  };
  // NMB: the chunk's 32-row MFMA blocks that hold rows (a chunk of <= 32
  // rows skips the second block's MFMAs and scaling)
  auto compute_blk = [&](auto nmbc, int blk, const KBuf& kb, int buf) {
    constexpr int NMB = decltype(nmbc)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8_t b0 = wt_operand<QMODE>(kb.w0[j], ak);
      const bf16x8_t b1 = SWIGLU ? wt_operand<QMODE>(kb.w1[j], ak) : b0;
      const int koff = G32 ? (2 * j + h) * 8 : h * 32 + j * 8;
      // first k-step of a group starts from a zero accumulator
      const bool fresh = ((blk * 4 + j) % KPG) == 0;
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const uint4 av = *reinterpret_cast<const uint4*>(&alds[buf][(mb * kGTileM + col) * kGLdsRow + koff]);
        const bf16x8_t xa = act_natural(av);
        acc0[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, b0, fresh ? f32x16_t{} : acc0[mb], 0, 0, 0);
        if (SWIGLU)
          acc1[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, b1, fresh ? f32x16_t{} : acc1[mb], 0, 0, 0);
      }
      if (((blk * 4 + j + 1) % KPG) == 0) {  // group complete: scale into the totals
        const int gi = (blk * 4 + j) / KPG;
        float s0, s1 = 0.0f;
        if (PLDS) {
          s0 = pscale(0, gi);
          if (SWIGLU) s1 = pscale(1, gi);
        } else {
          const int done = gi - ((blk * kGpb2) >> 1);
          s0 = decode_scale(done == 0 ? kb.s0[0] : kb.s0[1]);
          if (SWIGLU) s1 = decode_scale(done == 0 ? kb.s1[0] : kb.s1[1]);
        }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            tot0[mb][i] = fmaf(s0, acc0[mb][i], tot0[mb][i]);
            if (SWIGLU) tot1[mb][i] = fmaf(s1, acc1[mb][i], tot1[mb][i]);
          }
        }
      }
    }
    if (QMODE == ZMOE_Q_AFFINE && blk < nsteps) {
      // + (b_g - 128 s_g) * asum_g for groups 2 blk, 2 blk + 1
      const int gi = min(2 * blk + h, G - 1);
      const bool ok = 2 * blk + h < G;
      float c0, c1 = 0.0f, xs[kGBlocksM];
      if (PLDS) {
        c0 = ok ? poffset(0, gi) : 0.0f;
        if (SWIGLU) c1 = ok ? poffset(1, gi) : 0.0f;
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) xs[mb] = ok ? pxs[gi * kGChunk + mb * kGTileM + col] : 0.0f;
      } else {
        c0 = bf16_bits_to_f32(kb.ob0) - 128.0f * bf16_bits_to_f32(kb.os0);
        if (SWIGLU) c1 = bf16_bits_to_f32(kb.ob1) - 128.0f * bf16_bits_to_f32(kb.os1);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) xs[mb] = kb.xs[mb];
      }
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        tot0[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[mb], c0, tot0[mb], 0, 0, 0);
        if (SWIGLU) tot1[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[mb], c1, tot1[mb], 0, 0, 0);
      }
    }
  };

  // NB blocks of loads in flight: block s computes from LDS buffer s % 2
  // while block s + 1 is staged into the other and blocks up to s + NB - 1
  // load into registers.  The main loop issues its loads unconditionally
  // (the block index clamped at the end) so the compiler's wait counts stay
  // exact across iterations: a load behind a branch makes it fall back to
  // waiting for every load in flight, which serialises the ring.
  auto kloop = [&](auto nmbc) {
    KBuf kb[NB];
  #pragma unroll
    for (int i = 0; i < NB - 1; ++i) load_blk(min(i, nblk - 1), kb[i]);
    stage(kb[0], 0);
    __syncthreads();
    int blk = 0;
    for (; blk + NB < nblk; blk += NB) {
  #pragma unroll
      for (int q = 0; q < NB; ++q) {
        const int s = blk + q;
        load_blk(min(s + NB - 1, nblk - 1), kb[(q + NB - 1) % NB]);
        if (active) compute_blk(nmbc, s, kb[q], s & 1);
        stage(kb[(q + 1) % NB], (s + 1) & 1);
        __syncthreads();
      }
    }
  #pragma unroll
    for (int q = 0; q < NB; ++q) {  // the last 1..NB blocks
      const int s = blk + q;
      if (s < nblk) {
        if (s + NB - 1 < nblk) load_blk(s + NB - 1, kb[(q + NB - 1) % NB]);
        if (active) compute_blk(nmbc, s, kb[q], s & 1);
        if (s + 1 < nblk) {
          stage(kb[(q + 1) % NB], (s + 1) & 1);
          __syncthreads();
        }
      }
    }
  };
  if (r_end - r_begin > kGTileM)
    kloop(std::integral_constant<int, 2>{});
  else
    kloop(std::integral_constant<int, 1>{});
  // epilogue: element i of block mb is row mb*32 + (i/4)*8 + h*4 + i%4 of
  // the chunk, column n
  static_assert(kGBlocksM == 1, "one MFMA block per chunk");
  if (QMODE == ZMOE_Q_AFFINE && SWIGLU && g.asum_out != nullptr) {
    // group sums of the chunk's bf16 outputs for the down projection's
    // offset term: the 32 x 128 tile goes through LDS and one thread per
    // (row, group) adds it in k_row_group_sums' order (8-element pieces in
    // k order), so the sums are bit-identical to that kernel's
    uint16_t* tl = alds[0];  // [32 rows][kGTileN] (the staging buffers are free after the k loop)
    static_assert(kGTileM * kGTileN <= 2 * kGChunk * kGLdsRow, "tile fits the staging buffers");
    __syncthreads();
    if (active) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rl = (i >> 2) * 8 + h * 4 + (i & 3);
        tl[rl * kGTileN + wave * 32 + col] =
            static_cast<uint16_t>(swiglu_bf16(round_bf16(tot0[0][i]), round_bf16(tot1[0][i])));
      }
    }
    __syncthreads();
    const int gpt = kGTileN / GS;  // groups per tile
    const int Gn = g.N / GS;
    for (int it = threadIdx.x; it < kGTileM * gpt; it += kGThreads) {
      const int rl = it / gpt, gg = it - rl * gpt;
      const int r = r_begin + rl;
      const int n_first = tile * kGTileN + gg * GS;
      if (r < r_end && n_first < g.N) {
        const uint16_t* p = tl + rl * kGTileN + gg * GS;
        float sv = 0.0f;
        for (int j = 0; j < GS; j += 8) {
          const uint4 v = *reinterpret_cast<const uint4*>(p + j);
          sv += (bf16_bits_to_f32(v.x & 0xFFFFu) + bf16_bits_to_f32(v.x >> 16)) +
                (bf16_bits_to_f32(v.y & 0xFFFFu) + bf16_bits_to_f32(v.y >> 16)) +
                (bf16_bits_to_f32(v.z & 0xFFFFu) + bf16_bits_to_f32(v.z >> 16)) +
                (bf16_bits_to_f32(v.w & 0xFFFFu) + bf16_bits_to_f32(v.w >> 16));
        }
        const int64_t orow = g.scatter ? static_cast<int64_t>(g.sorted[r]) : static_cast<int64_t>(r);
        g.asum_out[orow * Gn + n_first / GS] = sv;
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int mb = 0; mb < kGBlocksM; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = r_begin + mb * kGTileM + (i >> 2) * 8 + h * 4 + (i & 3);
      if (r < r_end) {
        const int64_t orow = g.scatter ? static_cast<int64_t>(g.sorted[r]) : static_cast<int64_t>(r);
        const uint32_t v =
            SWIGLU ? swiglu_bf16(round_bf16(tot0[mb][i]), round_bf16(tot1[mb][i])) : f32_to_bf16_bits(tot0[mb][i]);
        g.out[orow * g.ldo + n] = static_cast<uint16_t>(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <int QMODE, int GS, bool SWIGLU, bool PLDS, int NB>
static void launch_grouped_nb(hipStream_t st, const GroupedArgs& g, unsigned blocks, size_t lds) {
  if (PLDS) {
    static bool prepared = false;
    if (!prepared) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_grouped_qmm<QMODE, GS, SWIGLU, PLDS, NB>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kGPcacheMax));
      prepared = true;
    }
  }
  hipLaunchKernelGGL((k_grouped_qmm<QMODE, GS, SWIGLU, PLDS, NB>), dim3(blocks), dim3(kGThreads), lds, st, g);
}

template <int QMODE, int GS, bool SWIGLU>
static void launch_grouped_t(hipStream_t st, const GroupedArgs& g, int n_experts) {
  const int ntiles = (g.N + kGTileN - 1) / kGTileN;
  const unsigned blocks = static_cast<unsigned>(grouped_max_blocks(g.M, n_experts) * ntiles);
  const size_t pc = grouped_pcache_bytes(QMODE, SWIGLU, g.K / GS);
  if (pc <= kGPcacheMax) {
    // with the parameter cache the workgroup holds a CU's LDS alone; its
    // register budget then allows a deeper load ring for gate/up
    static int nb = -1;
    if (nb < 0) {
      const char* e = getenv("ZMOE_GNB");
      nb = e ? atoi(e) : 4;
    }
    if constexpr (QMODE == ZMOE_Q_AFFINE && SWIGLU) {  // (mxfp4 would spill)
      if (nb == 4) return launch_grouped_nb<QMODE, GS, SWIGLU, true, 4>(st, g, blocks, pc);
      if (nb == 5) return launch_grouped_nb<QMODE, GS, SWIGLU, true, 5>(st, g, blocks, pc);
    }
    launch_grouped_nb<QMODE, GS, SWIGLU, true, 3>(st, g, blocks, pc);
  } else {
    launch_grouped_nb<QMODE, GS, SWIGLU, false, 3>(st, g, blocks, 0);
  }
}

bool grouped_params_cached(int quant_mode, bool swiglu, int K, int gs) {
  return grouped_pcache_bytes(quant_mode, swiglu, K / (quant_mode == ZMOE_Q_AFFINE ? gs : 32)) <= kGPcacheMax;
}

int launch_grouped(hipStream_t st, const GroupedArgs& g, int n_experts, int quant_mode, bool swiglu) {
  if (quant_mode == ZMOE_Q_AFFINE) {
    switch (g.gs) {
      case 32:
        swiglu ? launch_grouped_t<ZMOE_Q_AFFINE, 32, true>(st, g, n_experts)
               : launch_grouped_t<ZMOE_Q_AFFINE, 32, false>(st, g, n_experts);
        break;
      case 128:
        swiglu ? launch_grouped_t<ZMOE_Q_AFFINE, 128, true>(st, g, n_experts)
               : launch_grouped_t<ZMOE_Q_AFFINE, 128, false>(st, g, n_experts);
        break;
      default:
        swiglu ? launch_grouped_t<ZMOE_Q_AFFINE, 64, true>(st, g, n_experts)
               : launch_grouped_t<ZMOE_Q_AFFINE, 64, false>(st, g, n_experts);
    }
  } else {
    swiglu ? launch_grouped_t<ZMOE_Q_MXFP4, 32, true>(st, g, n_experts)
           : launch_grouped_t<ZMOE_Q_MXFP4, 32, false>(st, g, n_experts);
  }
  return check_launch("grouped gather_qmm");
}

int launch_sort_pairs(hipStream_t st, const uint32_t* idx, int npairs, int E, int* offsets, int* sorted, int* blocks,
                      int chunk) {
  hipLaunchKernelGGL(k_sort_pairs, dim3(1), dim3(1024), 0, st, idx, npairs, E, chunk, offsets, sorted, blocks);
  return check_launch("sort pairs by expert");
}

int launch_row_group_sums(hipStream_t st, const uint16_t* a, int64_t lda, int rows, int K, int gs, float* out) {
  const int64_t n = static_cast<int64_t>(rows) * (K / gs);
  if (n == 0) return ZMOE_OK;
  hipLaunchKernelGGL(k_row_group_sums, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, a, lda, rows, K,
                     gs, out);
  return check_launch("row group sums");
}

// Workspace of zmoe_grouped_gather_qmm: offsets | sorted | asum | (swiglu: none)
static size_t al(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

size_t grouped_ws_bytes(int64_t n_pairs, int E, int x_rows, int K, int gs) {
  return al(static_cast<size_t>(E + 2) * 4) + al(static_cast<size_t>(n_pairs) * 4) +
         al(static_cast<size_t>(grouped_max_blocks(static_cast<int>(n_pairs), E)) * 4) +
         al(static_cast<size_t>(x_rows) * (K / gs) * 4);
}

}  // namespace zmoe

using namespace zmoe;

extern "C" size_t zmoe_grouped_gather_qmm_workspace_size(int64_t n_pairs, int x_batch, int E, int K, int group_size) {
  if (n_pairs < 0 || x_batch < 1 || E < 1 || K < 1 || group_size < 32) return 0;
  return grouped_ws_bytes(n_pairs, E, x_batch, K, group_size);
}

extern "C" int zmoe_grouped_gather_qmm(void* stream, const void* x, int64_t x_batch, const uint32_t* w,
                                       const void* scales, const void* biases, const uint32_t* up_w,
                                       const void* up_scales, const void* up_biases, const uint32_t* lhs_indices,
                                       const uint32_t* rhs_indices, int64_t n_pairs, int N, int K, int E,
                                       int group_size, int bits, int quant_mode, void* workspace,
                                       size_t workspace_bytes, void* out) {
  const std::string tag = "[gather_qmm] ";
  ZMOE_REQUIRE(quant_mode == ZMOE_Q_AFFINE || quant_mode == ZMOE_Q_MXFP4, ZMOE_EUNSUPPORTED,
               tag + "Unsupported quantization mode.");
  ZMOE_REQUIRE(bits == 4, ZMOE_EUNSUPPORTED, tag + "Only bits == 4 is supported.");
  if (quant_mode == ZMOE_Q_AFFINE) {
    ZMOE_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128, ZMOE_EUNSUPPORTED,
                 tag + "group_size must be 32, 64 or 128.");
    ZMOE_REQUIRE(biases != nullptr && (up_w == nullptr || up_biases != nullptr), ZMOE_EINVAL_SHAPE,
                 tag + "affine mode requires biases.");
  } else {
    ZMOE_REQUIRE(group_size == 32, ZMOE_EUNSUPPORTED, tag + "mxfp4 requires group_size == 32.");
  }
  ZMOE_REQUIRE(N >= 32 && N % 32 == 0 && K % 128 == 0 && E >= 1 && E <= 1024 && x_batch >= 1 && n_pairs >= 0 &&
                   n_pairs <= (1 << 24),
               ZMOE_EINVAL_SHAPE, tag + "grouped path needs N % 32 == 0, K % 128 == 0, E <= 1024.");
  ZMOE_REQUIRE(x_batch <= (1 << 24), ZMOE_EINVAL_SHAPE, tag + "x_batch too large.");
  ZMOE_REQUIRE(n_pairs == 0 || (x && w && scales && lhs_indices && rhs_indices && out && workspace), ZMOE_EINVAL_SHAPE,
               tag + "null pointer.");
  ZMOE_REQUIRE(workspace_bytes >= grouped_ws_bytes(n_pairs, E, static_cast<int>(x_batch), K, group_size),
               ZMOE_EINVAL_SHAPE, tag + "workspace too small.");
  if (n_pairs == 0) return ZMOE_OK;
  hipStream_t st = as_stream(stream);
  char* base = static_cast<char*>(workspace);
  int* offsets = reinterpret_cast<int*>(base);
  int* sorted = reinterpret_cast<int*>(base + al(static_cast<size_t>(E + 2) * 4));
  int* blocks = reinterpret_cast<int*>(base + al(static_cast<size_t>(E + 2) * 4) + al(static_cast<size_t>(n_pairs) * 4));
  float* asum = reinterpret_cast<float*>(
      reinterpret_cast<char*>(blocks) + al(static_cast<size_t>(grouped_max_blocks(static_cast<int>(n_pairs), E)) * 4));
  int rc = launch_sort_pairs(st, rhs_indices, static_cast<int>(n_pairs), E, offsets, sorted, blocks);
  if (rc) return rc;
  if (quant_mode == ZMOE_Q_AFFINE) {
    rc = launch_row_group_sums(st, static_cast<const uint16_t*>(x), K, static_cast<int>(x_batch), K, group_size, asum);
    if (rc) return rc;
  }
  GroupedArgs g{};
  g.a = static_cast<const uint16_t*>(x);
  g.lda = K;
  g.asum = asum;
  g.offsets = offsets;
  g.blocks = blocks;
  g.E = E;
  g.sorted = sorted;
  g.lhs = lhs_indices;
  g.a_div = 0;
  g.scatter = 1;
  g.M = static_cast<int>(n_pairs);
  g.w0 = w;
  g.s0 = scales;
  g.b0 = biases;
  g.w1 = up_w;
  g.s1 = up_scales;
  g.b1 = up_biases;
  g.N = N;
  g.K = K;
  g.gs = group_size;
  g.out = static_cast<uint16_t*>(out);
  g.ldo = N;
  return launch_grouped(st, g, E, quant_mode, up_w != nullptr);
}
