// Grouped (per-expert) quantized GEMM on MFMA: the batched / prefill path.
//
// For many tokens the (token, expert) pairs are counting-sorted by expert
// and every expert's weights are streamed once for all of its rows (the role
// of mlx_lm's SwitchGLU sort path + gather_qmm(sorted_indices=True) that the
// reference keeps for M > 1, moe_mlp.py:540-543).
//
// Tiles: a workgroup of 4 waves owns (expert e, 128 output rows n); wave w
// computes n0 = 128*tile + 32*w .. +31 for every 32-row block of the
// expert's sorted rows, with v_mfma_f32_32x32x16_bf16.
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

namespace zmoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGThreads = 256;  // 4 waves
constexpr int kGTileN = 128;    // output rows per workgroup
constexpr int kGTileM = 32;     // sorted rows per MFMA block


// ---------------------------------------------------------------------------
// sort (token, k) pairs by expert: one workgroup, counts in LDS
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_sort_pairs(const uint32_t* __restrict__ idx, int npairs, int E,
                                                     int* __restrict__ offsets, int* __restrict__ sorted,
                                                     int* __restrict__ blocks) {
  __shared__ int cnt[1024];
  __shared__ int off[1025];
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int q = threadIdx.x; q < npairs; q += blockDim.x) atomicAdd(&cnt[min(static_cast<int>(idx[q]), E - 1)], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = run;
      run += cnt[e];
    }
    off[E] = run;
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) offsets[e] = off[e];
  if (blocks) {
    // 32-row blocks of every expert, in expert order (their starts reuse cnt)
    if (threadIdx.x == 0) {
      int nb = 0;
      for (int e = 0; e < E; ++e) {
        cnt[e] = nb;
        nb += (off[e + 1] - off[e] + 31) / 32;
      }
      offsets[E + 1] = nb;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      const int nbe = (off[e + 1] - off[e] + 31) / 32;
      for (int j = 0; j < nbe; ++j) blocks[cnt[e] + j] = e | (j << 11);
    }
    __syncthreads();
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
template <int QMODE, bool G32, bool SWIGLU>
__global__ __launch_bounds__(kGThreads) void k_grouped_qmm(GroupedArgs g) {
  const int ntiles = (g.N + kGTileN - 1) / kGTileN;
  const int wave = threadIdx.x / kWave;
  const int lane = __lane_id();
  const int h = lane >> 5, col = lane & 31;
  // workgroup -> (expert, 32-row blocks, 128-row output tile): one block per
  // workgroup from the block list (heavy experts spread over many
  // workgroups), else every block of expert blockIdx / ntiles
  int e, tile, m_first, m_last;
  if (g.blocks) {
    const int b = blockIdx.x / ntiles;
    tile = blockIdx.x - b * ntiles;
    if (b >= g.offsets[g.E + 1]) return;
    const int be = g.blocks[b];
    e = be & 2047;
    m_first = g.offsets[e] + (be >> 11) * kGTileM;
    m_last = min(m_first + kGTileM, g.offsets[e + 1]);
  } else {
    e = blockIdx.x / ntiles;
    tile = blockIdx.x - e * ntiles;
    m_first = g.offsets ? g.offsets[e] : 0;
    m_last = g.offsets ? g.offsets[e + 1] : g.M;
  }
  const int n0 = tile * kGTileN + wave * 32;
  if (n0 >= g.N) return;
  const int r_begin = m_first, r_end = g.offsets ? (g.blocks ? m_last : g.offsets[e + 1]) : g.M;
  if (r_begin >= r_end) return;

  const AffineK ak = affine_k();
  const int K = g.K;
  const int nblk = K >> 6;  // 64-k blocks
  const int G = K / g.gs;
  const int kpg = g.gs >> 4;  // k-steps per quantisation group
  const int64_t wpr = K >> 3;
  const int n = n0 + col;  // this lane's output row (B-operand column)
  const int64_t erow = static_cast<int64_t>(e) * g.N + n;
  const uint32_t* W0 = g.w0 + erow * wpr;
  const uint32_t* W1 = SWIGLU ? g.w1 + erow * wpr : nullptr;
  const int64_t prow = erow * G;  // scale/bias row

  for (int m0 = r_begin; m0 < r_end; m0 += kGTileM) {
    // this lane's A row (operand row = col) and its source row
    const int r_lane = min(m0 + col, r_end - 1);
    const int src = g.sorted ? g.sorted[r_lane] : r_lane;
    const int64_t arow = g.lhs ? static_cast<int64_t>(g.lhs[src])
                                : (g.a_div > 0 ? static_cast<int64_t>(src / g.a_div) : static_cast<int64_t>(r_lane));
    const uint16_t* A = g.a + arow * g.lda;

    f32x16_t tot0 = {}, tot1 = {};
    f32x16_t acc0 = {}, acc1 = {};
    int ks = 0;  // k-steps into the current group
    int grp = 0;
    const float* as_row = (QMODE == ZMOE_Q_AFFINE) ? g.asum + arow * G : nullptr;
    // Per 64-k block: weights, activations, the scales of the groups this
    // block completes (gs 32: two, 64: one, 128: one every other block) and
    // the operands of one affine-offset step (two groups per f32 MFMA,
    // G / 2 <= blocks), all loaded one block ahead of their use.
    struct KBuf {
      uint32_t w0[4], w1[4];
      uint4 av[4];
      uint32_t s0[2], s1[2];  // raw scales
      float xs;               // offset step: group sum of a
      uint32_t os0, ob0, os1, ob1;  // offset step: raw scale / bias
    };
    const int gpb2 = 128 / g.gs;  // groups completed per 2 blocks
    const int nsteps = G >> 1;
    auto raw_scale = [&](const void* sp, int64_t i) -> uint32_t {
      if (QMODE == ZMOE_Q_AFFINE) return gload(static_cast<const uint16_t*>(sp) + i);
      return gload(static_cast<const uint8_t*>(sp) + i);
    };
    auto load_blk = [&](int blk, KBuf& kb) {
      if (!G32) {
        const uint4 q0 = gload(reinterpret_cast<const uint4*>(W0 + blk * 8 + h * 4));
        kb.w0[0] = q0.x, kb.w0[1] = q0.y, kb.w0[2] = q0.z, kb.w0[3] = q0.w;
        if (SWIGLU) {
          const uint4 q1 = gload(reinterpret_cast<const uint4*>(W1 + blk * 8 + h * 4));
          kb.w1[0] = q1.x, kb.w1[1] = q1.y, kb.w1[2] = q1.z, kb.w1[3] = q1.w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) kb.av[j] = gload(reinterpret_cast<const uint4*>(A + blk * 64 + h * 32 + j * 8));
      } else {
        const uint4 qa = gload(reinterpret_cast<const uint4*>(W0 + blk * 8));
        const uint4 qb = gload(reinterpret_cast<const uint4*>(W0 + blk * 8 + 4));
        kb.w0[0] = h ? qa.y : qa.x, kb.w0[1] = h ? qa.w : qa.z, kb.w0[2] = h ? qb.y : qb.x, kb.w0[3] = h ? qb.w : qb.z;
        if (SWIGLU) {
          const uint4 ua = gload(reinterpret_cast<const uint4*>(W1 + blk * 8));
          const uint4 ub = gload(reinterpret_cast<const uint4*>(W1 + blk * 8 + 4));
          kb.w1[0] = h ? ua.y : ua.x, kb.w1[1] = h ? ua.w : ua.z, kb.w1[2] = h ? ub.y : ub.x,
          kb.w1[3] = h ? ub.w : ub.z;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) kb.av[j] = gload(reinterpret_cast<const uint4*>(A + blk * 64 + (2 * j + h) * 8));
      }
      // groups completed in this block: [first, first + cnt)
      const int first = (blk * gpb2) >> 1;
      const int cnt = (((blk + 1) * gpb2) >> 1) - first;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int gi = min(first + i, G - 1);
        kb.s0[i] = i < cnt ? raw_scale(g.s0, prow + gi) : 0u;
        if (SWIGLU) kb.s1[i] = i < cnt ? raw_scale(g.s1, prow + gi) : 0u;
      }
      if (QMODE == ZMOE_Q_AFFINE) {
        const int gi = min(2 * blk + h, G - 1);
        const bool ok = blk < nsteps && 2 * blk + h < G;
        kb.xs = ok ? as_row[gi] : 0.0f;
        kb.os0 = ok ? gload(static_cast<const uint16_t*>(g.s0) + prow + gi) : 0u;
        kb.ob0 = ok ? gload(static_cast<const uint16_t*>(g.b0) + prow + gi) : 0u;
        if (SWIGLU) {
          kb.os1 = ok ? gload(static_cast<const uint16_t*>(g.s1) + prow + gi) : 0u;
          kb.ob1 = ok ? gload(static_cast<const uint16_t*>(g.b1) + prow + gi) : 0u;
        }
      }
    };
    auto decode_scale = [&](uint32_t r) -> float {
      if (QMODE == ZMOE_Q_AFFINE) return bf16_bits_to_f32(r);
      return e8m0_to_f32(r);
    };
    auto compute_blk = [&](int blk, const KBuf& kb) {
      int done = 0;  // groups completed so far in this block
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8_t xa = (QMODE == ZMOE_Q_AFFINE) ? act_affine(kb.av[j]) : act_natural(kb.av[j]);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, wt_operand<QMODE>(kb.w0[j], ak), acc0, 0, 0, 0);
        if (SWIGLU) acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, wt_operand<QMODE>(kb.w1[j], ak), acc1, 0, 0, 0);
        if (++ks == kpg) {  // group complete: scale into the totals
          ks = 0;
          const float s0 = decode_scale(done == 0 ? kb.s0[0] : kb.s0[1]);
          const float s1 = SWIGLU ? decode_scale(done == 0 ? kb.s1[0] : kb.s1[1]) : 0.0f;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            tot0[i] = fmaf(s0, acc0[i], tot0[i]);
            acc0[i] = 0.0f;
            if (SWIGLU) {
              tot1[i] = fmaf(s1, acc1[i], tot1[i]);
              acc1[i] = 0.0f;
            }
          }
          ++grp;
          ++done;
        }
      }
      if (QMODE == ZMOE_Q_AFFINE && blk < nsteps) {
        // + (b_g - 128 s_g) * asum_g for groups 2 blk, 2 blk + 1
        const float c0 = bf16_bits_to_f32(kb.ob0) - 128.0f * bf16_bits_to_f32(kb.os0);
        tot0 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb.xs, c0, tot0, 0, 0, 0);
        if (SWIGLU) {
          const float c1 = bf16_bits_to_f32(kb.ob1) - 128.0f * bf16_bits_to_f32(kb.os1);
          tot1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb.xs, c1, tot1, 0, 0, 0);
        }
      }
    };
    // next block's loads in flight while the current one runs on MFMA
    KBuf kb0, kb1;
    load_blk(0, kb0);
    for (int blk = 0; blk < nblk; blk += 2) {
      if (blk + 1 < nblk) load_blk(blk + 1, kb1);
      compute_blk(blk, kb0);
      if (blk + 1 < nblk) {
        if (blk + 2 < nblk) load_blk(blk + 2, kb0);
        compute_blk(blk + 1, kb1);
      }
    }
    // epilogue: element i is row (i/4)*8 + h*4 + i%4 of the block, column n
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = m0 + (i >> 2) * 8 + h * 4 + (i & 3);
      if (r < r_end) {
        const int64_t orow = g.scatter ? static_cast<int64_t>(g.sorted[r]) : static_cast<int64_t>(r);
        const uint32_t v = SWIGLU ? swiglu_bf16(round_bf16(tot0[i]), round_bf16(tot1[i])) : f32_to_bf16_bits(tot0[i]);
        g.out[orow * g.ldo + n] = static_cast<uint16_t>(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <int QMODE, bool G32, bool SWIGLU>
static void launch_grouped_t(hipStream_t st, const GroupedArgs& g, int n_experts) {
  const int ntiles = (g.N + kGTileN - 1) / kGTileN;
  const int units = g.blocks ? grouped_max_blocks(g.M, n_experts) : n_experts;
  hipLaunchKernelGGL((k_grouped_qmm<QMODE, G32, SWIGLU>), dim3(units * ntiles), dim3(kGThreads), 0, st, g);
}

int launch_grouped(hipStream_t st, const GroupedArgs& g, int n_experts, int quant_mode, bool swiglu) {
  const bool g32 = g.gs == 32;
  if (quant_mode == ZMOE_Q_AFFINE) {
    if (g32)
      swiglu ? launch_grouped_t<ZMOE_Q_AFFINE, true, true>(st, g, n_experts)
             : launch_grouped_t<ZMOE_Q_AFFINE, true, false>(st, g, n_experts);
    else
      swiglu ? launch_grouped_t<ZMOE_Q_AFFINE, false, true>(st, g, n_experts)
             : launch_grouped_t<ZMOE_Q_AFFINE, false, false>(st, g, n_experts);
  } else {
    swiglu ? launch_grouped_t<ZMOE_Q_MXFP4, true, true>(st, g, n_experts)
           : launch_grouped_t<ZMOE_Q_MXFP4, true, false>(st, g, n_experts);
  }
  return check_launch("grouped gather_qmm");
}

int launch_sort_pairs(hipStream_t st, const uint32_t* idx, int npairs, int E, int* offsets, int* sorted, int* blocks) {
  hipLaunchKernelGGL(k_sort_pairs, dim3(1), dim3(1024), 0, st, idx, npairs, E, offsets, sorted, blocks);
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
