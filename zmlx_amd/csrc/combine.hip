// MoE combine kernels: out[b, d] = sum_k w[b, k] * y[b, k, d], k ascending,
// in the rounding modes of the reference's combine family, plus the
// streaming weighted-accumulate step.  One thread per output element; the
// expert dimension is walked in order so every mode is deterministic.
#include "zmoe_common.h"
#include "zmoe_host.h"
#include "zmoe_combine.h"

namespace zmoe {

__device__ __forceinline__ float load_w(const void* w, int dtype, int64_t i) {
  return dtype == ZMOE_DT_F32 ? static_cast<const float*>(w)[i]
                              : bf16_bits_to_f32(static_cast<const uint16_t*>(w)[i]);
}

// force_bf16: write bf16 even for the fp32 modes (the caller's .astype(bf16));
// shared (nullable): bf16 [B, D] addend applied to the bf16 result
// (``y + shared_experts(x)``, moe_mlp.py:1059-1061).
constexpr int kCombMaxK = 16;  // experts per token of the unrolled kernels

// any K (no unrolling): one expert at a time
__global__ __launch_bounds__(256) void k_moe_combine_any(const uint16_t* __restrict__ y, const void* __restrict__ w,
                                                         int w_dtype, int K, int D, int mode, int force_bf16,
                                                         const uint16_t* __restrict__ shared, void* __restrict__ out) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (d >= D) return;
  const float v = combine_one(
      mode, K, [&](int k) { return bf16_bits_to_f32(y[(b * K + k) * D + d]); },
      [&](int k) { return load_w(w, w_dtype, b * K + k); });
  if (combine_f32_out(mode) && !force_bf16) {
    static_cast<float*>(out)[b * D + d] = v;
  } else {
    float r = round_bf16(v);
    if (shared) r = add_nofma(r, bf16_bits_to_f32(shared[b * D + d]));
    static_cast<uint16_t*>(out)[b * D + d] = static_cast<uint16_t>(f32_to_bf16_bits(r));
  }
}

template <int KT, bool WF32>
__global__ __launch_bounds__(256) void k_moe_combine(const uint16_t* __restrict__ y, const void* __restrict__ w,
                                                     int w_dtype, int K, int D, int mode, int force_bf16,
                                                     const uint16_t* __restrict__ shared, void* __restrict__ out) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (d >= D) return;
  // every expert's value and weight loaded at once (KT = 0: K at run time,
  // indices clamped; the weight dtype is fixed at compile time because a load
  // behind a dtype branch makes the compiler wait for it)
  constexpr int NK = KT > 0 ? KT : kCombMaxK;
  if (KT > 0) K = KT;
  float yv[NK], wv[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int kc = KT > 0 ? k : min(k, K - 1);
    yv[k] = bf16_bits_to_f32(y[(b * K + kc) * D + d]);
    wv[k] = WF32 ? static_cast<const float*>(w)[b * K + kc]
                 : bf16_bits_to_f32(static_cast<const uint16_t*>(w)[b * K + kc]);
  }
  const float v = combine_one(mode, K, [&](int k) { return yv[k]; }, [&](int k) { return wv[k]; });
  if (combine_f32_out(mode) && !force_bf16) {
    static_cast<float*>(out)[b * D + d] = v;
  } else {
    float r = round_bf16(v);
    if (shared) r = add_nofma(r, bf16_bits_to_f32(shared[b * D + d]));
    static_cast<uint16_t*>(out)[b * D + d] = static_cast<uint16_t>(f32_to_bf16_bits(r));
  }
}

// One k-step and the final rounding of combine_one's modes, for a thread that
// owns 8 consecutive outputs: the same operations in the same k order, so the
// results are bit-identical to combine_one.
__device__ __forceinline__ float combine_step(int mode, float acc, float w, float y) {
  switch (mode) {
    case ZMOE_COMBINE_NATIVE:
      return add_nofma(acc, round_bf16(mul_nofma(w, y)));
    case ZMOE_COMBINE_FP32:
    case ZMOE_COMBINE_FLOAT:
      return fmaf(w, y, acc);
    case ZMOE_COMBINE_FP32_NO_FMA:
    case ZMOE_COMBINE_NO_FMA:
      return add_nofma(acc, mul_nofma(w, y));
    default:  // ZMOE_COMBINE_EXACT
      return round_bf16(add_nofma(acc, round_bf16(mul_nofma(round_bf16(w), y))));
  }
}
__device__ __forceinline__ float combine_finish(int mode, float acc) {
  return (mode == ZMOE_COMBINE_NATIVE || mode == ZMOE_COMBINE_FLOAT || mode == ZMOE_COMBINE_NO_FMA) ? round_bf16(acc)
                                                                                                   : acc;
}

// D % 8 == 0 and K <= kCombVecMaxK: thread owns outputs d0 .. d0 + 7 and
// reads 16 bytes per expert.  KT > 0 is the expert count at compile time;
// KT = 0 takes K at run time (loads clamped to K - 1); WF32: f32 weights
// (else bf16).
constexpr int kCombVecMaxK = kCombMaxK;
constexpr int kCombVecThreads = 256;
template <int KT, bool WF32>
__global__ __launch_bounds__(256) void k_moe_combine8(const uint16_t* __restrict__ y, const void* __restrict__ w,
                                                      int w_dtype, int K, int D, int mode, int force_bf16,
                                                      const uint16_t* __restrict__ shared, void* __restrict__ out) {
  const int d0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  const int64_t b = blockIdx.y;
  if (d0 >= D) return;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  // every expert's 16 bytes are loaded at once (indices clamped, loads
  // unconditional) so the kernel is one memory round trip deep
  constexpr int NK = KT > 0 ? KT : kCombVecMaxK;
  if (KT > 0) K = KT;
  uint4 v[NK];
  float wk[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int kc = KT > 0 ? k : min(k, K - 1);
    v[k] = gload(reinterpret_cast<const uint4*>(y + (b * K + kc) * D + d0));
    // dtype fixed at compile time: a load behind a dtype branch would make
    // the compiler wait for it before issuing the next
    wk[k] = WF32 ? static_cast<const float*>(w)[b * K + kc]
                 : bf16_bits_to_f32(static_cast<const uint16_t*>(w)[b * K + kc]);
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (KT > 0 || k < K) {
      const uint32_t wv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = combine_step(mode, acc[j], wk[k], bf16_bits_to_f32((wv[j >> 1] >> ((j & 1) * 16)) & 0xFFFFu));
    }
  }
  if (combine_f32_out(mode) && !force_bf16) {
    float* o = static_cast<float*>(out) + b * D + d0;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = combine_finish(mode, acc[j]);
  } else {
    uint4 sh = make_uint4(0, 0, 0, 0);
    if (shared) sh = gload(reinterpret_cast<const uint4*>(shared + b * D + d0));
    const uint32_t sv[4] = {sh.x, sh.y, sh.z, sh.w};
    uint32_t ov[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t pair = 0;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int j = q * 2 + hh;
        float r = round_bf16(combine_finish(mode, acc[j]));
        if (shared) r = add_nofma(r, bf16_bits_to_f32((sv[q] >> (hh * 16)) & 0xFFFFu));
        pair |= f32_to_bf16_bits(r) << (hh * 16);
      }
      ov[q] = pair;
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + b * D + d0) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
  }
}

int launch_combine(hipStream_t st, const void* y, const void* w, int w_dtype, int B, int K, int D, int mode,
                   int force_bf16, const void* shared, void* out) {
  // the 8-wide kernel pays off for prefill-sized batches; small batches
  // keep one output per thread (more waves in flight)
  const bool vec = B >= 64 && D % 8 == 0 && K <= kCombVecMaxK && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0 && (reinterpret_cast<uintptr_t>(shared) & 15) == 0;
  if (vec) {
    const bool f = w_dtype == ZMOE_DT_F32;
    auto fn = K == 8   ? (f ? k_moe_combine8<8, true> : k_moe_combine8<8, false>)
              : K == 4 ? (f ? k_moe_combine8<4, true> : k_moe_combine8<4, false>)
              : K == 2 ? (f ? k_moe_combine8<2, true> : k_moe_combine8<2, false>)
              : K == 1 ? (f ? k_moe_combine8<1, true> : k_moe_combine8<1, false>)
                       : (f ? k_moe_combine8<0, true> : k_moe_combine8<0, false>);
    const int bt = kCombVecThreads;
    hipLaunchKernelGGL(fn, dim3((D / 8 + bt - 1) / bt, B), dim3(bt), 0, st, static_cast<const uint16_t*>(y), w, w_dtype,
                       K, D, mode, force_bf16, static_cast<const uint16_t*>(shared), out);
  } else if (K <= kCombMaxK) {
    const bool f = w_dtype == ZMOE_DT_F32;
    auto fn = K == 8   ? (f ? k_moe_combine<8, true> : k_moe_combine<8, false>)
              : K == 4 ? (f ? k_moe_combine<4, true> : k_moe_combine<4, false>)
              : K == 2 ? (f ? k_moe_combine<2, true> : k_moe_combine<2, false>)
              : K == 1 ? (f ? k_moe_combine<1, true> : k_moe_combine<1, false>)
                       : (f ? k_moe_combine<0, true> : k_moe_combine<0, false>);
    hipLaunchKernelGGL(fn, dim3((D + 255) / 256, B), dim3(256), 0, st, static_cast<const uint16_t*>(y), w, w_dtype, K,
                       D, mode, force_bf16, static_cast<const uint16_t*>(shared), out);
  } else {
    hipLaunchKernelGGL(k_moe_combine_any, dim3((D + 255) / 256, B), dim3(256), 0, st, static_cast<const uint16_t*>(y),
                       w, w_dtype, K, D, mode, force_bf16, static_cast<const uint16_t*>(shared), out);
  }
  return check_launch("moe_combine");
}

__global__ __launch_bounds__(256) void k_weighted_accumulate(const void* __restrict__ acc,
                                                             const uint16_t* __restrict__ proj,
                                                             const float* __restrict__ gate, int64_t gstride, int D,
                                                             int acc_dtype, int no_fma, void* __restrict__ out) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (d >= D) return;
  const int64_t i = b * D + d;
  const float a = load_w(acc, acc_dtype, i);
  const float g = gate[b * gstride];
  const float v = bf16_bits_to_f32(proj[i]);
  const float r = no_fma ? add_nofma(a, mul_nofma(g, v)) : fmaf(g, v, a);
  if (acc_dtype == ZMOE_DT_F32)
    static_cast<float*>(out)[i] = r;
  else
    static_cast<uint16_t*>(out)[i] = static_cast<uint16_t>(f32_to_bf16_bits(r));
}

}  // namespace zmoe

using namespace zmoe;

extern "C" int zmoe_moe_combine(void* stream, const void* y, const void* w, int w_dtype, int B, int K, int D, int mode,
                                void* out) {
  ZMOE_REQUIRE(B >= 0 && K >= 1 && D >= 1, ZMOE_EINVAL_SHAPE, "[moe_combine] sizes must be positive.");
  ZMOE_REQUIRE(B <= 65535, ZMOE_EINVAL_SHAPE, "[moe_combine] B must be <= 65535.");
  ZMOE_REQUIRE(mode >= ZMOE_COMBINE_NATIVE && mode <= ZMOE_COMBINE_NO_FMA, ZMOE_EINVAL_SHAPE,
               "[moe_combine] unknown combine mode.");
  ZMOE_REQUIRE(w_dtype == ZMOE_DT_BF16 || w_dtype == ZMOE_DT_F32, ZMOE_EINVAL_DTYPE,
               "[moe_combine] weights must be bf16 or f32.");
  ZMOE_REQUIRE(!(mode == ZMOE_COMBINE_NATIVE && w_dtype != ZMOE_DT_BF16), ZMOE_EINVAL_DTYPE,
               "[moe_combine] native mode takes bf16 weights (f32 weights promote: use an fp32 mode).");
  if (B == 0) return ZMOE_OK;
  return launch_combine(as_stream(stream), y, w, w_dtype, B, K, D, mode, 0, nullptr, out);
}

extern "C" int zmoe_weighted_accumulate(void* stream, const void* acc, const void* proj, const float* gate,
                                        int64_t gate_stride, int B, int D, int acc_dtype, int no_fma, void* out) {
  ZMOE_REQUIRE(B >= 0 && D >= 1 && B <= 65535, ZMOE_EINVAL_SHAPE, "[weighted_accumulate] bad sizes.");
  ZMOE_REQUIRE(acc_dtype == ZMOE_DT_BF16 || acc_dtype == ZMOE_DT_F32, ZMOE_EINVAL_DTYPE,
               "[weighted_accumulate] acc must be bf16 or f32.");
  if (B == 0) return ZMOE_OK;
  hipLaunchKernelGGL(k_weighted_accumulate, dim3((D + 255) / 256, B), dim3(256), 0, as_stream(stream), acc,
                     static_cast<const uint16_t*>(proj), gate, gate_stride, D, acc_dtype, no_fma ? 1 : 0, out);
  return check_launch("weighted_accumulate");
}
