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
__global__ __launch_bounds__(256) void k_moe_combine(const uint16_t* __restrict__ y, const void* __restrict__ w,
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

int launch_combine(hipStream_t st, const void* y, const void* w, int w_dtype, int B, int K, int D, int mode,
                   int force_bf16, const void* shared, void* out) {
  hipLaunchKernelGGL(k_moe_combine, dim3((D + 255) / 256, B), dim3(256), 0, st, static_cast<const uint16_t*>(y), w,
                     w_dtype, K, D, mode, force_bf16, static_cast<const uint16_t*>(shared), out);
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
