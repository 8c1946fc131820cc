// Combine arithmetic shared by the combine kernels and the fused layer:
// out = sum_k w_k * y_k, k ascending, in the rounding modes of the
// reference's combine family (moe.py:830-1127, moe_mlp.py:1043).
#pragma once

#include "../../include/zmlx_amd.h"
#include "zmoe_common.h"

namespace zmoe {

// Products rounded to fp32 and sums rounded to fp32 separately (no FMA).
__device__ __forceinline__ float mul_nofma(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_nofma(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// Combine of one output element under `mode` (ZMOE_COMBINE_*).  `yk(k)`
// returns expert k's value (bf16 as f32), `wk(k)` its gate weight.
template <typename YF, typename WF>
__device__ __forceinline__ float combine_one(int mode, int K, YF yk, WF wk) {
  float acc = 0.0f;
  switch (mode) {
    case ZMOE_COMBINE_NATIVE:
      for (int k = 0; k < K; ++k) acc = add_nofma(acc, round_bf16(mul_nofma(wk(k), yk(k))));
      return round_bf16(acc);
    case ZMOE_COMBINE_FP32:
    case ZMOE_COMBINE_FLOAT:
      for (int k = 0; k < K; ++k) acc = fmaf(wk(k), yk(k), acc);
      return mode == ZMOE_COMBINE_FLOAT ? round_bf16(acc) : acc;
    case ZMOE_COMBINE_FP32_NO_FMA:
    case ZMOE_COMBINE_NO_FMA:
      for (int k = 0; k < K; ++k) acc = add_nofma(acc, mul_nofma(wk(k), yk(k)));
      return mode == ZMOE_COMBINE_NO_FMA ? round_bf16(acc) : acc;
    default:  // ZMOE_COMBINE_EXACT
      for (int k = 0; k < K; ++k) acc = round_bf16(add_nofma(acc, round_bf16(mul_nofma(round_bf16(wk(k)), yk(k)))));
      return acc;
  }
}

__device__ __forceinline__ bool combine_f32_out(int mode) {
  return mode == ZMOE_COMBINE_FP32 || mode == ZMOE_COMBINE_FP32_NO_FMA;
}

}  // namespace zmoe
