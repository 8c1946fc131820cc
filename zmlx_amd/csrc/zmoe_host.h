// Host-side helpers shared by the C-ABI translation units: error state,
// argument checks and status codes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/zmlx_amd.h"

namespace zmoe {

// Leading bytes of the layer workspace reserved for the single-launch
// kernel's barrier state; the multi-kernel path's buffers start after it.
constexpr size_t kSyncBlockBytes = 16384;
constexpr size_t kSyncErrorByte = 128;

void set_error(const std::string& msg);

inline int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(ZMOE_EHIP, std::string("[") + what + "] HIP launch failed: " + hipGetErrorString(e));
  }
  return ZMOE_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int gcd_int(int a, int b) {
  while (b) {
    int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Internal launchers shared between translation units (arguments validated by
// the caller).  Null lhs -> activation row p / lhs_div; null rhs -> expert 0.
int dispatch_qmv(bool swiglu, void* stream, const void* x, const uint32_t* wg, const void* sg, const void* bg,
                 const uint32_t* wu, const void* su, const void* bu, const uint32_t* lhs, const uint32_t* rhs,
                 int lhs_div, int64_t n_pairs, int M, int N, int K, int quant_mode, int gshift, void* out);
int launch_combine(hipStream_t st, const void* y, const void* w, int w_dtype, int B, int K, int D, int mode,
                   int force_bf16, const void* shared, void* out);
// router projection on MFMA (prefill batches; router.hip)
// With xsum: also the fp32 sums of every gs-group of each row of x,
// xsum[B][H / gs] (hidden 2048), bit-identical to k_row_group_sums'.
int launch_logits_mfma(hipStream_t st, const void* x, const void* w, int B, int E, int H, int out_dtype, void* out,
                       float* xsum = nullptr, int gs = 64);
int launch_topk_gating(hipStream_t st, const void* logits, int in_dtype, int B, int E, int k, const float* bias,
                       int norm, int out_bf16, void* out_w, uint32_t* out_idx);
int launch_deepseek_router(hipStream_t st, const void* logits, int in_dtype, const float* bias, int B, int E, int k,
                           int n_group, int topk_group, float scaling, float* out_w, uint32_t* out_idx);

// Fused single-launch decode layer (layer_fused.hip).
bool fused_supported(const zmoe_layer_desc* d, int B);
size_t fused_workspace_bytes(const zmoe_layer_desc* d, int B);
size_t fused_trace_info(const zmoe_layer_desc* d, int B, int* n_blocks, int* n_slots);
int launch_fused(hipStream_t st, const zmoe_layer_desc* d, const void* x, int B, void* out, uint32_t* out_idx,
                 float* out_w, void* workspace);

}  // namespace zmoe

#define ZMOE_REQUIRE(cond, code, msg)      \
  do {                                     \
    if (!(cond)) return ::zmoe::fail((code), (msg)); \
  } while (0)
