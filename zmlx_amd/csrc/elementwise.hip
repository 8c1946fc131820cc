// Elementwise ops of the MoE block's operator surface: the two-input SwiGLU
// (transformer.swiglu2 and its backward, transformer.py:882-935) and the
// token-to-expert-slot copy (moe.moe_dispatch, moe.py:776-827).  All are
// HBM-bound streams: 16-byte accesses where the row length allows, a
// grid-stride loop sized to the device.
#include "zmoe_common.h"
#include "zmoe_host.h"

namespace zmoe {

// SiLU(g) * u.  bf16: MLX's op-by-op rounding (swiglu_bf16: sigmoid, g * s
// and the product each rounded to bf16); f32: g * sigmoid(g) * u in f32.
// The sigmoid is the reference header's form: 1 / (1 + exp(|x|)) mirrored.
template <bool BF16>
__global__ __launch_bounds__(256) void k_swiglu2(const void* __restrict__ gate, const void* __restrict__ up,
                                                 int64_t n, void* __restrict__ out) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    if (BF16) {
      const float g = bf16_bits_to_f32(static_cast<const uint16_t*>(gate)[i]);
      const float u = bf16_bits_to_f32(static_cast<const uint16_t*>(up)[i]);
      static_cast<uint16_t*>(out)[i] = static_cast<uint16_t>(swiglu_bf16(g, u));
    } else {
      const float g = static_cast<const float*>(gate)[i];
      const float u = static_cast<const float*>(up)[i];
      static_cast<float*>(out)[i] = g * sigmoid_abs(g) * u;
    }
  }
}

// Backward (transformer.py:899-914): s = sigmoid(g), swish = g s,
// dgate = c u (s + swish (1 - s)), dup = c swish; computed in f32 from the
// inputs, rounded once to the output dtype.
template <bool BF16>
__global__ __launch_bounds__(256) void k_swiglu2_bwd(const void* __restrict__ gate, const void* __restrict__ up,
                                                     const void* __restrict__ cotan, int64_t n,
                                                     void* __restrict__ dgate, void* __restrict__ dup) {
  auto ld = [](const void* p, int64_t i) {
    return BF16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
  };
  auto st = [](void* p, int64_t i, float v) {
    if (BF16)
      static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    else
      static_cast<float*>(p)[i] = v;
  };
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float g = ld(gate, i), u = ld(up, i), c = ld(cotan, i);
    const float s = sigmoid_abs(g);
    const float swish = g * s;
    st(dgate, i, c * u * (s + swish * (1.0f - s)));
    st(dup, i, c * swish);
  }
}

// out[(b * K + k) * D + d] = x[b * D + d]: row b copied into its K slots.
// W-byte words (16 when a row is a multiple of 16 bytes, else the element).
template <typename W>
__global__ __launch_bounds__(256) void k_moe_dispatch(const W* __restrict__ x, int64_t B, int64_t words, int K,
                                                      W* __restrict__ out) {
  const int64_t total = B * words;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t b = i / words, d = i - b * words;
    const W v = x[i];
    W* o = out + b * K * words + d;
    for (int k = 0; k < K; ++k) o[k * words] = v;
  }
}

static unsigned grid_for(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return static_cast<unsigned>(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

}  // namespace zmoe

using namespace zmoe;

extern "C" int zmoe_swiglu2(void* stream, const void* gate, const void* up, int64_t n, int dtype, void* out) {
  ZMOE_REQUIRE(dtype == ZMOE_DT_BF16 || dtype == ZMOE_DT_F32, ZMOE_EINVAL_DTYPE,
               "[swiglu2] dtype must be bf16 or f32.");
  ZMOE_REQUIRE(n >= 0, ZMOE_EINVAL_SHAPE, "[swiglu2] n must be >= 0.");
  if (n == 0) return ZMOE_OK;
  ZMOE_REQUIRE(gate && up && out, ZMOE_EINVAL_SHAPE, "[swiglu2] null pointer.");
  auto fn = dtype == ZMOE_DT_BF16 ? k_swiglu2<true> : k_swiglu2<false>;
  hipLaunchKernelGGL(fn, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), gate, up, n, out);
  return check_launch("swiglu2");
}

extern "C" int zmoe_swiglu2_backward(void* stream, const void* gate, const void* up, const void* cotan, int64_t n,
                                     int dtype, void* dgate, void* dup) {
  ZMOE_REQUIRE(dtype == ZMOE_DT_BF16 || dtype == ZMOE_DT_F32, ZMOE_EINVAL_DTYPE,
               "[swiglu2] dtype must be bf16 or f32.");
  ZMOE_REQUIRE(n >= 0, ZMOE_EINVAL_SHAPE, "[swiglu2] n must be >= 0.");
  if (n == 0) return ZMOE_OK;
  ZMOE_REQUIRE(gate && up && cotan && dgate && dup, ZMOE_EINVAL_SHAPE, "[swiglu2] null pointer.");
  auto fn = dtype == ZMOE_DT_BF16 ? k_swiglu2_bwd<true> : k_swiglu2_bwd<false>;
  hipLaunchKernelGGL(fn, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), gate, up, cotan, n, dgate, dup);
  return check_launch("swiglu2 backward");
}

extern "C" int zmoe_moe_dispatch(void* stream, const void* x, int64_t B, int D, int K, int elem_bytes, void* out) {
  ZMOE_REQUIRE(B >= 0 && D >= 1 && K >= 1, ZMOE_EINVAL_SHAPE, "[moe_dispatch] need B >= 0, D >= 1, K >= 1.");
  ZMOE_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8, ZMOE_EINVAL_DTYPE,
               "[moe_dispatch] element size must be 1, 2, 4 or 8 bytes.");
  if (B == 0) return ZMOE_OK;
  ZMOE_REQUIRE(x && out, ZMOE_EINVAL_SHAPE, "[moe_dispatch] null pointer.");
  hipStream_t st = as_stream(stream);
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const bool vec = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (vec) {
    const int64_t words = row_bytes / 16;
    hipLaunchKernelGGL(k_moe_dispatch<uint4>, dim3(grid_for(B * words)), dim3(256), 0, st,
                       static_cast<const uint4*>(x), B, words, K, static_cast<uint4*>(out));
  } else if (elem_bytes == 1) {
    hipLaunchKernelGGL(k_moe_dispatch<uint8_t>, dim3(grid_for(B * D)), dim3(256), 0, st,
                       static_cast<const uint8_t*>(x), B, static_cast<int64_t>(D), K, static_cast<uint8_t*>(out));
  } else if (elem_bytes == 2) {
    hipLaunchKernelGGL(k_moe_dispatch<uint16_t>, dim3(grid_for(B * D)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(x), B, static_cast<int64_t>(D), K, static_cast<uint16_t*>(out));
  } else if (elem_bytes == 4) {
    hipLaunchKernelGGL(k_moe_dispatch<uint32_t>, dim3(grid_for(B * D)), dim3(256), 0, st,
                       static_cast<const uint32_t*>(x), B, static_cast<int64_t>(D), K, static_cast<uint32_t*>(out));
  } else {
    hipLaunchKernelGGL(k_moe_dispatch<uint64_t>, dim3(grid_for(B * D)), dim3(256), 0, st,
                       static_cast<const uint64_t*>(x), B, static_cast<int64_t>(D), K, static_cast<uint64_t*>(out));
  }
  return check_launch("moe_dispatch");
}
