// Device-side building blocks shared by every zmlx_amd kernel (gfx950, wave64).
//
// Numeric conventions (they define the parity contract with the CPU oracle):
//  * bf16 values are carried as raw uint16 bits; conversion to fp32 is exact,
//    conversion from fp32 rounds to nearest-even (NaN stays NaN).
//  * Affine 4-bit weights are MLX-packed: uint32 words, element i of a word at
//    bits 4*i, low nibble first; w_hat = scale*q + bias per group.
//  * mxfp4 weights use the same packing with OCP e2m1 codes and one e8m0
//    scale byte per 32 elements (no bias).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zmoe {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// ---------------------------------------------------------------------------
// Sigmoid / exp
// ---------------------------------------------------------------------------
// Logistic function in fp32, 1/(1+exp(-x)) with the |x| form so it never
// overflows (same algebra as the reference's kk_sigmoid, msl.py:20-24).
__device__ __forceinline__ float sigmoid_abs(float x) {
  float y = 1.0f / (1.0f + expf(fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

// MLX `nn.silu(g) * u` on bf16 operands: sig = bf16(sigmoid(g)),
// silu = bf16(g*sig), out = bf16(silu*u).  Returns bf16 bits.
__device__ __forceinline__ uint32_t swiglu_bf16(float g_bf16, float u_bf16) {
  float sig = round_bf16(sigmoid_abs(g_bf16));
  float silu = round_bf16(g_bf16 * sig);
  return f32_to_bf16_bits(silu * u_bf16);
}

// ---------------------------------------------------------------------------
// Wave reductions
// ---------------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ float wave_sum_width(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WIDTH);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_width<kWave>(v); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// ---------------------------------------------------------------------------
// Quantized dot products on one 16-byte segment (32 weights)
// ---------------------------------------------------------------------------
// Activation layout for affine 4-bit: every 8 consecutive elements
// e0..e7 of x are stored as four bf16 pairs (e0,e4) (e1,e5) (e2,e6) (e3,e7)
// so that masking nibble i and nibble i+4 of a packed word with 0x000F000F
// (after a shift by 4*i) yields a bf16x2 operand directly:
//    bits (q | 0x4300) are the bf16 number 128+q (exact for q < 128).
// The dot2 therefore accumulates sum x*(128+q); the caller removes the
// offset with the per-segment activation sum:  sum x*q = v - 128*sum x.
__device__ __forceinline__ float dot_affine4_word(uint32_t w, const uint32_t xp[4], float acc) {
  const uint32_t m = 0x000F000Fu, o = 0x43004300u;
  uint32_t a = (w & m) | o;
  uint32_t b = ((w >> 4) & m) | o;
  uint32_t c = ((w >> 8) & m) | o;
  uint32_t d = ((w >> 12) & m) | o;
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, xp[0]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, b), __builtin_bit_cast(bf16x2_t, xp[1]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, c), __builtin_bit_cast(bf16x2_t, xp[2]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d), __builtin_bit_cast(bf16x2_t, xp[3]), acc, false);
  return acc;
}

// mxfp4: the gfx950 converter turns one byte (two e2m1 codes, low nibble
// first) into a bf16 pair; with scale 1.0 every e2m1 value is exact in bf16.
// Activations for mxfp4 stay in natural order (pairs (e0,e1) (e2,e3) ...).
__device__ __forceinline__ float dot_mxfp4_word(uint32_t w, const uint32_t xp[4], float acc) {
  bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0);
  bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1);
  bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2);
  bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3);
  acc = __builtin_amdgcn_fdot2_f32_bf16(p0, __builtin_bit_cast(bf16x2_t, xp[0]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(p1, __builtin_bit_cast(bf16x2_t, xp[1]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(p2, __builtin_bit_cast(bf16x2_t, xp[2]), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(p3, __builtin_bit_cast(bf16x2_t, xp[3]), acc, false);
  return acc;
}

// Accumulate one segment's contribution into `acc` with an explicit operation
// order (identical in every kernel, independent of FP contraction choices):
//   affine: acc + fma(s, v, c*xsum)   (v = sum x*(128+q), c = bias - 128*scale)
//   mxfp4:  fma(s, v, acc)
template <int QMODE>
__device__ __forceinline__ float seg_accum(float acc, float s, float c, float v, float xsum) {
#pragma clang fp contract(off)
  if (QMODE == 0) {
    const float cx = c * xsum;
    return acc + fmaf(s, v, cx);
  }
  return fmaf(s, v, acc);
}

// e8m0 scale byte -> fp32 2^(e-127); 0xFF -> NaN; e == 0 -> 2^-127 (subnormal).
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  if (e == 0xFFu) return __uint_as_float(0x7fc00000u);
  if (e == 0u) return __uint_as_float(0x00400000u);
  return __uint_as_float(e << 23);
}

}  // namespace zmoe
