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

// Address-space qualifiers: pointers that reach a kernel through a struct or
// an array lose their address space and compile to flat accesses, which
// also count against the LDS wait counter (every LDS wait then waits for
// in-flight HBM loads).  Accesses on hot paths go through these instead.
#define ZMOE_GLOBAL __attribute__((address_space(1)))
#define ZMOE_LDS __attribute__((address_space(3)))

// (The host compilation pass never runs these; it only parses them.)
template <typename T>
__device__ __forceinline__ T gload(const T* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  T v;
  __builtin_memcpy(&v, (const ZMOE_GLOBAL T*)(p), sizeof(T));
  return v;
#else
  return *p;
#endif
}

template <typename T>
__device__ __forceinline__ void gstore(T* p, T v) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_memcpy((ZMOE_GLOBAL T*)(p), &v, sizeof(T));
#else
  *p = v;
#endif
}

// Device-scope (all XCDs) coherent accesses for data exchanged between
// workgroups inside one launch.
// Workgroup barrier that orders LDS only: unlike __syncthreads() it does
// not wait for this wave's outstanding global loads (prefetches stay in
// flight across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename T>
__device__ __forceinline__ T dev_load(const T* p) {
  return __hip_atomic_load((ZMOE_GLOBAL T*)(const_cast<T*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ void dev_store(T* p, T v) {
  __hip_atomic_store((ZMOE_GLOBAL T*)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Division by a launch-constant divisor d with a multiply-high and a shift
// (round-up method): q = (umulhi(a, m) + a) >> s, exact for 0 <= a < 2^31.
struct FastDiv {
  uint32_t d, m, s;
};

__host__ inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  f.s = 0;
  while ((1ull << f.s) < d) ++f.s;
  f.m = static_cast<uint32_t>(((1ull << 32) * ((1ull << f.s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t a, FastDiv f) { return (__umulhi(a, f.m) + a) >> f.s; }

// Pins a wave-uniform value in a scalar register at this point of the
// program (work assignment computed before a wait stays computed there).
template <typename T>
__device__ __forceinline__ void pin_s(T& x) {
  asm volatile("" : "+s"(x));
}

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}

// Round to nearest even with gfx950's v_cvt_pk_bf16_f32 (one instruction;
// NaN stays NaN, quieted).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_bf16(float f) {
  return static_cast<float>(static_cast<__bf16>(f));
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
// Sums over aligned groups of WIDTH lanes with DPP row operations (no LDS
// traffic): pair, quad, half-row (8) and row (16) steps; 32- and 64-lane
// groups add the rows through lane reads.  Every lane of a group receives
// the same value, and every kernel uses these same helpers, so results are
// reproducible across kernels.
#define ZMOE_DPP_ADD(v, ctrl)                                                                         \
  (v) = (v) + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), \
                                                                    (ctrl), 0xF, 0xF, false))
#define ZMOE_DPP_MAX(v, ctrl)                                                                               \
  (v) = fmaxf((v), __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), \
                                                                         (ctrl), 0xF, 0xF, false)))

constexpr int kDppQuadSwap1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// Row-pair and half-wave exchanges (gfx950 v_permlane16/32_swap): with both
// operands = v, result [0] holds the lower partner's value and [1] the
// upper partner's in every lane, so  [0] op [1]  is the same expression in
// both lanes of a pair.
__device__ __forceinline__ float rows_combine_add(float v) {
  const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<uint32_t>(q[0])) + __builtin_bit_cast(float, static_cast<uint32_t>(q[1]));
}
__device__ __forceinline__ float halves_combine_add(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) + __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}
__device__ __forceinline__ float rows_combine_max(float v) {
  const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(q[0])), __builtin_bit_cast(float, static_cast<uint32_t>(q[1])));
}
__device__ __forceinline__ float halves_combine_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])), __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

template <int WIDTH>
__device__ __forceinline__ float wave_sum_width(float v) {
  static_assert(WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "width");
  ZMOE_DPP_ADD(v, kDppQuadSwap1);
  if (WIDTH >= 4) ZMOE_DPP_ADD(v, kDppQuadSwap2);
  if (WIDTH >= 8) ZMOE_DPP_ADD(v, kDppHalfMirror);
  if (WIDTH >= 16) ZMOE_DPP_ADD(v, kDppRowMirror);
  // rows (16 lanes) combined as (row0 + row1) + (row2 + row3); every lane
  // ends with the sum of its WIDTH-lane group
  if (WIDTH >= 32) v = rows_combine_add(v);
  if (WIDTH == 64) v = halves_combine_add(v);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_width<kWave>(v); }

__device__ __forceinline__ float wave_max(float v) {
  ZMOE_DPP_MAX(v, kDppQuadSwap1);
  ZMOE_DPP_MAX(v, kDppQuadSwap2);
  ZMOE_DPP_MAX(v, kDppHalfMirror);
  ZMOE_DPP_MAX(v, kDppRowMirror);
  return halves_combine_max(rows_combine_max(v));
}

// Runtime group width L in {8, 16, 32, 64} (lanes sharing one weight row).
__device__ __forceinline__ float lanes_sum(float v, int L) {
  switch (L) {
    case 64: return wave_sum_width<64>(v);
    case 32: return wave_sum_width<32>(v);
    case 16: return wave_sum_width<16>(v);
    case 8: return wave_sum_width<8>(v);
    case 4: return wave_sum_width<4>(v);
    default: return wave_sum_width<2>(v);
  }
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
//
// The mask and offset come in as registers (AffineK) so that each pair is one
// v_and_or_b32 instead of an AND and an OR with literal operands.
struct AffineK {
  uint32_t m, o;
};

// 0x000F000F / 0x43004300 in registers the compiler cannot fold back into
// literals (call once, outside the hot loop).
__device__ __forceinline__ AffineK affine_k() {
  AffineK k{0x000F000Fu, 0x43004300u};
  asm("" : "+v"(k.m));
  asm("" : "+v"(k.o));
  return k;
}

__device__ __forceinline__ float dot_affine4_word(uint32_t w, const uint32_t xp[4], float acc, AffineK k) {
  const uint32_t m = k.m, o = k.o;
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

// Contribution of one 16-byte weight segment `w` against the matching 16
// staged activation words x0..x3 (see the layouts above).
template <int QMODE>
__device__ __forceinline__ float seg_dot(const uint4 w, const uint4 x0, const uint4 x1, const uint4 x2,
                                         const uint4 x3, AffineK k) {
  const uint32_t a0[4] = {x0.x, x0.y, x0.z, x0.w};
  const uint32_t a1[4] = {x1.x, x1.y, x1.z, x1.w};
  const uint32_t a2[4] = {x2.x, x2.y, x2.z, x2.w};
  const uint32_t a3[4] = {x3.x, x3.y, x3.z, x3.w};
  float v = 0.0f;
  if (QMODE == 0) {
    v = dot_affine4_word(w.x, a0, v, k);
    v = dot_affine4_word(w.y, a1, v, k);
    v = dot_affine4_word(w.z, a2, v, k);
    v = dot_affine4_word(w.w, a3, v, k);
  } else {
    v = dot_mxfp4_word(w.x, a0, v);
    v = dot_mxfp4_word(w.y, a1, v);
    v = dot_mxfp4_word(w.z, a2, v);
    v = dot_mxfp4_word(w.w, a3, v);
  }
  return v;
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
