// Grouped (per-expert) quantized GEMM on MFMA (grouped.hip): arguments and
// host launchers shared with the layer composition.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zmoe {

struct GroupedArgs {
  const uint16_t* a;     // activation rows (bf16)
  int64_t lda;           // elements between rows
  const float* asum;     // affine: [a rows][K/gs] group sums of a (fp32)
  const int* offsets;    // [E+2] sorted row ranges, [E+1] = number of row chunks
  const int* blocks;     // [chunks] expert | (chunk within the expert << 11)
  const int* sorted;     // [rows] pair ids in expert order; nullptr: identity
  const uint32_t* lhs;   // a row = lhs[pair] when set, else pair / a_div
  int a_div;             //   (a_div > 0), else the sorted row r itself
  int scatter;           // out row = sorted[r] (pair order), else r
  int M;
  int E;                 // experts (with blocks)
  const uint32_t* w0;    // [E, N, K/8] (gate, or the only matrix)
  const void* s0;
  const void* b0;
  const uint32_t* w1;    // up (SwiGLU only)
  const void* s1;
  const void* b1;
  int N, K, gs;
  uint16_t* out;         // bf16 [rows][ldo]
  int64_t ldo;
  float* asum_out;       // affine SwiGLU (optional): [out rows][N/gs] group sums of the bf16 outputs
};

// k_grouped_qmm over every expert's sorted rows; SwiGLU of two matrices when
// swiglu (w1/s1/b1 = up), else one matrix.
int launch_grouped(hipStream_t st, const GroupedArgs& g, int n_experts, int quant_mode, bool swiglu);
// Whether the MFMA GEMM over K inputs keeps its scales/biases in the LDS
// parameter cache (else it loads them per k block and runs slower).
bool grouped_params_cached(int quant_mode, bool swiglu, int K, int gs);
// offsets[E+2] / sorted[npairs]: the pairs (token, k) in expert order;
// blocks[]: every expert's chunks of `chunk` rows (at most npairs / chunk + E
// of them; 64 for the MFMA GEMM, kGroupedGemvRows for the GEMV).
// Sorted rows per chunk of the MFMA GEMM (one workgroup's rows).
constexpr int kGroupedChunk = 32;
int launch_sort_pairs(hipStream_t st, const uint32_t* idx, int npairs, int E, int* offsets, int* sorted, int* blocks,
                      int chunk = kGroupedChunk);
// Upper bound on the MFMA GEMM's chunks of npairs pairs over E experts.
inline int grouped_max_blocks(int npairs, int E) { return (npairs + kGroupedChunk - 1) / kGroupedChunk + E; }

// Expert-major GEMV (qmv.hip) for batches with few rows per expert: each
// expert's weight rows are read once per chunk of kGroupedGemvRows sorted
// rows and dotted with all of them (the same GroupedArgs; asum unused, the
// chunk list from launch_sort_pairs(..., kGroupedGemvRows)).
constexpr int kGroupedGemvRows = 4;
inline int grouped_gemv_max_chunks(int npairs, int E) {
  return (npairs + kGroupedGemvRows - 1) / kGroupedGemvRows + E;
}
int launch_grouped_qmv(hipStream_t st, const GroupedArgs& g, int n_experts, int quant_mode, bool swiglu);
// out[r][g] = fp32 sum of a[r][g*gs .. +gs).
int launch_row_group_sums(hipStream_t st, const uint16_t* a, int64_t lda, int rows, int K, int gs, float* out);

}  // namespace zmoe
