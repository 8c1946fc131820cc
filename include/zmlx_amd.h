/*
 * zmlx_amd -- C ABI of the MI355X (gfx950) fused quantized-MoE decode path.
 *
 * Drop-in boundary for the MoE block that ZMLX's patch(model) rewrites.  Each
 * entry point names the reference interface it replaces (paths relative to the
 * Hmbown/ZMLX source tree).
 *
 * Conventions (all entry points):
 *  - Every pointer is a caller-owned DEVICE buffer (e.g. torch data_ptr()).
 *    Nothing on these paths allocates, synchronises the host or keeps state
 *    between calls, except the layer workspace the caller passes in.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is
 *    enqueued in stream order; calls on different streams are independent.
 *  - bf16 tensors are passed as raw 16-bit storage (torch.bfloat16).
 *  - Packed weights use MLX's layout: uint32 words, element i of a word at
 *    bits 4*i.  Expert banks are stacked [E, N, K/8]; affine scales/biases
 *    are bf16 [E, N, K/group_size]; mxfp4 scales are uint8 e8m0 [E, N, K/32].
 *  - Return value: ZMOE_OK (0) or a negative ZMOE_E* code; the message of the
 *    last failure on the calling thread is available from zmoe_last_error().
 *    Argument errors are detected before anything is enqueued.
 */
#ifndef ZMLX_AMD_H_
#define ZMLX_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZMOE_OK 0
#define ZMOE_EINVAL_SHAPE (-1)
#define ZMOE_EINVAL_DTYPE (-2)
#define ZMOE_EUNSUPPORTED (-3)
#define ZMOE_EHIP (-4)

/* element types */
#define ZMOE_DT_BF16 0
#define ZMOE_DT_F32 2

/* quantization modes (MLX `mode=`) */
#define ZMOE_Q_AFFINE 0
#define ZMOE_Q_MXFP4 1

/* combine modes: see zmoe_moe_combine */
#define ZMOE_COMBINE_NATIVE 0      /* (y*w[...,None]).sum(-2), bf16 operands */
#define ZMOE_COMBINE_FP32 1        /* moe_combine_fp32: f32 FMA chain, f32 out */
#define ZMOE_COMBINE_FP32_NO_FMA 2 /* moe_combine_fp32_no_fma: f32 out, no FMA */
#define ZMOE_COMBINE_EXACT 3       /* moe_combine_exact: bf16 after every op */
#define ZMOE_COMBINE_FLOAT 4       /* moe_combine: f32 FMA chain, bf16 out */
#define ZMOE_COMBINE_NO_FMA 5      /* moe_combine_no_fma: f32 no-FMA, bf16 out */

/* router kinds for the fused layer */
#define ZMOE_ROUTER_SOFTMAX_PROBS 0  /* Qwen: precise softmax -> bf16 probs -> top-k (-> /sum) */
#define ZMOE_ROUTER_TOPK_LOGITS 1    /* moe.topk_gating_softmax fast path: top-k logits, softmax over k */
#define ZMOE_ROUTER_SIGMOID_GROUPED 2 /* DeepSeek/GLM: sigmoid + bias, grouped top-k */

/* Library version string, e.g. "zmlx_amd 0.1.0 gfx950 src:0123456789abcdef": the
 * version, the target and a hash of the sources the library was built from. */
const char* zmoe_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* zmoe_last_error(void);

/* n zeroed words of page-locked host memory that kernels may store to and
 * the host may read at any time (hipHostMalloc, mapped and coherent), for
 * zmoe_layer_desc.error_flag_host; NULL on failure.  Free with
 * zmoe_host_flags_free.  No counterpart in the reference (its kernels have
 * no waits that can give up). */
unsigned* zmoe_host_flags_alloc(int n);
void zmoe_host_flags_free(unsigned* flags);

/*
 * Fused gather + quantized GEMV + SwiGLU.
 * Replaces mx.gather_qmm_swiglu (integrations/mlx_local_integration/
 * gather_qmm_swiglu.patch:695-800, op; :552-624 host dispatch; :329-510
 * kernel) and zmlx.kernels.fused_moe.gather_qmm_swiglu (fused_moe.py:39-106).
 *
 * For each pair p < n_pairs and each row m < M:
 *   g = x[lhs[p], m, :] . deq(gate_w[rhs[p]])^T   (f32 accumulate -> bf16)
 *   u = x[lhs[p], m, :] . deq(up_w[rhs[p]])^T     (f32 accumulate -> bf16)
 *   out[p, m, :] = bf16(bf16(g * bf16(sigmoid(g))) * u)
 * x: bf16 [x_batch, M, K]; out: bf16 [n_pairs, M, N].
 * lhs/rhs: uint32 [n_pairs]; rhs values must be < E, lhs values < x_batch
 * (not checked on the device).
 * Requirements: K % 256 == 0, group_size in {32,64,128} (affine) / 32 (mxfp4),
 * bits == 4.  gate_b/up_b are ignored (may be NULL) for mxfp4.
 */
int zmoe_gather_qmm_swiglu(void* stream, const void* x, int64_t x_batch,
                           const uint32_t* gate_w, const void* gate_s, const void* gate_b,
                           const uint32_t* up_w, const void* up_s, const void* up_b,
                           const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                           int64_t n_pairs, int M, int N, int K, int E,
                           int group_size, int bits, int quant_mode, void* out);

/*
 * Gather + quantized GEMV (the down projection).
 * Replaces mx.gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices,
 * transpose=True) as called by QuantizedSwitchLinear (moe_mlp.py:572) and
 * moe.gather_qmm_combine_quantized (moe.py:2043-2174).
 * out[p, m, :] = bf16(x[lhs[p], m, :] . deq(w[rhs[p]])^T); same layouts and
 * requirements as zmoe_gather_qmm_swiglu.
 */
int zmoe_gather_qmm(void* stream, const void* x, int64_t x_batch,
                    const uint32_t* w, const void* scales, const void* biases,
                    const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                    int64_t n_pairs, int M, int N, int K, int E,
                    int group_size, int bits, int quant_mode, void* out);

/*
 * Grouped gather + quantized matmul on MFMA: the batched / prefill form of
 * zmoe_gather_qmm(_swiglu) for M == 1 rows and many pairs.  Replaces
 * mx.gather_qmm(..., sorted_indices=True) as mlx_lm's SwitchGLU calls it for
 * more than one token (the sort path noted at moe_mlp.py:540-543; the
 * reference's fused op is token-gated to M == 1, moe_mlp.py:298, 523-525).
 *   out[p, :] = bf16(x[lhs[p], :] . deq(w[rhs[p]])^T)                (up_w NULL)
 *   out[p, :] = bf16(bf16(g*bf16(sigmoid(g))) * u)  with g, u as above (SwiGLU)
 * x: bf16 [x_batch, K]; out: bf16 [n_pairs, N] in pair order; rhs need not be
 * sorted (pairs are counting-sorted by expert in the workspace).  The
 * products are exact as in the GEMV (fp32 accumulation order differs).
 * workspace: zmoe_grouped_gather_qmm_workspace_size(...) bytes, no zero-fill.
 * Requirements: N % 32 == 0, K % 128 == 0, E <= 1024; group_size / mode as
 * zmoe_gather_qmm.
 */
size_t zmoe_grouped_gather_qmm_workspace_size(int64_t n_pairs, int x_batch, int E, int K, int group_size);
int zmoe_grouped_gather_qmm(void* stream, const void* x, int64_t x_batch, const uint32_t* w, const void* scales,
                            const void* biases, const uint32_t* up_w, const void* up_scales, const void* up_biases,
                            const uint32_t* lhs_indices, const uint32_t* rhs_indices, int64_t n_pairs, int N, int K,
                            int E, int group_size, int bits, int quant_mode, void* workspace, size_t workspace_bytes,
                            void* out);

/*
 * Dense router projection (the gate nn.Linear of the MoE block,
 * moe_mlp.py:218 `gate_fn(x)`; deepseek_router.py:108 `x @ weight.T`).
 * x: bf16 [B, H]; w: bf16 [E, H]; out: bf16 [B, E] (out_dtype ZMOE_DT_BF16)
 * or f32 [B, E] (ZMOE_DT_F32, unrounded accumulation).  H % 8 == 0.
 */
int zmoe_dense_logits(void* stream, const void* x, const void* w, int B, int E, int H,
                      int out_dtype, void* out);

/*
 * Qwen3 MoE gating (moe_mlp.py:255-266): precise softmax of bf16 logits ->
 * bf16 probabilities -> top-k (ties: lower expert index first, order by
 * probability descending) -> gather -> if norm_topk_prob, divide by the bf16
 * sum.  logits: bf16 [B, E]; out_w: bf16 [B, k]; out_idx: uint32 [B, k].
 * E <= 1024, 1 <= k <= 16.
 */
int zmoe_router_softmax_topk(void* stream, const void* logits, int B, int E, int k,
                             int norm_topk_prob, void* out_w, uint32_t* out_idx);

/*
 * moe.topk_gating_softmax (moe.py:1239-1396), compute dtype f32.
 * logits: bf16 or f32 [B, E] (in_dtype); expert_bias: f32 [E] or NULL.
 * No bias and norm_topk_prob != 0: top-k of the logits, softmax over the k
 * selected (moe.py:1287-1315).  Otherwise: full softmax, + bias, top-k,
 * optional /(sum + 1e-20) (moe.py:1326-1377).
 * out_w: f32 [B, k]; out_idx: uint32 [B, k]; E <= 1024, 1 <= k <= 16.
 * Also serves moe.router_argpartition_logits_topk (moe.py:1448-1490), whose
 * result is the no-bias renormalised case.
 */
int zmoe_topk_gating_softmax(void* stream, const void* logits, int in_dtype, int B, int E,
                             int k, const float* expert_bias, int norm_topk_prob,
                             float* out_w, uint32_t* out_idx);

/*
 * moe.deepseek_router_topk_sigmoid (moe.py:1745-1817; kernel :1501-1679)
 * with the routed scaling of deepseek_router.py:118-119.
 * logits: f32 [B, E]; bias: f32 [E].  score = sigmoid(l) + bias; groups of
 * E/n_group keep the topk_group best (group score = top1+top2; others set to
 * 0.0); top-k with ties to the lower index; weights = sigmoid / sum, times
 * routed_scaling_factor.  out_w f32 [B,k], out_idx uint32 [B,k] in selection
 * order.  E <= 1024, k <= 16, E % n_group == 0, 1 <= topk_group <= n_group.
 */
int zmoe_deepseek_router_topk_sigmoid(void* stream, const float* logits, const float* bias,
                                      int B, int E, int k, int n_group, int topk_group,
                                      float routed_scaling_factor, float* out_w,
                                      uint32_t* out_idx);

/*
 * MoE combine: out[b, d] = sum_k w[b, k] * y[b, k, d], k ascending.
 * Replaces moe.moe_combine / _no_fma / _exact / _fp32 / _fp32_no_fma
 * (moe.py:830-1127) and the native (y*w[...,None]).sum(-2) (moe_mlp.py:1043).
 * y: bf16 [B, K, D]; w: bf16 or f32 [B, K] (w_dtype);
 * out: f32 for ZMOE_COMBINE_FP32 / FP32_NO_FMA, bf16 otherwise.
 */
int zmoe_moe_combine(void* stream, const void* y, const void* w, int w_dtype, int B, int K,
                     int D, int mode, void* out);

/*
 * Two-input SwiGLU out = SiLU(gate) * up, elementwise over n elements.
 * Replaces transformer.swiglu2 (transformer.py:882-935).  dtype ZMOE_DT_BF16
 * (MLX op-by-op rounding: sigmoid, gate*sigmoid and the product each rounded
 * to bf16) or ZMOE_DT_F32; gate, up, out of that dtype.
 */
int zmoe_swiglu2(void* stream, const void* gate, const void* up, int64_t n, int dtype, void* out);

/*
 * Its backward (transformer.py:899-914): dgate = c*up*(s + g*s*(1 - s)),
 * dup = c*g*s with s = sigmoid(gate), c = cotan; f32 arithmetic, one rounding
 * to the dtype.
 */
int zmoe_swiglu2_backward(void* stream, const void* gate, const void* up, const void* cotan, int64_t n,
                          int dtype, void* dgate, void* dup);

/*
 * Token-to-expert-slot copy out[b, k, :] = x[b, :] for k < K.  Replaces
 * moe.moe_dispatch (moe.py:776-827; its indices only give K).  x: [B, D],
 * out: [B, K, D], elements of elem_bytes (1, 2, 4 or 8) bytes.
 */
int zmoe_moe_dispatch(void* stream, const void* x, int64_t B, int D, int K, int elem_bytes, void* out);

/*
 * Streaming combine step out = acc + gate[b] * proj[b, :] (moe.py:1820-1921,
 * used by gather_qmm_combine_quantized's streaming loop :2143-2172).
 * acc/out: bf16 or f32 (acc_dtype, same for both; in-place allowed);
 * proj: bf16 [B, D]; gate: f32 [B] (gate_stride elements between rows).
 */
int zmoe_weighted_accumulate(void* stream, const void* acc, const void* proj,
                             const float* gate, int64_t gate_stride, int B, int D,
                             int acc_dtype, int no_fma, void* out);

/*
 * Description of one quantized MoE layer for the fused decode path.  All
 * weight pointers are device pointers in MLX layout (see top of file).
 */
typedef struct zmoe_layer_desc {
  int hidden;          /* H */
  int n_experts;       /* E */
  int top_k;           /* K */
  int inter;           /* I: routed expert intermediate size */
  int group_size;      /* affine: 32/64/128; mxfp4: 32 */
  int bits;            /* 4 */
  int quant_mode;      /* ZMOE_Q_* */
  int router_kind;     /* ZMOE_ROUTER_* */
  int norm_topk_prob;  /* renormalise the selected weights */
  int n_group;         /* grouped router only (1 = no grouping) */
  int topk_group;
  float routed_scaling_factor;
  int combine_mode;    /* ZMOE_COMBINE_*; the layer output is always bf16 */
  const void* router_w;     /* bf16 [E, H] */
  const float* router_bias; /* f32 [E] or NULL (expert_bias / e_score_correction_bias) */
  const uint32_t* gate_w; const void* gate_s; const void* gate_b; /* [E, I, H/8] */
  const uint32_t* up_w;   const void* up_s;   const void* up_b;
  const uint32_t* down_w; const void* down_s; const void* down_b; /* [E, H, I/8] */
  int shared_inter;         /* 0 = no shared expert */
  const uint32_t* sh_gate_w; const void* sh_gate_s; const void* sh_gate_b; /* [I_s, H/8] */
  const uint32_t* sh_up_w;   const void* sh_up_s;   const void* sh_up_b;
  const uint32_t* sh_down_w; const void* sh_down_s; const void* sh_down_b; /* [H, I_s/8] */
  int flags;                /* ZMOE_LAYER_* bits */
  /* Single-launch kernels: when a wait for data exchanged between workgroups
   * gives up, the kernel sets the workspace's sticky error word, writes NaN
   * into the outputs that depend on the missing data, and stores 1 here if
   * non-NULL (host-visible memory, e.g. hipHostMalloc), so that the host can
   * notice without a synchronisation.  No counterpart in the reference
   * (MLX kernels have no cross-workgroup waits). */
  unsigned* error_flag_host;
  /* Polls before such a wait gives up; 0 = the library's default.  Tests set
   * it small to force the give-up path from the host. */
  int spin_limit;
} zmoe_layer_desc;

/* zmoe_layer_desc.flags */
#define ZMOE_LAYER_FORCE_MULTI 1  /* run the kernel sequence even when the single-launch kernel applies */
#define ZMOE_LAYER_TRACE 2        /* single-launch kernel: record per-workgroup phase timestamps */

/*
 * Where ZMOE_LAYER_TRACE stamps land: byte offset into the workspace of a
 * uint64 array [n_blocks][n_slots] of 100 MHz realtime-counter values, one
 * row per workgroup, slots 0..12 = kernel start, router partials done,
 * x staged, router logits received, token 0 routed, units built, first
 * gate/up batch done, gate/up done, down prefetch issued, phase-A LDS
 * released, act rows received, down done, combine done; slots 13/14 =
 * shader-clock counter at
 * start / end.  Returns 0 if the single-launch kernel does not apply.
 * No counterpart in the reference (its profiling is wall-clock only,
 * profile.py:22); used for performance analysis.
 */
size_t zmoe_moe_layer_trace_info(const zmoe_layer_desc* desc, int B, int* n_blocks, int* n_slots);

/* Bytes of device workspace zmoe_moe_layer needs for B tokens.  The
 * workspace belongs to one (desc, B): zero-fill it once before its first use
 * and do not write it otherwise.  The single-launch kernel keeps a launch
 * count per workgroup in it and tags the data its workgroups exchange with
 * that count.  Bytes 128..131 hold a sticky error word: nonzero if a wait for
 * exchanged data timed out; the outputs of that call are then NaN where they
 * depend on the missing data (zero-fill the workspace again before reuse). */
size_t zmoe_moe_layer_workspace_size(const zmoe_layer_desc* desc, int B);

/*
 * Whole MoE block forward for B tokens (the patched __call__ of
 * moe_mlp.py:883-1063 / deepseek_router.py:76-120):
 *   router logits -> gating -> gate/up + SwiGLU -> down -> combine (+ shared)
 * x: bf16 [B, H]; out: bf16 [B, H].  Optional outputs (may be NULL):
 * out_idx uint32 [B, K] and out_w f32 [B, K] (the routing actually used).
 * workspace: device buffer of zmoe_moe_layer_workspace_size bytes, zeroed
 * before first use, not shared by calls that may overlap on the device.
 * Decode batches (B <= 8, within LDS limits) run as ONE persistent kernel
 * launch with two grid barriers; larger batches run as a kernel sequence.
 */
int zmoe_moe_layer(void* stream, const zmoe_layer_desc* desc, const void* x, int B, void* out,
                   uint32_t* out_idx, float* out_w, void* workspace, size_t workspace_bytes);

/*
 * zmoe_moe_layer without a workspace argument: allocates nothing (no
 * hipMalloc / hipFree, no allocating library call), for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid it.  No counterpart in the reference.  It runs the kernel
 * sequence with its buffers in a library-owned device array of
 * zmoe_moe_layer_noalloc_max_bytes() bytes per GPU (held until the process
 * ends); a batch whose buffers exceed it is rejected (ZMOE_EINVAL_SHAPE).
 * Outputs equal zmoe_moe_layer's.  Calls that overlap on one GPU share the
 * array and race: issue them on one stream.
 */
int zmoe_moe_layer_noalloc(void* stream, const zmoe_layer_desc* desc, const void* x, int B, void* out,
                           uint32_t* out_idx, float* out_w);
size_t zmoe_moe_layer_noalloc_max_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* ZMLX_AMD_H_ */
