// Whole MoE block forward (zmoe_moe_layer): router projection, gating,
// gate/up + SwiGLU, down projection, combine and the optional shared expert,
// enqueued back to back on one stream with all intermediates in the
// caller's workspace.
#include "zmoe_common.h"
#include "zmoe_grouped.h"
#include "zmoe_host.h"

#include <cstdlib>
#include <mutex>
#include <string>

namespace zmoe {

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// How the kernel sequence runs the routed experts (the reference's mlx_lm
// SwitchGLU sorts the pairs by expert from 64 indices on,
// moe_mlp.py:540-543):
//   per-pair GEMV    below kGroupedGemvMinB tokens, or while the experts
//                    average under kGroupedGemvRowsMin rows: each (token, k)
//                    pair streams its expert's rows (k_gather_qmv);
//   expert-major GEMV (pairs sorted by expert): each expert's rows are read
//                    once per 4 of its rows (k_grouped_qmv);
//   grouped MFMA GEMM from kGroupedMinB tokens when the experts average at
//                    least kGroupedMfmaRows rows or its parameters fit the
//                    LDS cache (k_grouped_qmm).
// ZMOE_GROUPED_MIN_B overrides kGroupedMinB; ZMOE_GROUPED_GEMV=0 turns the
// expert-major GEMV off.
constexpr int kGroupedMinB = 32;
constexpr int kGroupedGemvMinB = 9;
constexpr int kGroupedMfmaRows = 16;
constexpr int kGroupedGemvRowsMin = 2;
enum SeqMode { kSeqPairs = 0, kSeqGemv = 1, kSeqMfma = 2 };

static int grouped_min_b() {
  static int v = -1;
  if (v < 0) {
    const char* e = getenv("ZMOE_GROUPED_MIN_B");
    v = e ? atoi(e) : kGroupedMinB;
    if (v < 1) v = 1;
  }
  return v;
}

static bool gemv_enabled() {
  static int v = -1;
  if (v < 0) {
    const char* e = getenv("ZMOE_GROUPED_GEMV");
    v = (e && atoi(e) == 0) ? 0 : 1;
  }
  return v == 1;
}

static bool use_grouped(const zmoe_layer_desc* d, int B) {
  return B >= grouped_min_b() && d->hidden % 128 == 0 && d->inter % 128 == 0 && d->n_experts <= 1024;
}

static SeqMode seq_mode(const zmoe_layer_desc* d, int B) {
  const int64_t pairs = static_cast<int64_t>(B) * d->top_k;
  const bool gemv_ok = gemv_enabled() && B >= kGroupedGemvMinB && d->n_experts <= 1024 &&
                       pairs >= static_cast<int64_t>(kGroupedGemvRowsMin) * d->n_experts;
  // the MFMA GEMM wins from 16 rows per expert, and below that too while its
  // parameters fit the LDS cache (measured: Qwen3 B=32, 2 rows per expert,
  // 157 us vs 170 us on the GEMV; DeepSeek-V3 B=64, hidden 7168, 3182 us vs
  // 1846 us)
  const bool cached = grouped_params_cached(d->quant_mode, true, d->hidden, d->group_size);
  if (use_grouped(d, B) &&
      (pairs >= static_cast<int64_t>(kGroupedMfmaRows) * d->n_experts || cached || !gemv_ok))
    return kSeqMfma;
  return gemv_ok ? kSeqGemv : kSeqPairs;
}

struct LayerWs {
  void* logits;   // [B, E] bf16
  uint32_t* idx;  // [B, K]
  void* w;        // [B, K] bf16 or f32
  void* act;      // [B*K, I] bf16
  void* y;        // [B*K, H] bf16
  void* sh_act;   // [B, I_s] bf16
  void* sh_y;     // [B, H] bf16
  int* offsets;   // grouped path: [E+1] pair ranges by expert
  int* sorted;    //   [B*K] pairs in expert order
  int* blocks;    //   32-row blocks of every expert
  float* xsum;    //   affine: [B][H/gs] group sums of x
  float* asum;    //   affine: [B*K][I/gs] group sums of act
  size_t bytes;
};

static LayerWs layout_ws(const zmoe_layer_desc* d, int B, char* base) {
  LayerWs ws{};
  size_t off = 0;
  auto take = [&](size_t n) {
    void* p = base ? base + off : nullptr;
    off += align_up(n);
    return p;
  };
  const size_t BK = static_cast<size_t>(B) * d->top_k;
  ws.logits = take(static_cast<size_t>(B) * d->n_experts * 2);
  ws.idx = static_cast<uint32_t*>(take(BK * 4));
  ws.w = take(BK * 4);
  ws.act = take(BK * d->inter * 2);
  ws.y = take(BK * d->hidden * 2);
  ws.sh_act = take(static_cast<size_t>(B) * (d->shared_inter > 0 ? d->shared_inter : 0) * 2);
  ws.sh_y = take(static_cast<size_t>(B) * (d->shared_inter > 0 ? d->hidden : 0) * 2);
  const SeqMode mode = seq_mode(d, B);
  if (mode != kSeqPairs) {
    const int nb = mode == kSeqMfma ? grouped_max_blocks(static_cast<int>(BK), d->n_experts)
                                    : grouped_gemv_max_chunks(static_cast<int>(BK), d->n_experts);
    ws.offsets = static_cast<int*>(take(static_cast<size_t>(d->n_experts + 2) * 4));
    ws.sorted = static_cast<int*>(take(BK * 4));
    ws.blocks = static_cast<int*>(take(static_cast<size_t>(nb) * 4));
  }
  if (mode == kSeqMfma) {
    const int gs = d->group_size > 0 ? d->group_size : 32;
    ws.xsum = static_cast<float*>(take(static_cast<size_t>(B) * (d->hidden / gs) * 4));
    ws.asum = static_cast<float*>(take(BK * (d->inter / gs) * 4));
  }
  ws.bytes = off;
  return ws;
}

__global__ void k_weights_to_f32(const void* __restrict__ w, int is_f32, int n, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n)
    out[i] = is_f32 ? static_cast<const float*>(w)[i] : bf16_bits_to_f32(static_cast<const uint16_t*>(w)[i]);
}

static int validate_layer(const zmoe_layer_desc* d, int B) {
  ZMOE_REQUIRE(d != nullptr, ZMOE_EINVAL_SHAPE, "[moe_layer] null descriptor.");
  ZMOE_REQUIRE(B >= 0 && B <= 65535, ZMOE_EINVAL_SHAPE, "[moe_layer] B out of range.");
  ZMOE_REQUIRE(d->hidden > 0 && d->n_experts > 0 && d->inter > 0, ZMOE_EINVAL_SHAPE, "[moe_layer] sizes must be positive.");
  ZMOE_REQUIRE(d->top_k >= 1 && d->top_k <= 16 && d->top_k <= d->n_experts && d->n_experts <= 1024,
               ZMOE_EINVAL_SHAPE, "[moe_layer] need 1 <= top_k <= min(16, E) and E <= 1024.");
  ZMOE_REQUIRE(d->hidden % 256 == 0 && d->inter % 256 == 0, ZMOE_EINVAL_SHAPE,
               "[moe_layer] hidden and inter must be multiples of 256.");
  ZMOE_REQUIRE(d->shared_inter >= 0 && d->shared_inter % 256 == 0, ZMOE_EINVAL_SHAPE,
               "[moe_layer] shared_inter must be a multiple of 256.");
  ZMOE_REQUIRE(d->router_kind >= ZMOE_ROUTER_SOFTMAX_PROBS && d->router_kind <= ZMOE_ROUTER_SIGMOID_GROUPED,
               ZMOE_EINVAL_SHAPE, "[moe_layer] unknown router kind.");
  ZMOE_REQUIRE(d->combine_mode >= ZMOE_COMBINE_NATIVE && d->combine_mode <= ZMOE_COMBINE_NO_FMA, ZMOE_EINVAL_SHAPE,
               "[moe_layer] unknown combine mode.");
  ZMOE_REQUIRE(!(d->router_kind == ZMOE_ROUTER_SIGMOID_GROUPED && d->combine_mode == ZMOE_COMBINE_NATIVE),
               ZMOE_EINVAL_DTYPE, "[moe_layer] the sigmoid router yields f32 weights: use an fp32 combine mode.");
  if (d->router_kind == ZMOE_ROUTER_SIGMOID_GROUPED) {
    ZMOE_REQUIRE(d->n_group >= 1 && d->n_group <= 64 && d->n_experts % d->n_group == 0 && d->topk_group >= 1 &&
                     d->topk_group <= d->n_group,
                 ZMOE_EINVAL_SHAPE, "[moe_layer] invalid n_group / topk_group.");
    ZMOE_REQUIRE(d->router_bias != nullptr, ZMOE_EINVAL_SHAPE, "[moe_layer] sigmoid router needs a bias.");
  }
  ZMOE_REQUIRE(d->router_w && d->gate_w && d->up_w && d->down_w && d->gate_s && d->up_s && d->down_s,
               ZMOE_EINVAL_SHAPE, "[moe_layer] null weight pointer.");
  return ZMOE_OK;
}

}  // namespace zmoe

using namespace zmoe;

// Layer path selection: the fused single-launch kernel when it supports the
// shape (decode batches), else the multi-kernel sequence.  ZMOE_LAYER_PATH=
// "multi" forces the sequence (used by tests to compare the two paths).
static bool use_fused(const zmoe_layer_desc* d, int B) {
  static int forced = -1;
  if (forced < 0) {
    const char* e = getenv("ZMOE_LAYER_PATH");
    forced = (e && std::string(e) == "multi") ? 0 : 1;
  }
  return forced == 1 && !(d->flags & ZMOE_LAYER_FORCE_MULTI) && fused_supported(d, B);
}

// The kernel sequence's buffers start after the single-launch kernel's (so
// that data it leaves behind can never be mistaken for tagged data).
static size_t multi_ws_offset(const zmoe_layer_desc* d, int B) {
  const size_t fused = fused_supported(d, B) ? fused_workspace_bytes(d, B) : kSyncBlockBytes;
  return (fused + 255) & ~static_cast<size_t>(255);
}

extern "C" size_t zmoe_moe_layer_workspace_size(const zmoe_layer_desc* desc, int B) {
  if (!desc || B < 0) return 0;
  return multi_ws_offset(desc, B) + layout_ws(desc, B, nullptr).bytes;
}

extern "C" size_t zmoe_moe_layer_trace_info(const zmoe_layer_desc* desc, int B, int* n_blocks, int* n_slots) {
  if (!desc || !n_blocks || !n_slots || !fused_supported(desc, B)) return 0;
  return fused_trace_info(desc, B, n_blocks, n_slots);
}

static int run_sequence(void* stream, const zmoe_layer_desc* d, const void* x, int B, void* out, uint32_t* out_idx,
                        float* out_w, char* ws_base, bool side_ok);

extern "C" int zmoe_moe_layer(void* stream, const zmoe_layer_desc* d, const void* x, int B, void* out,
                              uint32_t* out_idx, float* out_w, void* workspace, size_t workspace_bytes) {
  int rc = validate_layer(d, B);
  if (rc) return rc;
  if (B == 0) return ZMOE_OK;
  const size_t need = zmoe_moe_layer_workspace_size(d, B);
  ZMOE_REQUIRE(workspace != nullptr && workspace_bytes >= need, ZMOE_EINVAL_SHAPE,
               "[moe_layer] workspace too small (need " + std::to_string(need) + " bytes).");
  if (use_fused(d, B)) {
    return launch_fused(as_stream(stream), d, x, B, out, out_idx, out_w, workspace);
  }
  ZMOE_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, ZMOE_EINVAL_SHAPE,
               "[moe_layer] x must be 16-byte and workspace 256-byte aligned.");
  // multi-kernel sequence: its buffers follow the single-launch kernel's
  return run_sequence(stream, d, x, B, out, out_idx, out_w, static_cast<char*>(workspace) + multi_ws_offset(d, B),
                      true);
}

// The shared expert (a dense SwiGLU MLP on every token): gate/up + SwiGLU,
// then down, into sh_y.  From 32 tokens as one "pair" of B token rows (each
// workgroup reads the shared weights once for 4 rows; DeepSeek-V3 B=64 1511
// -> 1500 us); smaller batches as B one-row pairs (more workgroups; GLM-shape
// B=8 71 us vs 79 us).  The per-token arithmetic is the same either way.
static int run_shared(void* stream, const zmoe_layer_desc* d, const void* x, int B, int gshift, void* sh_act,
                      void* sh_y) {
  const int H = d->hidden, Is = d->shared_inter;
  const bool rows = B >= 32;
  const int64_t np = rows ? 1 : B;
  const int M = rows ? B : 1;
  int rc = dispatch_qmv(true, stream, x, d->sh_gate_w, d->sh_gate_s, d->sh_gate_b, d->sh_up_w, d->sh_up_s,
                        d->sh_up_b, nullptr, nullptr, 1, np, M, Is, H, d->quant_mode, gshift, sh_act);
  if (rc) return rc;
  return dispatch_qmv(false, stream, sh_act, d->sh_down_w, d->sh_down_s, d->sh_down_b, nullptr, nullptr, nullptr,
                      nullptr, nullptr, 1, np, M, H, Is, d->quant_mode, gshift, sh_y);
}

// A second stream per device for the shared expert of the kernel sequence
// (created once, default priority), with the fork and join events.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kSideMaxDevices = 64;
static SideStream g_side[kSideMaxDevices];
static std::mutex g_side_mu;

static bool side_stream_enabled() {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("ZMOE_SHARED_STREAM");
    on = (e && e[0] == '0') ? 0 : 1;
  }
  return on == 1;
}

static int side_stream(SideStream** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  ZMOE_REQUIRE(e == hipSuccess && dev >= 0 && dev < kSideMaxDevices, ZMOE_EHIP, "[moe_layer] hipGetDevice failed.");
  SideStream& ss = g_side[dev];
  if (ss.s == nullptr) {
    hipStream_t s = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&f, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&j, hipEventDisableTiming);
    ZMOE_REQUIRE(e == hipSuccess, ZMOE_EHIP, std::string("[moe_layer] side stream: ") + hipGetErrorString(e));
    ss.fork = f;
    ss.join = j;
    ss.s = s;
  }
  *out = &ss;
  return ZMOE_OK;
}

// The multi-kernel sequence over workspace buffers at ws_base (layout_ws);
// keeps nothing from call to call.  With side_ok, a layer's shared expert
// (it reads only x) runs on a second stream of the library's while the
// router and the routed experts run on the caller's stream; the combine waits
// for both (an event fork and join, which a HIP graph capture records as
// parallel branches).
static int run_sequence(void* stream, const zmoe_layer_desc* d, const void* x, int B, void* out, uint32_t* out_idx,
                        float* out_w, char* ws_base, bool side_ok) {
  int rc = ZMOE_OK;
  LayerWs ws = layout_ws(d, B, ws_base);
  ZMOE_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(ws_base) & 255) == 0,
               ZMOE_EINVAL_SHAPE, "[moe_layer] x must be 16-byte and workspace 256-byte aligned.");
  hipStream_t st = as_stream(stream);
  const int H = d->hidden, E = d->n_experts, K = d->top_k, I = d->inter;
  int gshift = 0;
  if (d->quant_mode == ZMOE_Q_AFFINE) {
    ZMOE_REQUIRE(d->group_size == 32 || d->group_size == 64 || d->group_size == 128, ZMOE_EUNSUPPORTED,
                 "[moe_layer] group_size must be 32, 64 or 128.");
    for (int v = d->group_size / 32; v > 1; v >>= 1) ++gshift;
  } else {
    ZMOE_REQUIRE(d->quant_mode == ZMOE_Q_MXFP4 && d->group_size == 32, ZMOE_EUNSUPPORTED,
                 "[moe_layer] unsupported quantization.");
  }
  ZMOE_REQUIRE(d->bits == 4, ZMOE_EUNSUPPORTED, "[moe_layer] only 4-bit weights.");

  const SeqMode mode = seq_mode(d, B);
  // 0. the shared expert, on the side stream when allowed
  const void* shared = nullptr;
  SideStream* side = nullptr;
  std::unique_lock<std::mutex> side_lock(g_side_mu, std::defer_lock);
  if (d->shared_inter > 0) {
    if (side_ok && side_stream_enabled()) {
      side_lock.lock();
      rc = side_stream(&side);
      if (rc) return rc;
      hipError_t e = hipEventRecord(side->fork, st);
      if (e == hipSuccess) e = hipStreamWaitEvent(side->s, side->fork, 0);
      ZMOE_REQUIRE(e == hipSuccess, ZMOE_EHIP, std::string("[moe_layer] side stream fork: ") + hipGetErrorString(e));
    }
    rc = run_shared(side ? static_cast<void*>(side->s) : stream, d, x, B, gshift, ws.sh_act, ws.sh_y);
    if (rc) return rc;
    shared = ws.sh_y;
    if (side) {
      hipError_t e = hipEventRecord(side->join, side->s);
      ZMOE_REQUIRE(e == hipSuccess, ZMOE_EHIP, std::string("[moe_layer] side stream join: ") + hipGetErrorString(e));
    }
  }
  // 1. router projection (bf16 logits, as the gate nn.Linear returns them)
  // (prefill batches on MFMA; decode batches keep the chunk order that the
  // single-launch kernels reproduce).  At hidden 2048 the MFMA router also
  // writes the grouped GEMM's x group sums.
  const bool mfma_router = use_grouped(d, B) && H % 2048 == 0;
  const bool xsum_fused = mfma_router && mode == kSeqMfma && d->quant_mode == ZMOE_Q_AFFINE && H == 2048;
  rc = mfma_router ? launch_logits_mfma(st, x, d->router_w, B, E, H, ZMOE_DT_BF16, ws.logits,
                                        xsum_fused ? ws.xsum : nullptr, d->group_size)
                   : zmoe_dense_logits(stream, x, d->router_w, B, E, H, ZMOE_DT_BF16, ws.logits);
  if (rc) return rc;
  // 2. gating
  int w_dtype = ZMOE_DT_BF16;
  if (d->router_kind == ZMOE_ROUTER_SOFTMAX_PROBS) {
    rc = zmoe_router_softmax_topk(stream, ws.logits, B, E, K, d->norm_topk_prob, ws.w, ws.idx);
  } else if (d->router_kind == ZMOE_ROUTER_TOPK_LOGITS) {
    rc = launch_topk_gating(st, ws.logits, ZMOE_DT_BF16, B, E, K, d->router_bias, d->norm_topk_prob, 1, ws.w, ws.idx);
  } else {
    w_dtype = ZMOE_DT_F32;
    rc = launch_deepseek_router(st, ws.logits, ZMOE_DT_BF16, d->router_bias, B, E, K, d->n_group, d->topk_group,
                                d->routed_scaling_factor, static_cast<float*>(ws.w), ws.idx);
  }
  if (rc) return rc;
  // 3. routed experts: gate/up + SwiGLU, then down
  if (mode == kSeqGemv) {
    // expert-major GEMV over the pairs sorted by expert; act and y stay in
    // pair order
    const int npairs = B * K;
    rc = launch_sort_pairs(st, ws.idx, npairs, E, ws.offsets, ws.sorted, ws.blocks, kGroupedGemvRows);
    if (rc) return rc;
    GroupedArgs g{};
    g.a = static_cast<const uint16_t*>(x);
    g.lda = H;
    g.offsets = ws.offsets;
    g.blocks = ws.blocks;
    g.E = E;
    g.sorted = ws.sorted;
    g.a_div = K;  // pair (b, k) reads token b
    g.scatter = 1;
    g.M = npairs;
    g.w0 = d->gate_w;
    g.s0 = d->gate_s;
    g.b0 = d->gate_b;
    g.w1 = d->up_w;
    g.s1 = d->up_s;
    g.b1 = d->up_b;
    g.N = I;
    g.K = H;
    g.gs = d->group_size;
    g.out = static_cast<uint16_t*>(ws.act);
    g.ldo = I;
    rc = launch_grouped_qmv(st, g, E, d->quant_mode, true);
    if (rc) return rc;
    g.a = static_cast<const uint16_t*>(ws.act);
    g.lda = I;
    g.a_div = 1;  // pair p reads act row p
    g.w0 = d->down_w;
    g.s0 = d->down_s;
    g.b0 = d->down_b;
    g.w1 = nullptr;
    g.s1 = nullptr;
    g.b1 = nullptr;
    g.N = H;
    g.K = I;
    g.out = static_cast<uint16_t*>(ws.y);
    g.ldo = H;
    rc = launch_grouped_qmv(st, g, E, d->quant_mode, false);
    if (rc) return rc;
  } else if (mode == kSeqMfma) {
    // grouped GEMMs on MFMA over the (token, k) pairs sorted by expert; act
    // and y stay in pair order
    const int npairs = B * K;
    const bool affine = d->quant_mode == ZMOE_Q_AFFINE;
    rc = launch_sort_pairs(st, ws.idx, npairs, E, ws.offsets, ws.sorted, ws.blocks);
    if (rc) return rc;
    if (affine && !xsum_fused) {
      rc = launch_row_group_sums(st, static_cast<const uint16_t*>(x), H, B, H, d->group_size, ws.xsum);
      if (rc) return rc;
    }
    GroupedArgs g{};
    g.a = static_cast<const uint16_t*>(x);
    g.lda = H;
    g.asum = ws.xsum;
    g.offsets = ws.offsets;
    g.blocks = ws.blocks;
    g.E = E;
    g.sorted = ws.sorted;
    g.lhs = nullptr;
    g.a_div = K;  // pair (b, k) reads token b
    g.scatter = 1;
    g.M = npairs;
    g.w0 = d->gate_w;
    g.s0 = d->gate_s;
    g.b0 = d->gate_b;
    g.w1 = d->up_w;
    g.s1 = d->up_s;
    g.b1 = d->up_b;
    g.N = I;
    g.K = H;
    g.gs = d->group_size;
    g.out = static_cast<uint16_t*>(ws.act);
    g.ldo = I;
    g.asum_out = affine ? ws.asum : nullptr;  // the act group sums of the down projection, from the epilogue
    rc = launch_grouped(st, g, E, d->quant_mode, true);
    if (rc) return rc;
    g.asum_out = nullptr;
    g.a = static_cast<const uint16_t*>(ws.act);
    g.lda = I;
    g.asum = ws.asum;
    g.a_div = 1;  // pair p reads act row p
    g.w0 = d->down_w;
    g.s0 = d->down_s;
    g.b0 = d->down_b;
    g.w1 = nullptr;
    g.s1 = nullptr;
    g.b1 = nullptr;
    g.N = H;
    g.K = I;
    g.out = static_cast<uint16_t*>(ws.y);
    g.ldo = H;
    rc = launch_grouped(st, g, E, d->quant_mode, false);
    if (rc) return rc;
  } else {
    rc = dispatch_qmv(true, stream, x, d->gate_w, d->gate_s, d->gate_b, d->up_w, d->up_s, d->up_b, nullptr, ws.idx, K,
                      static_cast<int64_t>(B) * K, 1, I, H, d->quant_mode, gshift, ws.act);
    if (rc) return rc;
    rc = dispatch_qmv(false, stream, ws.act, d->down_w, d->down_s, d->down_b, nullptr, nullptr, nullptr, nullptr,
                      ws.idx, 1, static_cast<int64_t>(B) * K, 1, H, I, d->quant_mode, gshift, ws.y);
    if (rc) return rc;
  }
  // 4. the shared expert's result (step 0) is joined before the combine
  if (side) {
    const hipError_t e = hipStreamWaitEvent(st, side->join, 0);
    ZMOE_REQUIRE(e == hipSuccess, ZMOE_EHIP, std::string("[moe_layer] side stream join: ") + hipGetErrorString(e));
    side_lock.unlock();
  }
  // 5. combine (+ shared) -> bf16
  rc = launch_combine(st, ws.y, ws.w, w_dtype, B, K, H, d->combine_mode, 1, shared, out);
  if (rc) return rc;
  if (out_idx) {
    hipError_t e = hipMemcpyAsync(out_idx, ws.idx, static_cast<size_t>(B) * K * 4, hipMemcpyDeviceToDevice, st);
    ZMOE_REQUIRE(e == hipSuccess, ZMOE_EHIP, std::string("[moe_layer] copy failed: ") + hipGetErrorString(e));
  }
  if (out_w) {
    const int n = B * K;
    hipLaunchKernelGGL(k_weights_to_f32, dim3((n + 255) / 256), dim3(256), 0, st, ws.w, w_dtype == ZMOE_DT_F32, n,
                       out_w);
    rc = check_launch("moe_layer");
    if (rc) return rc;
  }
  return ZMOE_OK;
}

// ---------------------------------------------------------------------------
// The layer without a caller workspace, for callers that cannot allocate
// ---------------------------------------------------------------------------
// The kernel sequence's buffers live in `scratch`, a file-scope device array
// of kNoAllocScratchBytes that every GPU the library runs on holds until the
// process ends.  Host code never passes `scratch` itself to a kernel: on the
// host the name is a stand-in, not a device address.  The device address is
// taken once per device with hipGetSymbolAddress, with that device current,
// and kept in g_scratch_ptr.  The sequence keeps nothing from call to call
// and writes every buffer before reading it, so nothing needs clearing; calls
// that overlap on one GPU (two streams, or two host threads) share the array
// and race.
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static char* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_ptr(char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  ZMOE_REQUIRE(e == hipSuccess, ZMOE_EHIP, std::string("[moe_layer_noalloc] hipGetDevice failed: ") + hipGetErrorString(e));
  ZMOE_REQUIRE(dev >= 0 && dev < kMaxDevices, ZMOE_EUNSUPPORTED, "[moe_layer_noalloc] device index out of range.");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    ZMOE_REQUIRE(e == hipSuccess && p != nullptr, ZMOE_EHIP,
                 std::string("[moe_layer_noalloc] hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return ZMOE_OK;
}

extern "C" size_t zmoe_moe_layer_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int zmoe_moe_layer_noalloc(void* stream, const zmoe_layer_desc* d, const void* x, int B, void* out,
                                      uint32_t* out_idx, float* out_w) {
  int rc = validate_layer(d, B);
  if (rc) return rc;
  if (B == 0) return ZMOE_OK;
  const size_t need = layout_ws(d, B, nullptr).bytes;
  ZMOE_REQUIRE(need <= kNoAllocScratchBytes, ZMOE_EINVAL_SHAPE,
               "[moe_layer_noalloc] this batch needs " + std::to_string(need) + " bytes of scratch; the maximum is " +
                   std::to_string(kNoAllocScratchBytes) + " (use zmoe_moe_layer with a workspace).");
  char* base = nullptr;
  rc = scratch_ptr(&base);
  if (rc) return rc;
  return run_sequence(stream, d, x, B, out, out_idx, out_w, base, false);
}
