"""One quantized MoE block over device-resident weights.

``QuantizedMoELayer`` is the unit that ``patch(model)`` installs in place of a
``Qwen3MoeSparseMoeBlock`` / LFM2 / GLM / DeepSeek MoE block (the patched
``__call__`` of ``moe_mlp.py:883-1063`` plus ``deepseek_router.py:76-120``).
Its forward is one call of ``zmoe_moe_layer``: router projection, gating,
gate/up + SwiGLU, down projection, combine and the optional shared expert,
all on the current torch stream, intermediates in a cached workspace.

Family conventions (router kind, combine mode) follow the reference's
unpatched evaluation of each family:

  qwen3     softmax(precise) -> bf16 probs -> top-k -> /sum ; native combine
  lfm2      top-k logits -> softmax over k (f32) -> bf16 weights ; native combine
  glm       sigmoid + e_score_correction_bias top-k -> f32 weights ;
            fp32 no-FMA combine -> bf16 (+ shared expert)
  deepseek  grouped sigmoid top-k x routed_scaling_factor ; fp32 no-FMA
            combine -> bf16 (+ shared expert)
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _native as N

ROUTERS = {
    "softmax_probs": N.ROUTER_SOFTMAX_PROBS,
    "topk_logits": N.ROUTER_TOPK_LOGITS,
    "sigmoid_grouped": N.ROUTER_SIGMOID_GROUPED,
}
COMBINES = {
    "native": N.COMBINE_NATIVE,
    "fp32": N.COMBINE_FP32,
    "fp32_no_fma": N.COMBINE_FP32_NO_FMA,
    "exact": N.COMBINE_EXACT,
    "float": N.COMBINE_FLOAT,
    "no_fma": N.COMBINE_NO_FMA,
}
FAMILIES = {
    "qwen3": ("softmax_probs", "native"),
    "lfm2": ("topk_logits", "native"),
    "glm": ("sigmoid_grouped", "fp32_no_fma"),
    "deepseek": ("sigmoid_grouped", "fp32_no_fma"),
}


@dataclass
class QuantProj:
    """A stacked quantized projection in MLX layout."""

    weight: torch.Tensor                 # uint32 [E, N, K/8] (or [N, K/8] for a dense expert)
    scales: torch.Tensor                 # bf16 [.., N, K/gs] or uint8 e8m0 [.., N, K/32]
    biases: torch.Tensor | None = None   # bf16, affine only


class QuantizedMoELayer:
    """Whole MoE block forward on the MI355X kernels.

    Args mirror the MoE block attributes the reference reads: ``top_k``
    (num_experts_per_tok), ``norm_topk_prob``, ``n_group``/``topk_group``/
    ``routed_scaling_factor`` (DeepSeek gate), expert bias
    (``expert_bias`` / ``e_score_correction_bias``).  ``single_launch=False``
    forces the multi-kernel sequence (the single persistent kernel is used
    for decode batches whenever it applies).

    The single-launch kernels run one workgroup per CU and exchange data
    between workgroups inside the launch, so they assume that all of their
    workgroups are resident at once: run the layer on one stream, with no
    other kernel occupying CUs of the GPU at the same time.  If that fails, a
    wait gives up (after a bounded number of polls), the affected outputs are
    NaN and the next call raises ``ZmoeError`` (``sync_error()`` reads the
    sticky error word directly)."""

    def __init__(
        self,
        router_weight: torch.Tensor,
        gate: QuantProj,
        up: QuantProj,
        down: QuantProj,
        *,
        top_k: int,
        router: str = "softmax_probs",
        combine: str = "native",
        norm_topk_prob: bool = True,
        router_bias: torch.Tensor | None = None,
        n_group: int = 1,
        topk_group: int = 1,
        routed_scaling_factor: float = 1.0,
        group_size: int = 64,
        bits: int = 4,
        mode: str = "affine",
        shared: tuple[QuantProj, QuantProj, QuantProj] | None = None,
        single_launch: bool = True,
        trace: bool = False,
    ) -> None:
        if router not in ROUTERS:
            raise ValueError(f"unknown router kind {router!r}")
        if combine not in COMBINES:
            raise ValueError(f"unknown combine mode {combine!r}")
        self.device = router_weight.device
        if self.device.type != "cuda":
            raise ValueError("QuantizedMoELayer: weights must be device (GPU) tensors")
        for p in (gate, up, down) + (tuple(shared) if shared is not None else ()):
            for t in (p.weight, p.scales, p.biases):
                if t is not None and t.device != self.device:
                    raise ValueError("QuantizedMoELayer: all weights must be on the router weight's device")
        E, H = (int(s) for s in router_weight.shape)
        self.hidden, self.n_experts, self.top_k = H, E, int(top_k)
        self.inter = int(gate.weight.shape[-2])
        self.router, self.combine = router, combine
        self._keep = []  # tensors whose pointers live in the descriptor

        def keep(t):
            if t is None:
                return None
            t = t.contiguous()
            self._keep.append(t)
            return t.data_ptr()

        d = N.LayerDesc()
        d.hidden, d.n_experts, d.top_k, d.inter = H, E, self.top_k, self.inter
        d.group_size, d.bits = int(group_size), int(bits)
        d.quant_mode = N.Q_AFFINE if mode == "affine" else N.Q_MXFP4
        d.router_kind = ROUTERS[router]
        d.norm_topk_prob = int(bool(norm_topk_prob))
        d.n_group, d.topk_group = int(n_group), int(topk_group)
        d.routed_scaling_factor = float(routed_scaling_factor)
        d.combine_mode = COMBINES[combine]
        self._router_w = router_weight.to(torch.bfloat16).contiguous()
        d.router_w = keep(self._router_w)
        d.router_bias = keep(None if router_bias is None else router_bias.to(torch.float32))
        self._proj = {}
        for name, p in (("gate", gate), ("up", up), ("down", down)):
            self._proj[name] = tuple(None if t is None else t.contiguous() for t in (p.weight, p.scales, p.biases))
            setattr(d, f"{name}_w", keep(self._proj[name][0]))
            setattr(d, f"{name}_s", keep(self._proj[name][1]))
            setattr(d, f"{name}_b", keep(self._proj[name][2]))
        d.shared_inter = 0
        if shared is not None:
            sg, su, sd = shared
            d.shared_inter = int(sg.weight.shape[-2])
            for name, p in (("sh_gate", sg), ("sh_up", su), ("sh_down", sd)):
                setattr(d, f"{name}_w", keep(p.weight))
                setattr(d, f"{name}_s", keep(p.scales))
                setattr(d, f"{name}_b", keep(p.biases))
        d.flags = (0 if single_launch else N.LAYER_FORCE_MULTI) | (N.LAYER_TRACE if trace else 0)
        # host-visible flag the single-launch kernels set when a wait for
        # exchanged data gives up (their outputs are then NaN); checked at the
        # next call without a synchronisation
        self._lib = N.lib()  # fail loudly now if the library is missing
        self._err_ptr = self._lib.zmoe_host_flags_alloc(1)
        if not self._err_ptr:
            raise N.ZmoeError("moe_layer: could not allocate the host-visible error flag")
        self._err_flag = ctypes.cast(self._err_ptr, ctypes.POINTER(ctypes.c_uint))
        d.error_flag_host = self._err_ptr
        d.spin_limit = 0
        self.desc = d
        self._ws: dict[int, torch.Tensor] = {}
        self._scratch: torch.Tensor | None = None

    def __del__(self):
        ptr, lib = getattr(self, "_err_ptr", None), getattr(self, "_lib", None)
        if ptr and lib is not None:
            lib.zmoe_host_flags_free(ptr)
            self._err_ptr = None

    @classmethod
    def for_family(cls, family: str, *args, **kwargs) -> QuantizedMoELayer:
        router, combine = FAMILIES[family]
        kwargs.setdefault("router", router)
        kwargs.setdefault("combine", combine)
        return cls(*args, **kwargs)

    def workspace_bytes(self, B: int) -> int:
        return int(N.lib().zmoe_moe_layer_workspace_size(ctypes.byref(self.desc), int(B)))

    def _single_launch(self, B: int) -> bool:
        """Whether batch B runs a single-launch kernel (whose workspace keeps
        launch counts from call to call)."""
        nb, ns = ctypes.c_int(0), ctypes.c_int(0)
        return int(N.lib().zmoe_moe_layer_trace_info(ctypes.byref(self.desc), int(B), ctypes.byref(nb),
                                                          ctypes.byref(ns))) != 0

    def _workspace(self, B: int) -> torch.Tensor:
        """Single-launch batches (at most 16 sizes) keep one zero-filled
        workspace each: it holds launch counts that only grow from call to
        call.  Every other batch shares one scratch buffer that grows to the
        largest batch seen (the kernel sequence keeps nothing across calls)."""
        ws = self._ws.get(B)
        if ws is not None:
            return ws
        need = self.workspace_bytes(B)
        if self._single_launch(B):
            ws = torch.zeros(need, dtype=torch.uint8, device=self.device)
            self._ws[B] = ws
            return ws
        if self._scratch is None or self._scratch.numel() < need:
            self._scratch = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self._scratch

    def _check_previous_call(self) -> None:
        if self._err_flag[0] != 0:
            self._err_flag[0] = 0
            for ws in self._ws.values():  # launch counts restart from zero
                ws.zero_()
            raise N.ZmoeError(
                "moe_layer: a wait for data exchanged between workgroups gave up in an earlier call "
                "(another kernel occupying CUs of this GPU?); that call's outputs are NaN where affected")

    def __call__(self, x: torch.Tensor, *, return_routing: bool = False):
        if x.dtype != torch.bfloat16:
            raise ValueError("QuantizedMoELayer: x must be bfloat16")
        if x.device != self.device:
            raise ValueError("QuantizedMoELayer: x must be on the layer's device")
        shape = x.shape
        xc = x.contiguous().reshape(-1, self.hidden)
        B = int(xc.shape[0])
        out = torch.empty_like(xc)
        idx = w = None
        if return_routing:
            idx = torch.empty((B, self.top_k), dtype=torch.int32, device=self.device)
            w = torch.empty((B, self.top_k), dtype=torch.float32, device=self.device)
        self._check_previous_call()
        ws = self._workspace(B)
        rc = N.lib().zmoe_moe_layer(
            torch.cuda.current_stream(self.device).cuda_stream, ctypes.byref(self.desc), xc.data_ptr(), B,
            out.data_ptr(), None if idx is None else idx.data_ptr(), None if w is None else w.data_ptr(),
            ws.data_ptr(), ws.numel(),
        )
        N.check(rc, "moe_layer")
        out = out.reshape(shape)
        if return_routing:
            return out, idx.reshape(*shape[:-1], self.top_k), w.reshape(*shape[:-1], self.top_k)
        return out

    forward = __call__

    def phase_trace(self, B: int):
        """Per-workgroup phase timestamps of the last single-launch call at
        batch B (requires ``trace=True``): int64 tensor [blocks, slots] of
        100 MHz realtime-counter values, or None."""
        nb, ns = ctypes.c_int(0), ctypes.c_int(0)
        off = int(N.lib().zmoe_moe_layer_trace_info(ctypes.byref(self.desc), int(B), ctypes.byref(nb),
                                                        ctypes.byref(ns)))
        ws = self._ws.get(B)
        if off == 0 or ws is None:
            return None
        n = nb.value * ns.value
        return ws[off: off + 8 * n].view(torch.int64).reshape(nb.value, ns.value).clone()

    def sync_error(self) -> int:
        """Sticky error word of the single-launch kernels' cross-workgroup
        waits, over every workspace (0 = ok).  Synchronises."""
        flags = 0
        for ws in self._ws.values():
            flags |= int(ws[128:132].view(torch.int32).item())
        return flags
