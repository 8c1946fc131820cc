"""patch(model): swap a torch model's MoE blocks for the MI355X layer.

The model-level drop-in boundary of the reference (``src/zmlx/patch``):
patterns with ``name``, ``matches(module, name, parent)`` and
``apply(module, config)`` (the ``PatchPattern`` protocol,
``_types.py:39-51``), a walk over every submodule that asks each pattern
(``_walk_modules``, ``_traversal.py:10-81``), and replacement by class swap
with the original kept on the module (``module._zmlx_original_call``), so
``unpatch`` restores it.

Patterns (torch / transformers module layouts):

``moe_mlp``
    softmax top-k blocks (Qwen3-MoE, Mixtral; ``moe_mlp.py:226-266``): a
    router ``gate.weight [E, H]`` with ``top_k``/``norm_topk_prob`` and experts
    stacked as ``gate_up_proj [E, 2I, H]`` + ``down_proj [E, H, I]`` (or a
    ``ModuleList`` of ``gate_proj``/``up_proj``/``down_proj`` MLPs).  Gating
    follows the reference's Qwen branch: precise softmax, probabilities
    rounded to bf16, top-k, renormalised in bf16; native bf16 combine.
``deepseek_router``
    sigmoid + correction-bias grouped routers with routed scaling and shared
    experts (DeepSeek-V3, GLM-4-MoE; ``deepseek_router.py:76-120``,
    ``moe_mlp.py:995-1002, 1059-1061``): fp32 no-FMA combine, shared expert
    added after it.

Expert weights are quantised to MLX's affine 4-bit layout (group 64 by
default) or mxfp4 when patched; an MLX-format checkpoint that is already
quantised (mlx_lm ``switch_mlp`` tensors) loads without requantising through
``read_mlx_moe_tensors`` / ``layer_from_mlx``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Iterable

import torch

from .layer import QuantizedMoELayer, QuantProj
from .quant import quantize_affine, quantize_mxfp4

__all__ = [
    "PatchConfig",
    "PatchPattern",
    "MoEMLPPattern",
    "DeepSeekRouterPattern",
    "PatchResult",
    "register",
    "get_pattern",
    "list_patterns",
    "patch",
    "unpatch",
    "find_moe_blocks",
    "read_mlx_moe_tensors",
    "layer_from_mlx",
]


@dataclass
class PatchConfig:
    """Options of a patch run (the reference's ``PatchConfig`` fields that
    apply to this path)."""

    group_size: int = 64
    bits: int = 4
    mode: str = "affine"          # "affine" or "mxfp4"
    device: torch.device | None = None
    verbose: bool = False


class PatchPattern:
    """One kind of module the walker can replace."""

    name = "base"

    def matches(self, module: torch.nn.Module, name: str, parent: torch.nn.Module | None) -> bool:
        raise NotImplementedError

    def apply(self, module: torch.nn.Module, config: PatchConfig) -> torch.nn.Module:
        raise NotImplementedError


# ---------------------------------------------------------------------------
# weight access
# ---------------------------------------------------------------------------
def _expert_mats(experts: torch.nn.Module):
    """(gate [E, I, H], up [E, I, H], down [E, H, I]) of a stacked or
    ModuleList expert set, or None."""
    if hasattr(experts, "gate_up_proj") and hasattr(experts, "down_proj"):
        gu = experts.gate_up_proj
        dn = experts.down_proj
        if not (isinstance(gu, torch.Tensor) and isinstance(dn, torch.Tensor)) or gu.dim() != 3 or dn.dim() != 3:
            return None
        inter = gu.shape[1] // 2
        return gu[:, :inter, :], gu[:, inter:, :], dn
    if isinstance(experts, torch.nn.ModuleList) and len(experts) > 0:
        e0 = experts[0]
        names = (("gate_proj", "up_proj", "down_proj"), ("w1", "w3", "w2"))
        for g, u, d in names:
            if all(hasattr(e0, a) for a in (g, u, d)):
                return (torch.stack([getattr(e, g).weight for e in experts]),
                        torch.stack([getattr(e, u).weight for e in experts]),
                        torch.stack([getattr(e, d).weight for e in experts]))
    return None


def _shapes_supported(module) -> bool:
    """The kernels' shape limits: hidden, expert and shared intermediate
    sizes multiples of 256, 1 <= top_k <= min(16, E), E <= 1024.  Blocks
    outside them keep their own forward."""
    mats = _expert_mats(module.experts)
    if mats is None:
        return False
    g, _, _ = mats
    E, inter, hidden = (int(v) for v in g.shape)
    top_k = int(getattr(module.gate, "top_k", getattr(module, "top_k", 0)) or 0)
    if hidden % 256 or inter % 256 or not (1 <= top_k <= min(16, E)) or E > 1024:
        return False
    sh = getattr(module, "shared_experts", None)
    if sh is not None and int(sh.gate_proj.weight.shape[0]) % 256:
        return False
    return True


def _quant(w: torch.Tensor, config: PatchConfig, device) -> QuantProj:
    w = w.detach().to(device=device).contiguous()
    if config.mode == "mxfp4":
        q, s = quantize_mxfp4(w)
        return QuantProj(q, s, None)
    q, s, b = quantize_affine(w, config.group_size)
    return QuantProj(q, s, b)


def _dense_quant(linear: torch.nn.Module, config: PatchConfig, device) -> QuantProj:
    p = _quant(linear.weight[None], config, device)
    return QuantProj(p.weight[0].contiguous(), p.scales[0].contiguous(),
                     None if p.biases is None else p.biases[0].contiguous())


def _patched_forward(self, hidden_states: torch.Tensor, *args, **kwargs):
    shape, dtype = hidden_states.shape, hidden_states.dtype
    x = hidden_states.reshape(-1, shape[-1]).to(torch.bfloat16).contiguous()
    y = self._zmoe_layer(x)
    return y.reshape(shape).to(dtype)


def _swap(module: torch.nn.Module, layer: QuantizedMoELayer, pattern: str) -> torch.nn.Module:
    cls = module.__class__
    module._zmoe_layer = layer
    module._zmlx_original_call = cls
    module._zmlx_pattern = pattern
    module.__class__ = type(f"ZMoE{cls.__name__}", (cls,), {"forward": _patched_forward})
    return module


# ---------------------------------------------------------------------------
# patterns
# ---------------------------------------------------------------------------
class MoEMLPPattern(PatchPattern):
    """Softmax top-k sparse MoE blocks (Qwen3-MoE, Mixtral layouts)."""

    name = "moe_mlp"

    def matches(self, module, name, parent) -> bool:
        gate = getattr(module, "gate", None)
        experts = getattr(module, "experts", None)
        if gate is None or experts is None or getattr(module, "_zmlx_original_call", None) is not None:
            return False
        w = getattr(gate, "weight", None)
        if not isinstance(w, torch.Tensor) or w.dim() != 2:
            return False
        if hasattr(gate, "e_score_correction_bias") or hasattr(module, "shared_experts"):
            return False  # sigmoid routers: deepseek_router
        if hasattr(module, "shared_expert") or hasattr(module, "shared_expert_gate"):
            return False  # Qwen2-MoE: a sigmoid-gated shared expert the routed-only layer would drop
        if getattr(module, "use_expert_bias", False) or hasattr(gate, "routed_scaling_factor"):
            return False  # sigmoid + bias routers this pattern does not cover
        return _shapes_supported(module)

    def apply(self, module, config: PatchConfig):
        dev = config.device or module.gate.weight.device
        g, u, d = _expert_mats(module.experts)
        top_k = int(getattr(module.gate, "top_k", getattr(module, "top_k", 2)))
        norm = bool(getattr(module.gate, "norm_topk_prob", getattr(module, "norm_topk_prob", True)))
        layer = QuantizedMoELayer.for_family(
            "qwen3", module.gate.weight.detach().to(device=dev, dtype=torch.bfloat16),
            _quant(g, config, dev), _quant(u, config, dev), _quant(d, config, dev), top_k=top_k,
            norm_topk_prob=norm, group_size=config.group_size if config.mode == "affine" else 32,
            mode=config.mode)
        return _swap(module, layer, self.name)


class DeepSeekRouterPattern(PatchPattern):
    """Sigmoid + correction-bias grouped routers with shared experts
    (DeepSeek-V3, GLM-4-MoE layouts)."""

    name = "deepseek_router"

    def matches(self, module, name, parent) -> bool:
        gate = getattr(module, "gate", None)
        experts = getattr(module, "experts", None)
        if gate is None or experts is None or getattr(module, "_zmlx_original_call", None) is not None:
            return False
        if not hasattr(gate, "e_score_correction_bias") or not isinstance(getattr(gate, "weight", None), torch.Tensor):
            return False
        if not bool(getattr(gate, "norm_topk_prob", True)):
            return False  # the kernels renormalise the selected sigmoids
        return _shapes_supported(module)

    def apply(self, module, config: PatchConfig):
        gate = module.gate
        dev = config.device or gate.weight.device
        g, u, d = _expert_mats(module.experts)
        shared = None
        sh = getattr(module, "shared_experts", None)
        if sh is not None:
            shared = tuple(_dense_quant(getattr(sh, n), config, dev) for n in ("gate_proj", "up_proj", "down_proj"))
        layer = QuantizedMoELayer.for_family(
            "deepseek", gate.weight.detach().to(device=dev, dtype=torch.bfloat16),
            _quant(g, config, dev), _quant(u, config, dev), _quant(d, config, dev),
            top_k=int(gate.top_k),
            router_bias=gate.e_score_correction_bias.detach().to(device=dev, dtype=torch.float32),
            n_group=int(getattr(gate, "num_group", getattr(gate, "n_group", 1))),
            topk_group=int(getattr(gate, "topk_group", 1)),
            routed_scaling_factor=float(getattr(gate, "routed_scaling_factor", 1.0)),
            group_size=config.group_size if config.mode == "affine" else 32, mode=config.mode, shared=shared)
        return _swap(module, layer, self.name)


_PATTERNS: dict[str, PatchPattern] = {}


def register(pattern: PatchPattern) -> PatchPattern:
    """Adds a pattern to the registry under its name (``_registry.py:8``)."""
    _PATTERNS[pattern.name] = pattern
    return pattern


def get_pattern(name: str) -> PatchPattern:
    """The registered pattern ``name``; KeyError naming the available ones
    otherwise (``_registry.py:14-19``)."""
    if name not in _PATTERNS:
        raise KeyError(f"Unknown patch pattern: {name!r}. Available: {list_patterns()}")
    return _PATTERNS[name]


def list_patterns() -> list[str]:
    return sorted(_PATTERNS)


register(MoEMLPPattern())
register(DeepSeekRouterPattern())

# workload modes and curated profiles (``__init__.py:182-188``): every mode
# selects the MoE patterns, the only ones this library has
_MODES = {"inference": ("moe_mlp", "deepseek_router")}
_PROFILES = {"qwen3": ("moe_mlp",), "qwen3-minimal": ("moe_mlp",), "deepseek": ("deepseek_router",),
             "glm": ("deepseek_router",)}


@dataclass
class PatchResult:
    """What a patch run did (``_types.py:18-36``)."""

    patched_count: int = 0
    pattern_counts: dict = field(default_factory=dict)
    skipped: list = field(default_factory=list)
    patched: list = field(default_factory=list)   # module paths, in walk order

    def summary(self) -> str:
        lines = [f"Patched {self.patched_count} modules:"]
        lines += [f"  {n}: {c}" for n, c in sorted(self.pattern_counts.items())]
        if self.skipped:
            lines.append(f"  Skipped: {len(self.skipped)}")
        return "\n".join(lines)


# ---------------------------------------------------------------------------
# walker
# ---------------------------------------------------------------------------
def _walk(model: torch.nn.Module, fn: Callable[[torch.nn.Module, str, torch.nn.Module | None], None]) -> None:
    """Pre-order walk over every submodule with its parent."""
    def rec(mod, name, parent):
        fn(mod, name, parent)
        for child_name, child in list(mod.named_children()):
            rec(child, f"{name}.{child_name}" if name else child_name, mod)
    rec(model, "", None)


def _select(patterns, exclude, mode, profile) -> list[PatchPattern]:
    """Explicit patterns > profile > mode > default (``__init__.py:196-219``)."""
    if patterns is not None:
        names = list(patterns)
    elif profile is not None:
        if profile not in _PROFILES:
            raise ValueError(f"Unknown profile {profile!r}. Expected one of: {', '.join(sorted(_PROFILES))}")
        names = list(_PROFILES[profile])
    else:
        m = mode or "inference"
        if m not in _MODES:
            raise ValueError(f"Unknown mode {m!r}. Expected one of: {', '.join(_MODES)}")
        names = list(_MODES[m])
    selected = [get_pattern(n) for n in names]
    if exclude:
        selected = [p for p in selected if p.name not in set(exclude)]
    return selected


def find_moe_blocks(model: torch.nn.Module, patterns: Iterable[str] | None = None) -> list[tuple[str, str]]:
    """(module path, pattern name) of every block a pattern would replace;
    the first matching pattern wins, as in ``_traversal.py:52-66``."""
    pats = _select(patterns, None, None, None)
    found = []

    def visit(mod, name, parent):
        for p in pats:
            if p.matches(mod, name, parent):
                found.append((name, p.name))
                break
    _walk(model, visit)
    return found


def patch(model: torch.nn.Module, *, mode: str | None = None, profile: str | None = None,
          patterns: list[str] | None = None, exclude: list[str] | None = None, group_size: int = 64,
          bits: int = 4, quant_mode: str = "affine", device: torch.device | str | None = None,
          verbose: bool = False) -> torch.nn.Module:
    """Replaces every matching MoE block of ``model`` in place and returns the
    model (``__init__.py:129-305``).

    ``mode`` / ``profile`` / ``patterns`` / ``exclude`` select patterns as the
    reference does; ``group_size``, ``bits`` and ``quant_mode`` ("affine" or
    "mxfp4") set how expert weights are quantised.  The blocks' weights must be
    on the GPU (or ``device`` names it).  A block whose ``apply`` fails is left
    as it was and listed in ``PatchResult.skipped``; the result is
    ``model._zmlx_patch_result``."""
    if bits != 4:
        raise ValueError("patch: only 4-bit weights are supported.")
    if quant_mode not in ("affine", "mxfp4"):
        raise ValueError(f"patch: unknown quant_mode {quant_mode!r}.")
    selected = _select(patterns, exclude, mode, profile)
    config = PatchConfig(group_size=group_size, bits=bits, mode=quant_mode,
                         device=None if device is None else torch.device(device), verbose=verbose)
    result = PatchResult()
    if verbose:
        print(f"[zmlx_amd.patch] Applying {len(selected)} patterns: {[p.name for p in selected]}")
    targets = []

    def visit(mod, name, parent):
        for p in selected:
            if p.matches(mod, name, parent):
                targets.append((mod, name, p))
                break
    _walk(model, visit)
    for mod, name, p in targets:
        try:
            p.apply(mod, config)
        except Exception as e:  # the reference records and goes on (_traversal.py:59-60)
            result.skipped.append(f"{name}: {e}")
            continue
        result.patched_count += 1
        result.pattern_counts[p.name] = result.pattern_counts.get(p.name, 0) + 1
        result.patched.append(name)
        if verbose:
            print(f"  [zmlx_amd.patch] {name}: {p.name}")
    if verbose:
        print(result.summary())
    model._zmlx_patch_result = result
    return model


def unpatch(model: torch.nn.Module) -> torch.nn.Module:
    """Restores every block ``patch`` replaced (``__init__.py:308-331``)."""
    def visit(mod, name, parent):
        orig = getattr(mod, "_zmlx_original_call", None)
        if orig is not None:
            mod.__class__ = orig
            for a in ("_zmoe_layer", "_zmlx_original_call", "_zmlx_pattern"):
                if hasattr(mod, a):
                    delattr(mod, a)
    _walk(model, visit)
    if hasattr(model, "_zmlx_patch_result"):
        del model._zmlx_patch_result
    return model


# ---------------------------------------------------------------------------
# MLX-format quantised checkpoints
# ---------------------------------------------------------------------------
_SHARED_NAMES = ("shared_experts", "shared_expert")


def read_mlx_moe_tensors(source, prefix: str) -> dict:
    """Tensors of one mlx_lm MoE block from a local ``.safetensors`` file (or
    a dict of tensors): router ``{prefix}.gate.weight`` (+ optional
    ``e_score_correction_bias``), experts ``{prefix}.switch_mlp.{gate,up,
    down}_proj.{weight,scales,biases}`` (uint32 [E, N, K/8], bf16 or uint8
    scales) and an optional shared expert.  Returns {"router", "bias",
    "gate", "up", "down", "shared"} with QuantProj values (CPU tensors)."""
    if isinstance(source, dict):
        t = source
    else:
        from safetensors.torch import load_file  # safe loader: tensors only

        t = load_file(str(source))

    def get(key, required=True):
        if key in t:
            return t[key]
        if required:
            raise KeyError(f"read_mlx_moe_tensors: missing tensor {key!r}")
        return None

    def proj(base, required=True):
        w = get(f"{base}.weight", required)
        if w is None:
            return None
        if w.dtype != torch.int32 and w.dtype != torch.uint32:
            raise ValueError(f"read_mlx_moe_tensors: {base}.weight is not packed 4-bit (dtype {w.dtype}).")
        return QuantProj(w.view(torch.int32).view(torch.uint32) if w.dtype == torch.int32 else w,
                         get(f"{base}.scales"), get(f"{base}.biases", False))

    out = {
        "router": get(f"{prefix}.gate.weight"),
        "bias": get(f"{prefix}.gate.e_score_correction_bias", False),
        "gate": proj(f"{prefix}.switch_mlp.gate_proj"),
        "up": proj(f"{prefix}.switch_mlp.up_proj"),
        "down": proj(f"{prefix}.switch_mlp.down_proj"),
        "shared": None,
    }
    for sn in _SHARED_NAMES:
        g = proj(f"{prefix}.{sn}.gate_proj", False)
        if g is not None:
            out["shared"] = (g, proj(f"{prefix}.{sn}.up_proj"), proj(f"{prefix}.{sn}.down_proj"))
            break
    return out


def layer_from_mlx(source, prefix: str, family: str, *, top_k: int, device="cuda", group_size: int = 64,
                   mode: str = "affine", **kwargs) -> QuantizedMoELayer:
    """A QuantizedMoELayer over one MoE block of an MLX-format checkpoint
    (already quantised: no requantisation)."""
    t = read_mlx_moe_tensors(source, prefix)
    dev = torch.device(device)

    def mv(p: QuantProj | None):
        if p is None:
            return None
        return QuantProj(p.weight.to(dev), p.scales.to(dev), None if p.biases is None else p.biases.to(dev))

    if t["bias"] is not None and "router_bias" not in kwargs:
        kwargs["router_bias"] = t["bias"].to(device=dev, dtype=torch.float32)
    shared = None if t["shared"] is None else tuple(mv(p) for p in t["shared"])
    return QuantizedMoELayer.for_family(family, t["router"].to(device=dev, dtype=torch.bfloat16), mv(t["gate"]),
                                        mv(t["up"]), mv(t["down"]), top_k=top_k, group_size=group_size, mode=mode,
                                        shared=shared, **kwargs)
