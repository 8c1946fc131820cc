"""patch(model) over transformers MoE blocks and the MLX checkpoint reader.

CPU: which blocks each pattern matches on tiny transformers models (Qwen3-MoE,
Mixtral, DeepSeek-V3, GLM-4-MoE; LFM2-MoE's sigmoid router is left alone),
refusal of host-resident weights, and a safetensors round trip of the mlx_lm
tensor layout.  GPU: a patched block, and a whole patched model, against the
unpatched transformers forward (fp32) whose expert weights are replaced by
the dequantised ones, so the only difference left is the kernels' bf16
arithmetic (2e-2: bf16 rounding of x, activations, gating and output)."""

from __future__ import annotations

import copy

import numpy as np
import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

from zmlx_amd import patch as P  # noqa: E402
from zmlx_amd.quant import dequantize, quantize_affine, quantize_mxfp4  # noqa: E402

H, I, E, K = 512, 256, 16, 4


def _qwen3_model(layers=2):
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(hidden_size=H, intermediate_size=2 * H, moe_intermediate_size=I, num_experts=E,
                         num_experts_per_tok=K, num_hidden_layers=layers, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=64, vocab_size=256, norm_topk_prob=True,
                         decoder_sparse_step=1, mlp_only_layers=[])
    torch.manual_seed(0)
    return Qwen3MoeForCausalLM(cfg).eval()


def _deepseek_block():
    from transformers import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3MoE

    cfg = DeepseekV3Config(hidden_size=H, intermediate_size=2 * H, moe_intermediate_size=I, n_routed_experts=32,
                           num_local_experts=32, num_experts_per_tok=K, n_group=4, topk_group=2,
                           n_shared_experts=1, routed_scaling_factor=2.5, norm_topk_prob=True)
    cfg.num_local_experts = 32
    torch.manual_seed(1)
    return DeepseekV3MoE(cfg).eval()


def _init_block(block, std=0.05):
    """Random weights at realistic scale: router logits of a few units, so the
    bf16 rounding of the logits (the MLX convention) moves the gating weights
    by well under 1%."""
    with torch.no_grad():
        for name, p in block.named_parameters():
            p.normal_(0.0, std)
        if hasattr(block.gate, "e_score_correction_bias"):
            block.gate.e_score_correction_bias.normal_(0.0, 0.05)


def _roundtrip(w, gs, mode):
    if mode == "mxfp4":
        q, s = quantize_mxfp4(w)
        return dequantize(q, s, None, mode="mxfp4")
    q, s, b = quantize_affine(w, gs)
    return dequantize(q, s, b, group_size=gs)


def _dequantise_experts_(block, gs=64, mode="affine"):
    """Replace the block's expert weights by their 4-bit round trip (affine
    or mxfp4) and its router weight by its bf16 rounding (the kernels'
    operands)."""
    with torch.no_grad():
        block.gate.weight.copy_(block.gate.weight.to(torch.bfloat16).float())
        for name in ("gate_up_proj", "down_proj"):
            w = getattr(block.experts, name)
            w.copy_(_roundtrip(w.detach().float(), gs, mode))
        sh = getattr(block, "shared_experts", None)
        if sh is not None:
            for n in ("gate_proj", "up_proj", "down_proj"):
                w = getattr(sh, n).weight
                w.copy_(_roundtrip(w.detach().float(), gs, mode))


# ---------------------------------------------------------------------------
# CPU
# ---------------------------------------------------------------------------
def test_find_blocks_qwen3_model():
    m = _qwen3_model(layers=3)
    found = P.find_moe_blocks(m)
    assert found == [(f"model.layers.{i}.mlp", "moe_mlp") for i in range(3)]
    assert P.find_moe_blocks(m, ["deepseek_router"]) == []


def test_find_blocks_deepseek_and_glm():
    blk = _deepseek_block()
    assert P.find_moe_blocks(blk) == [("", "deepseek_router")]
    from transformers import Glm4MoeConfig
    from transformers.models.glm4_moe.modeling_glm4_moe import Glm4MoeMoE

    g = Glm4MoeMoE(Glm4MoeConfig(hidden_size=H, moe_intermediate_size=I, n_routed_experts=16, num_experts_per_tok=K,
                                 n_group=1, topk_group=1, n_shared_experts=1))
    assert P.find_moe_blocks(g) == [("", "deepseek_router")]


def test_mixtral_matches_lfm2_does_not():
    from transformers import Lfm2MoeConfig, MixtralConfig
    from transformers.models.lfm2_moe.modeling_lfm2_moe import Lfm2MoeSparseMoeBlock
    from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock

    mx = MixtralSparseMoeBlock(MixtralConfig(hidden_size=H, intermediate_size=I, num_local_experts=8,
                                             num_experts_per_tok=2))
    assert P.find_moe_blocks(mx) == [("", "moe_mlp")]
    lf = Lfm2MoeSparseMoeBlock(Lfm2MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=8,
                                             num_experts_per_tok=2))
    assert P.find_moe_blocks(lf) == []
    # shapes outside the kernels' limits (inter not a multiple of 256) stay unpatched
    small = MixtralSparseMoeBlock(MixtralConfig(hidden_size=H, intermediate_size=128, num_local_experts=8,
                                                num_experts_per_tok=2))
    assert P.find_moe_blocks(small) == []


def test_qwen2_moe_gated_shared_expert_not_matched():
    """Qwen2-MoE blocks add a sigmoid-gated shared expert that the routed
    layer does not compute; swapping them would drop that term, so neither
    pattern may take them."""
    from transformers import Qwen2MoeConfig
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeSparseMoeBlock

    blk = Qwen2MoeSparseMoeBlock(Qwen2MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E,
                                                num_experts_per_tok=K, shared_expert_intermediate_size=I))
    assert hasattr(blk, "shared_expert") and hasattr(blk, "shared_expert_gate")
    assert P.find_moe_blocks(blk) == []
    out = P.patch(blk, device=torch.device("cpu"))
    assert out._zmlx_patch_result.patched == [] and blk.__class__ is Qwen2MoeSparseMoeBlock


def test_patch_selection_and_errors():
    m = _qwen3_model(layers=2)
    # host-resident weights: each block's apply fails, is recorded, and the
    # block keeps its own forward (the reference's skipped list)
    P.patch(m)
    r = m._zmlx_patch_result
    assert r.patched_count == 0 and len(r.skipped) == 2
    assert r.skipped[0].startswith("model.layers.0.mlp:") and "device" in r.skipped[0]
    assert type(m.model.layers[0].mlp).__name__ == "Qwen3MoeSparseMoeBlock"
    with pytest.raises(KeyError, match="Unknown patch pattern"):
        P.patch(m, patterns=["nope"])
    with pytest.raises(ValueError, match="Unknown profile"):
        P.patch(m, profile="nope")
    with pytest.raises(ValueError, match="Unknown mode"):
        P.patch(m, mode="training")
    with pytest.raises(ValueError, match="4-bit"):
        P.patch(m, bits=8)
    # exclude removes a pattern from the selection
    P.patch(m, exclude=["moe_mlp"])
    assert m._zmlx_patch_result.patched_count == 0 and m._zmlx_patch_result.skipped == []
    assert P.list_patterns() == ["deepseek_router", "moe_mlp"]
    P.unpatch(m)
    assert not hasattr(m, "_zmlx_patch_result")


def test_read_mlx_tensors_round_trip(tmp_path):
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(3)
    pre = "model.layers.0.mlp"
    t = {f"{pre}.gate.weight": torch.randn(E, H, generator=g).to(torch.bfloat16),
         f"{pre}.gate.e_score_correction_bias": torch.randn(E, generator=g)}
    ref = {}
    for n, shape in (("gate_proj", (E, I, H)), ("up_proj", (E, I, H)), ("down_proj", (E, H, I)),
                     ("sh_gate", (I, H)), ("sh_up", (I, H)), ("sh_down", (H, I))):
        q, s, b = quantize_affine(torch.randn(*shape, generator=g), 64)
        ref[n] = (q, s, b)
        base = f"{pre}.switch_mlp.{n}" if not n.startswith("sh_") else f"{pre}.shared_experts.{n[3:]}_proj"
        t[f"{base}.weight"], t[f"{base}.scales"], t[f"{base}.biases"] = q, s, b
    path = tmp_path / "model.safetensors"
    save_file(t, str(path))
    got = P.read_mlx_moe_tensors(path, pre)
    assert torch.equal(got["router"], t[f"{pre}.gate.weight"])
    assert torch.equal(got["bias"], t[f"{pre}.gate.e_score_correction_bias"])
    for n, key in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
        for a, b_ in zip((got[key].weight, got[key].scales, got[key].biases), ref[n]):
            assert a.dtype == b_.dtype and torch.equal(a, b_)
    for i, n in enumerate(("sh_gate", "sh_up", "sh_down")):
        assert torch.equal(got["shared"][i].weight, ref[n][0])
    # a missing expert tensor names the key
    del t[f"{pre}.switch_mlp.down_proj.scales"]
    with pytest.raises(KeyError, match="down_proj.scales"):
        P.read_mlx_moe_tensors(t, pre)
    # dense (unquantised) expert weights are refused
    t2 = dict(t)
    t2[f"{pre}.switch_mlp.gate_proj.weight"] = torch.zeros(E, I, H, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="packed"):
        P.read_mlx_moe_tensors(t2, pre)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
def _routing_split(blk, ref_blk, x):
    """Rows whose selected expert set agrees between the kernels (softmax
    probabilities rounded to bf16 before top-k, the MLX Qwen convention) and
    transformers (fp32 top-k).  Every row that disagrees must be a bf16 tie at
    the k-th place (within one bf16 ulp); returns the boolean mask of agreeing rows."""
    xf = x.reshape(-1, x.shape[-1])
    _, idx, _ = blk._zmoe_layer(xf.to(torch.bfloat16), return_routing=True)
    _, _, ridx = ref_blk.gate(xf)
    k = idx.shape[-1]
    same = (idx.long().sort(-1).values == ridx.long().sort(-1).values).all(-1)
    if not bool(same.all()):
        # the MLX convention rounds the router logits to bf16 before the
        # softmax, which makes exact ties that the kernels break by index
        lg = (xf.to(torch.bfloat16).float() @ ref_blk.gate.weight.float().t()).to(torch.bfloat16)
        p = torch.softmax(lg.float(), -1).to(torch.bfloat16)
        pv = p.float().sort(-1, descending=True).values
        # one bf16 ulp (2^-7 relative, upper bound): the kernel's exp and
        # torch's differ in the last fp32 bits, which can move a value across
        # a bf16 rounding boundary
        gap = (pv[:, k - 1] - pv[:, k]) / pv[:, k - 1]
        assert bool((gap[~same] <= 2.0 ** -7).all()), f"routing differs beyond a bf16 tie: {gap[~same].tolist()}"
    return same.cpu().numpy()


def _close(got, ref, rows=None):
    got, ref = got.float().cpu().numpy(), ref.float().cpu().numpy()
    if rows is not None:
        got, ref = got.reshape(-1, got.shape[-1])[rows], ref.reshape(-1, ref.shape[-1])[rows]
    # against an fp32 model: the kernels round x, the SwiGLU activations,
    # the gating weights and the output to bf16 (two ulps at |y| ~ 2);
    # bit-level parity with the float64 oracle is in test_gpu_layer
    np.testing.assert_allclose(got, ref, atol=2e-2, rtol=2e-2)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-12)
    assert rel < 2e-2, rel


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 5, 48])
def test_patched_qwen3_block_matches_transformers(dev, B):
    m = _qwen3_model(layers=1)
    blk = m.model.layers[0].mlp
    _init_block(blk)
    blk = blk.to(dev)
    ref_blk = copy.deepcopy(blk)
    _dequantise_experts_(ref_blk)
    P.patch(blk)
    assert type(blk).__name__.startswith("ZMoE")
    g = torch.Generator(device=dev).manual_seed(B)
    x = torch.randn(1, B, H, device=dev, generator=g).to(torch.bfloat16).float()
    with torch.no_grad():
        ref = ref_blk(x)
        got = blk(x)
    torch.cuda.synchronize()
    assert got.shape == x.shape and got.dtype == x.dtype
    rows = _routing_split(blk, ref_blk, x)
    assert rows.mean() >= 0.9
    _close(got, ref, rows)
    P.unpatch(blk)
    assert type(blk).__name__ == "Qwen3MoeSparseMoeBlock"


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["affine", "mxfp4"])
@pytest.mark.parametrize("B", [1, 6])
def test_patched_deepseek_block_matches_transformers(dev, B, mode):
    blk = _deepseek_block()
    _init_block(blk)
    blk = blk.to(dev)
    ref_blk = copy.deepcopy(blk)
    _dequantise_experts_(ref_blk, mode=mode)
    P.patch(blk, quant_mode=mode)
    res = blk._zmlx_patch_result
    assert res.patched_count == 1, res.summary()
    g = torch.Generator(device=dev).manual_seed(10 + B)
    x = torch.randn(1, B, H, device=dev, generator=g).to(torch.bfloat16).float()
    with torch.no_grad():
        ref = ref_blk(x)
        got = blk(x)
    torch.cuda.synchronize()
    _close(got, ref)


@pytest.mark.gpu
def test_patched_qwen3_model_logits(dev):
    """Whole tiny model: every MoE block patched, logits against the
    unpatched model with dequantised experts."""
    m = _qwen3_model(layers=2)
    for layer in m.model.layers:
        _init_block(layer.mlp)
    m = m.to(dev)
    ref = copy.deepcopy(m)
    for layer in ref.model.layers:
        _dequantise_experts_(layer.mlp)
    P.patch(m)
    r = m._zmlx_patch_result
    assert r.patched == ["model.layers.0.mlp", "model.layers.1.mlp"] and r.pattern_counts == {"moe_mlp": 2}
    ids = torch.arange(7, device=dev)[None] * 13 % 256
    with torch.no_grad():
        lr = ref(ids).logits
        lg = m(ids).logits
    torch.cuda.synchronize()
    rel = (lg - lr).norm() / lr.norm()
    assert rel < 2e-2, float(rel)
    assert (lg.argmax(-1) == lr.argmax(-1)).float().mean() >= 0.85


@pytest.mark.gpu
def test_layer_from_mlx_checkpoint_matches_patched_block(dev, tmp_path):
    """The patched block's quantised tensors saved under mlx_lm names and
    loaded back through layer_from_mlx give bit-identical outputs."""
    from safetensors.torch import save_file

    m = _qwen3_model(layers=1)
    blk = m.model.layers[0].mlp
    _init_block(blk)
    blk = blk.to(dev)
    P.patch(blk)
    L = blk._zmoe_layer
    pre = "model.layers.0.mlp"
    t = {f"{pre}.gate.weight": L._router_w.cpu()}
    for n in ("gate", "up", "down"):
        w, s, b = L._proj[n]
        t[f"{pre}.switch_mlp.{n}_proj.weight"] = w.cpu()
        t[f"{pre}.switch_mlp.{n}_proj.scales"] = s.cpu()
        t[f"{pre}.switch_mlp.{n}_proj.biases"] = b.cpu()
    path = tmp_path / "model.safetensors"
    save_file(t, str(path))
    L2 = P.layer_from_mlx(path, pre, "qwen3", top_k=K, device=dev)
    g = torch.Generator(device=dev).manual_seed(9)
    for B in (1, 3, 40):
        x = torch.randn(B, H, device=dev, generator=g).to(torch.bfloat16)
        assert torch.equal(L(x), L2(x))
