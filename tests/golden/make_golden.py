"""Writes tests/golden/moe_golden.npz: small seeded input/output vectors for
every stage of the decode path.

The outputs are RESTATEMENT-GENERATED (oracle/moe_oracle.py), not MLX-
generated: MLX cannot run in this environment and the reference holds no
numeric fixtures for this path.  They freeze the oracle's answers so that a
later change to it shows up as a fixture diff, and they give the GPU tests
fixed inputs.  bf16 arrays are stored as uint16 bit patterns.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import moe_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "moe_golden.npz"
SEED = 20260101


def bits(a):
    return O.bf16_to_bits(a)


def generate() -> dict[str, np.ndarray]:
    from tests.moe_case import bf16_randn, make_bank

    rng = np.random.default_rng(SEED)
    g: dict[str, np.ndarray] = {}

    # affine g64 and mxfp4 dequantisation (one expert, 32 rows x 256)
    ba = make_bank(rng, 1, 32, 256)
    g["deq_a_w"], g["deq_a_s"], g["deq_a_b"] = ba.w, bits(ba.s), bits(ba.b)
    g["deq_a_out"] = ba.deq(0)
    bm = make_bank(rng, 1, 32, 256, mode="mxfp4")
    g["deq_m_w"], g["deq_m_e"] = bm.w, bm.s
    g["deq_m_out"] = bm.deq(0)

    # Qwen gating on bf16 logits [4, 128], top-8 renormalised
    lq = bf16_randn(rng, (4, 128))
    idx, w, _ = O.qwen_gating(lq, 8, True)
    g["qwen_logits"], g["qwen_idx"], g["qwen_w"] = bits(lq), idx, bits(w)

    # LFM2 topk_gating_softmax on float32 logits [4, 32], top-4
    ll = rng.standard_normal((4, 32)).astype(np.float32)
    w, idx = O.topk_gating_softmax(ll, 4)
    g["lfm2_logits"], g["lfm2_idx"], g["lfm2_w"] = ll, idx, w

    # DeepSeek grouped sigmoid router [2, 256], 8 groups keep 4, top-8, x2.5
    ld = rng.standard_normal((2, 256)).astype(np.float32)
    bd = (rng.standard_normal(256) * 0.5).astype(np.float32)
    w, idx = O.deepseek_router_topk_sigmoid(ld, bd, k=8, n_group=8, topk_group=4, routed_scaling_factor=2.5)
    g["ds_logits"], g["ds_bias"], g["ds_idx"], g["ds_w"] = ld, bd, idx, w

    # combines: y bf16 [2, 4, 256]; w float32 (fp32 modes) / bf16 (others)
    y = bf16_randn(rng, (2, 4, 256))
    wf = rng.random((2, 4)).astype(np.float32)
    g["comb_y"], g["comb_wf"], g["comb_wb"] = bits(y), wf, bits(O.bf16_round(wf))
    for mode in O.COMBINE_MODES:
        wm = wf if mode.startswith("fp32") else O.bf16_round(wf)
        g[f"comb_out_{mode}"] = O.moe_combine(y, wm, mode)

    # whole layer, Qwen-style (softmax top-2 of 4 experts, native combine)
    H, E, I, K, B = 256, 4, 256, 2, 2
    banks = {n: make_bank(rng, E, *shape) for n, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    wr = bf16_randn(rng, (E, H), 0.05)
    x = bf16_randn(rng, (B, H))
    logits = O.dense_logits(x, wr)
    idx, w, _ = O.qwen_gating(logits, K, True)
    yk = O.moe_experts(x, idx, banks["gate"].as_tuple(), banks["up"].as_tuple(), banks["down"].as_tuple())
    out = O.bf16_round(O.moe_combine(yk, w, "native"))
    g["layer_x"], g["layer_wr"] = bits(x), bits(wr)
    for n, bk in banks.items():
        g[f"layer_{n}_w"], g[f"layer_{n}_s"], g[f"layer_{n}_b"] = bk.w, bits(bk.s), bits(bk.b)
    g["layer_logits"], g["layer_idx"], g["layer_w"], g["layer_out"] = bits(logits), idx, bits(w), bits(out)
    g["seed"] = np.array(SEED)
    return g


def main() -> None:
    g = generate()
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
