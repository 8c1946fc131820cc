"""The committed fixtures (tests/golden/moe_golden.npz, restatement-generated
by tests/golden/make_golden.py) against the oracle as it is now, and the
whole-layer fixture against the independently written C++ restatement
(oracle/moe_ref.cpp).  CPU only."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import moe_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "moe_golden.npz"


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf(b):
    return O.bf16_from_bits(b)


def test_fixture_regenerates_identically(g):
    """The generator reproduces every stored array bit for bit."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN.parent / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.generate()
    assert sorted(fresh) == sorted(g)
    for k, v in fresh.items():
        np.testing.assert_array_equal(np.asarray(v), g[k], err_msg=k)


def test_dequant_fixtures(g):
    np.testing.assert_array_equal(O.dequant_affine(g["deq_a_w"][0], bf(g["deq_a_s"][0]), bf(g["deq_a_b"][0])),
                                  g["deq_a_out"])
    np.testing.assert_array_equal(O.dequant_mxfp4(g["deq_m_w"][0], g["deq_m_e"][0]), g["deq_m_out"])


def test_router_fixtures(g):
    idx, w, _ = O.qwen_gating(bf(g["qwen_logits"]), 8, True)
    np.testing.assert_array_equal(idx, g["qwen_idx"])
    np.testing.assert_array_equal(O.bf16_to_bits(w), g["qwen_w"])
    w, idx = O.topk_gating_softmax(g["lfm2_logits"], 4)
    np.testing.assert_array_equal(idx, g["lfm2_idx"])
    np.testing.assert_array_equal(w, g["lfm2_w"])
    w, idx = O.deepseek_router_topk_sigmoid(g["ds_logits"], g["ds_bias"], k=8, n_group=8, topk_group=4,
                                            routed_scaling_factor=2.5)
    np.testing.assert_array_equal(idx, g["ds_idx"])
    np.testing.assert_array_equal(w, g["ds_w"])


def test_combine_fixtures(g):
    y = bf(g["comb_y"])
    for mode in O.COMBINE_MODES:
        wm = g["comb_wf"] if mode.startswith("fp32") else bf(g["comb_wb"])
        np.testing.assert_array_equal(O.moe_combine(y, wm, mode), g[f"comb_out_{mode}"], err_msg=mode)


def test_layer_fixture_against_cpp_restatement(g):
    """numpy oracle (float64 GEMVs) vs the C++ restatement (fp32 group-
    factored GEMVs): same experts, outputs within the reference tolerance and
    mostly bit-identical."""
    from oracle import ref_lib

    x, wr = bf(g["layer_x"]), bf(g["layer_wr"])
    proj = tuple((g[f"layer_{n}_w"], bf(g[f"layer_{n}_s"]), bf(g[f"layer_{n}_b"])) for n in ("gate", "up", "down"))
    out, idx = ref_lib.moe_layer_qwen(x, wr, *proj, k=2, group_size=64, norm=True, threads=2)
    np.testing.assert_array_equal(np.sort(idx, -1), np.sort(g["layer_idx"], -1))
    ref = bf(g["layer_out"])
    np.testing.assert_allclose(out, ref, atol=1e-2, rtol=1e-2)
    assert (O.bf16_ulp_diff(out, ref) == 0).mean() >= 0.9
