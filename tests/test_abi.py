"""CPU checks of the C-ABI boundary: the library loads, exports every function
the public header declares, and rejects bad arguments on the host (before any
GPU work) with the reference's error classes and messages.  No compute call
is made here: there is no GPU in this container."""

from __future__ import annotations

import ctypes

import pytest

from zmlx_amd import _native as N


@pytest.fixture(scope="module")
def lib():
    return N.lib()


def test_header_symbols_exported(lib):
    names = N.header_functions()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/zmlx_amd.h but not exported"
        assert name in N._SIGNATURES, f"{name} has no ctypes signature"
    assert sorted(N._SIGNATURES) == sorted(names)


def test_version(lib):
    v = N.version()
    assert v.startswith("zmlx_amd ") and "gfx950" in v


def _check_built_from_tree():
    from zmlx_amd.build import source_hash

    v = N.version()
    assert v.endswith(f"src:{source_hash()}"), f"loaded library ({v}) was not built from these sources"


def test_library_built_from_this_tree(lib):
    _check_built_from_tree()


@pytest.mark.gpu
def test_gpu_library_built_from_this_tree():
    """On the GPU box: the mapped library carries the hash of the sources it
    runs next to."""
    N.lib()
    _check_built_from_tree()


def _qmm_swiglu(lib, **kw):
    a = dict(stream=None, x=None, x_batch=1, gw=None, gs=None, gb=None, uw=None, us=None, ub=None, lhs=None,
             rhs=None, n_pairs=1, M=1, Nn=64, K=512, E=4, group_size=64, bits=4, quant_mode=N.Q_AFFINE, out=None)
    a.update(kw)
    return lib.zmoe_gather_qmm_swiglu(*a.values())


def _msg(lib) -> str:
    return lib.zmoe_last_error().decode()


def test_qmm_rejects_mode_bits_group(lib):
    assert _qmm_swiglu(lib, quant_mode=7) == N.ZMOE_EUNSUPPORTED
    assert "quantization mode" in _msg(lib)
    assert _qmm_swiglu(lib, bits=8) == N.ZMOE_EUNSUPPORTED
    assert _qmm_swiglu(lib, group_size=48) == N.ZMOE_EUNSUPPORTED
    assert _qmm_swiglu(lib, quant_mode=N.Q_MXFP4, group_size=64) == N.ZMOE_EUNSUPPORTED


def test_qmm_rejects_shapes(lib):
    rc = _qmm_swiglu(lib, K=320, gb=ctypes.c_void_p(16))
    assert rc == N.ZMOE_EINVAL_SHAPE and "multiple of 256" in _msg(lib)
    assert _qmm_swiglu(lib, M=0) == N.ZMOE_EINVAL_SHAPE
    # affine without biases
    assert _qmm_swiglu(lib) == N.ZMOE_EINVAL_SHAPE and "biases" in _msg(lib)
    # null pointers with pairs to compute
    assert _qmm_swiglu(lib, gb=ctypes.c_void_p(16)) == N.ZMOE_EINVAL_SHAPE


def test_router_rejects(lib):
    assert lib.zmoe_router_softmax_topk(None, None, 1, 8, 9, 1, None, None) == N.ZMOE_EINVAL_SHAPE
    assert lib.zmoe_deepseek_router_topk_sigmoid(None, None, None, 1, 10, 2, 3, 1, 1.0, None, None) == \
        N.ZMOE_EINVAL_SHAPE


def test_combine_rejects_mode(lib):
    assert lib.zmoe_moe_combine(None, None, None, N.DT_F32, 1, 2, 64, 99, None) < 0


def test_layer_rejects_null_and_small_workspace(lib):
    assert lib.zmoe_moe_layer(None, None, None, 1, None, None, None, None, 0) == N.ZMOE_EINVAL_SHAPE
    d = N.LayerDesc(hidden=2048, n_experts=128, top_k=8, inter=768, group_size=64, bits=4, quant_mode=N.Q_AFFINE,
                    router_kind=N.ROUTER_SOFTMAX_PROBS, norm_topk_prob=1, n_group=1, topk_group=1,
                    routed_scaling_factor=1.0, combine_mode=N.COMBINE_NATIVE)
    need = lib.zmoe_moe_layer_workspace_size(ctypes.byref(d), 1)
    assert need >= 16384
    rc = lib.zmoe_moe_layer(None, ctypes.byref(d), None, 1, None, None, None, None, 16)
    assert rc == N.ZMOE_EINVAL_SHAPE


def test_ops_fail_loudly_on_cpu_tensors():
    """No CPU fallback: ops reject host tensors instead of computing."""
    import torch

    from zmlx_amd import ops

    x = torch.zeros(1, 512, dtype=torch.bfloat16)
    w = torch.zeros(4, 64, 64, dtype=torch.int32)
    s = torch.zeros(4, 64, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.gather_qmm_swiglu(x, w, s, s, w, s, s)
    with pytest.raises(ValueError, match="GPU"):
        ops.moe_combine_fp32_no_fma(torch.zeros(1, 2, 64, dtype=torch.bfloat16), torch.ones(1, 2))


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setenv("ZMOE_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(N.NativeLibraryMissing):
        N.lib()
    monkeypatch.setattr(N, "_lib", None)
