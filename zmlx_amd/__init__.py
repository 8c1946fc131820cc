"""zmlx_amd -- MI355X-native (gfx950) fused quantized-MoE decode path.

A drop-in for the MoE block that Hmbown/ZMLX's ``patch(model)`` rewrites:
router top-k gating, ``gather_qmm_swiglu``, the down projection and
``moe_combine``, as hand-written HIP kernels behind the C ABI of
``include/zmlx_amd.h``, called from PyTorch-ROCm through ctypes.

Submodules:
  ops     reference-named torch ops (gather_qmm_swiglu, topk_gating_softmax, ...)
  layer   QuantizedMoELayer: one whole MoE block over device-resident weights
  patch   patch()/unpatch() model walker with the moe_mlp / deepseek_router patterns
  quant   MLX-format quantisers (affine g32/64/128, mxfp4) for building weights
"""

from __future__ import annotations

from ._native import NativeLibraryMissing, ZmoeError, version  # noqa: F401
from .ops import *  # noqa: F401,F403
from .ops import __all__ as _ops_all

__all__ = ["NativeLibraryMissing", "ZmoeError", "version", *_ops_all]
__version__ = "0.1.0"
