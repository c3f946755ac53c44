"""glmserve_amd -- MI355X (gfx950) native MoE-layer hot path for glmserve.

The compute path is the HIP library glmserve_amd/_lib/libglmmoe.so (sources in
glmserve_amd/csrc/, C-ABI in include/glmmoe.h). This package is the host-side
mirror of the reference's launch API (cuda/kernels.cuh) over torch tensors.
"""
from ._lib import LIB_PATH, GlmMoeError, lib  # noqa: F401
from .ops import (FP8MoELayer, W4A16MoELayer, moe_dispatch, moe_router,  # noqa: F401
                  pack_fp8, pack_w4a16, quant_act_fp8, router_logits, router_logits_f32)
from .checkpoint import load_layer, quantize_w4, read_layer  # noqa: F401,E402
