"""Loads the in-tree HIP library (glmserve_amd/_lib/libglmmoe.so) via ctypes.

There is no fallback: if the library is missing, every entry point raises.
"""
import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libglmmoe.so")
# Diagnostics only: load a differently built copy of the same library.
LIB_PATH = os.environ.get("GLMMOE_LIB_PATH", LIB_PATH)

# Every exported symbol of include/glmmoe.h, with its ctypes signature.
_vp, _i, _f, _sz, _i64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_int64
SIGNATURES = {
    "glmmoe_version": (C.c_char_p, []),
    "glmmoe_router_logits_workspace_bytes": (_sz, [_i, _i, _i]),
    "glmmoe_router_logits": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _sz, _vp]),
    "glmmoe_router_logits_f32": (_i, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "glmmoe_moe_router": (_i, [_vp, _vp, _i, _i, _i, _i, _f, _vp, _vp, _vp]),
    "glmmoe_moe_dispatch": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "glmmoe_w4_packed_bytes": (_sz, [_i, _i]),
    "glmmoe_w4_packed_scale_bytes": (_sz, [_i, _i]),
    "glmmoe_pack_w4a16": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "glmmoe_layer_workspace_bytes": (_sz, [_vp, _i]),
    "glmmoe_layer_workspace_view": (_i, [_vp, _i, _vp, _vp]),
    "glmmoe_moe_layer_w4a16": (_i, [_vp, _vp, _i, _vp, _vp, _sz, _vp]),
    "glmmoe_layer_f32_workspace_bytes": (_sz, [_vp, _i]),
    "glmmoe_moe_layer_w4a16_f32": (_i, [_vp, _vp, _i, _vp, _vp, _sz, _vp]),
    "glmmoe_noalloc_scratch_bytes": (_sz, []),
    "glmmoe_moe_layer_w4a16_noalloc": (_i, [_vp, _vp, _i, _vp, _vp]),
    "glmmoe_moe_route_w4a16": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _sz, _vp]),
    "glmmoe_expert_ffn_w4a16": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "glmmoe_fp8_packed_bytes": (_sz, [_i, _i]),
    "glmmoe_pack_fp8": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "glmmoe_quant_act_fp8": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "glmmoe_fp8_layer_workspace_bytes": (_sz, [_vp, _i]),
    "glmmoe_fp8_layer_workspace_view": (_i, [_vp, _i, _vp, _vp]),
    "glmmoe_moe_layer_fp8": (_i, [_vp, _vp, _i, _vp, _vp, _sz, _vp]),
    "glmmoe_expert_ffn_fp8": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "glmmoe_profile_enable": (_i, [_i]),
    "glmmoe_profile_read": (_i, [_vp, _vp]),
    "glmmoe_ref_register_w4a16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "glmmoe_ref_unregister_w4a16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "glmmoe_ref_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "glmmoe_ref_set_workspace": (_i, [_vp, _sz]),
    "glmmoe_ref_moe_expert_ffn_w4a16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "glmmoe_ref_moe_expert_ffn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp,
                                       _vp]),
    "glmmoe_ref_gemm_w4a16": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "glmmoe_ref_gemm_fp8": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "glmmoe_ref_silu_mul": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "glmmoe_ref_add_inplace": (_i, [_vp, _vp, _i64, _vp]),
    "glmmoe_ref_gemm_q": (_i, [C.c_uint32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "glmmoe_ref_moe_expert_ffn_q": (_i, [C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _i, _i, _i, _i, _i, _i64, _i64, _i64, _vp,
                                         _vp, _vp, _vp, _vp, _vp]),
    "glmmoe_ref_qtype_has_i8": (_i, [C.c_uint32]),
    "glmmoe_ref_quantize_act_q8": (_i, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "glmmoe_ref_gemm_q_i8": (_i, [C.c_uint32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                  _vp]),
    "glmmoe_ref_moe_expert_ffn_q_i8": (_i, [C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i64, _i64,
                                            _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
}

STAGES = ["router_logits", "router_topk", "dispatch", "gate_up", "down", "combine"]

ERRORS = {-1: "GLMMOE_ERR_ARG", -2: "GLMMOE_ERR_SHAPE", -3: "GLMMOE_ERR_WORKSPACE",
          -4: "GLMMOE_ERR_LAUNCH"}


class GlmMoeError(RuntimeError):
    pass


class Layer(C.Structure):
    """glmmoe_w4a16_layer (include/glmmoe.h)."""
    _fields_ = [("hidden", _i), ("moe_inter", _i), ("n_experts", _i), ("topk", _i),
                ("norm_topk", _i), ("routed_scale", _f), ("router_w", _vp), ("e_bias", _vp),
                ("gate_q", _vp), ("gate_s", _vp), ("up_q", _vp), ("up_s", _vp),
                ("down_q", _vp), ("down_s", _vp), ("sh_gate_q", _vp), ("sh_gate_s", _vp),
                ("sh_up_q", _vp), ("sh_up_s", _vp), ("sh_down_q", _vp), ("sh_down_s", _vp)]


class Fp8Layer(Layer):
    """glmmoe_fp8_layer (include/glmmoe.h): the same fields, fp32 block scales."""
    _fields_ = []


class LayerWs(C.Structure):
    """glmmoe_layer_ws (include/glmmoe.h)."""
    _fields_ = [("logits", _vp), ("rpart", _vp), ("xsum", _vp), ("topk_ids", _vp), ("topk_w", _vp),
                ("expert_offsets", _vp), ("sorted_token_ids", _vp), ("sorted_row", _vp),
                ("inv", _vp), ("tiles", _vp), ("ntiles", _vp), ("h", _vp), ("hsum", _vp),
                ("dpart", _vp), ("sync", _vp), ("bytes", _sz)]


class Fp8Ws(C.Structure):
    """glmmoe_fp8_ws (include/glmmoe.h)."""
    _fields_ = [("logits", _vp), ("rpart", _vp), ("xq", _vp), ("xscale", _vp), ("topk_ids", _vp),
                ("topk_w", _vp), ("expert_offsets", _vp), ("sorted_token_ids", _vp),
                ("sorted_row", _vp), ("inv", _vp), ("tiles", _vp), ("ntiles", _vp),
                ("hq", _vp), ("hscale", _vp), ("dpart", _vp), ("bytes", _sz)]


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise GlmMoeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(rc, what):
    if rc != 0:
        raise GlmMoeError(f"{what} failed: {ERRORS.get(rc, rc)}")
