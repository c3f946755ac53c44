"""The C-ABI library without a GPU: it loads, exports every function that
include/glmmoe.h declares, validates arguments on the host (no HIP call is
made before the checks), sizes workspaces, and the C++ header compiles
against it."""
import ctypes as C
import os
import re
import subprocess

import pytest

from glmserve_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "glmmoe.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(glmmoe_\w+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(L, name), name
    # and the Python binding table covers the header exactly
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    assert b"gfx950" in L.glmmoe_version()


def test_host_argument_checks():
    L = _lib.lib()
    # NULL pointers / non-positive sizes -> GLMMOE_ERR_ARG before any HIP call.
    assert L.glmmoe_moe_router(None, None, 4, 256, 8, 1, 2.5, None, None, None) == -1
    assert L.glmmoe_moe_dispatch(None, 4, 8, 256, None, None, None, None) == -1
    assert L.glmmoe_router_logits(None, None, 1, 6144, 256, None, None, None, 0, None) == -1
    dummy = C.c_void_p(16)   # never dereferenced: the shape checks reject first
    # Shapes outside the kernels' range -> GLMMOE_ERR_SHAPE.
    assert L.glmmoe_moe_router(dummy, None, 4, 256, 9, 1, 2.5, dummy, dummy, None) == -2
    assert L.glmmoe_moe_router(dummy, None, 4, 600, 8, 1, 2.5, dummy, dummy, None) == -2
    assert L.glmmoe_moe_router(dummy, None, 4, 4, 8, 1, 2.5, dummy, dummy, None) == -2
    assert L.glmmoe_moe_dispatch(dummy, 4, 8, 513, dummy, dummy, dummy, None) == -2
    assert L.glmmoe_router_logits(dummy, dummy, 1, 6145, 256, dummy, None, None, 0, None) == -2
    # small batches need the partials scratch; from 256 tokens none
    assert L.glmmoe_router_logits_workspace_bytes(64, 6144, 256) == 64 * 48 * 256 * 4
    assert L.glmmoe_router_logits_workspace_bytes(256, 6144, 256) == 0
    assert L.glmmoe_router_logits(dummy, dummy, 64, 6144, 256, dummy, None, None, 0, None) == -3
    assert L.glmmoe_pack_w4a16(dummy, dummy, 0, 1, 15, 128, 128, dummy, dummy, None) == -2
    assert L.glmmoe_pack_w4a16(dummy, dummy, 0, 1, 16, 100, 128, dummy, dummy, None) == -2
    assert L.glmmoe_pack_w4a16(dummy, dummy, 0, 1, 16, 128, 64, dummy, dummy, None) == -2
    assert L.glmmoe_pack_w4a16(dummy, dummy, 2, 1, 16, 128, 128, dummy, dummy, None) == -1


def test_reference_signature_host_checks():
    L = _lib.lib()
    dummy = C.c_void_p(16)   # never dereferenced: the checks below reject first
    assert L.glmmoe_ref_moe_expert_ffn_w4a16(None, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                                             dummy, 1, 8, 6144, 2048, 256, 128, dummy, None) == -1
    # group sizes other than 128 are outside the packed format
    assert L.glmmoe_ref_moe_expert_ffn_w4a16(dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                                             dummy, dummy, 1, 8, 6144, 2048, 256, 64, dummy,
                                             None) == -2
    assert L.glmmoe_ref_gemm_w4a16(None, dummy, dummy, None, dummy, 1, 6144, 2048, 128, None) == -1
    assert L.glmmoe_ref_gemm_w4a16(dummy, dummy, dummy, None, dummy, -1, 6144, 2048, 128, None) == -1
    assert L.glmmoe_ref_gemm_fp8(dummy, None, None, None, dummy, 1, 64, 64, None) == -1
    assert L.glmmoe_ref_silu_mul(dummy, dummy, None, 8, None) == -1
    assert L.glmmoe_ref_add_inplace(dummy, dummy, -1, None) == -1
    assert L.glmmoe_ref_moe_expert_ffn(dummy, dummy, dummy, None, dummy, dummy, 1, 8, 64, 64, 16,
                                       dummy, None) == -1
    # x in bf16 plus the routed-only layer workspace
    lw = L.glmmoe_layer_workspace_bytes(C.byref(_layer(shared=False)), 64)
    assert L.glmmoe_ref_workspace_bytes(64, 8, 6144, 2048, 256) == 64 * 6144 * 2 + lw
    assert L.glmmoe_ref_workspace_bytes(0, 8, 6144, 2048, 256) == 0
    # registry: host-side table keyed by the reference's qweight and scale pointers
    packed = _layer(shared=False)
    a, b, c = C.c_void_p(0x1000), C.c_void_p(0x2000), C.c_void_p(0x3000)
    sa, sb, sc = C.c_void_p(0x4000), C.c_void_p(0x5000), C.c_void_p(0x6000)
    assert L.glmmoe_ref_register_w4a16(None, sa, b, sb, c, sc, C.byref(packed)) == -1
    assert L.glmmoe_ref_register_w4a16(a, None, b, sb, c, sc, C.byref(packed)) == -1
    assert L.glmmoe_ref_register_w4a16(a, sa, b, sb, c, sc, C.byref(packed)) == 0
    # a call naming the same qweights with other scale arrays finds no set
    dummy2 = C.c_void_p(16)
    assert L.glmmoe_ref_moe_expert_ffn_w4a16(dummy2, dummy2, dummy2, a, sa, b, C.c_void_p(0x7000), c, sc,
                                             4, 8, 6144, 2048, 256, 128, dummy2, None) == -1
    assert L.glmmoe_ref_unregister_w4a16(a, sa, b, C.c_void_p(0x7000), c, sc) == -1
    assert L.glmmoe_ref_unregister_w4a16(a, sa, b, sb, c, sc) == 0
    assert L.glmmoe_ref_unregister_w4a16(a, sa, b, sb, c, sc) == -1
    # GGUF: supported types, row lengths a multiple of the block, row_bytes large enough
    assert L.glmmoe_ref_gemm_q(18, None, dummy, None, dummy, 1, 6144, 64, 2352, None) == -1
    assert L.glmmoe_ref_gemm_q(99, dummy, dummy, None, dummy, 1, 6144, 64, 2352, None) == -2
    assert L.glmmoe_ref_gemm_q(18, dummy, dummy, None, dummy, 1, 6100, 64, 2352, None) == -2
    assert L.glmmoe_ref_gemm_q(18, dummy, dummy, None, dummy, 1, 6144, 64, 2351, None) == -2
    assert L.glmmoe_ref_moe_expert_ffn_q(18, 18, 23, dummy, dummy, dummy, dummy, dummy, dummy,
                                         1, 8, 6144, 2048, 256, 2352, 2352, 1088, None, dummy,
                                         dummy, None, None, None) == -1
    assert L.glmmoe_ref_moe_expert_ffn_q(18, 18, 23, dummy, dummy, dummy, dummy, dummy, dummy,
                                         1, 8, 6144, 2048, 256, 2352, 2352, 1087, dummy, dummy,
                                         dummy, None, None, None) == -2
    # int8 twins: int8-capable types only, rows a multiple of 32, 4-byte aligned int8 rows
    assert [t for t in range(32) if L.glmmoe_ref_qtype_has_i8(t)] == [8, 11, 12, 13, 14, 18, 23]
    assert L.glmmoe_ref_quantize_act_q8(dummy, 2, 48, dummy, dummy, None) == -2
    assert L.glmmoe_ref_quantize_act_q8(None, 2, 64, dummy, dummy, None) == -1
    assert L.glmmoe_ref_gemm_q_i8(1, dummy, dummy, dummy, None, dummy, 1, 256, 8, 512, None) == -2
    assert L.glmmoe_ref_gemm_q_i8(8, C.c_void_p(18), dummy, dummy, None, dummy, 1, 256, 8, 272,
                                  None) == -2
    assert L.glmmoe_ref_gemm_q_i8(8, dummy, None, dummy, None, dummy, 1, 256, 8, 272, None) == -1
    i8 = [18, 18, 23, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1, 8, 6144, 2048, 256,
          2352, 2352, 1088, dummy, dummy, dummy, dummy, dummy, None, None, None]
    bad = list(i8); bad[2] = 0                    # F32 down: no int8 form
    assert L.glmmoe_ref_moe_expert_ffn_q_i8(*bad) == -2
    bad = list(i8); bad[19] = None                # hq
    assert L.glmmoe_ref_moe_expert_ffn_q_i8(*bad) == -1
    bad = list(i8); bad[13] = 2040                # moe_inter % 32
    assert L.glmmoe_ref_moe_expert_ffn_q_i8(*bad) == -2


def _layer(H=6144, I=2048, E=256, k=8, shared=True):
    st = _lib.Layer()
    st.hidden, st.moe_inter, st.n_experts, st.topk = H, I, E, k
    st.norm_topk, st.routed_scale = 1, 2.5
    p = 4096
    for f in ("router_w", "gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s"):
        setattr(st, f, p)
    if shared:
        for f in ("sh_gate_q", "sh_gate_s", "sh_up_q", "sh_up_s", "sh_down_q", "sh_down_s"):
            setattr(st, f, p)
    return st


def test_workspace_sizing_and_view():
    L = _lib.lib()
    st = _layer()
    for n in (1, 64, 4096):
        b = L.glmmoe_layer_workspace_bytes(C.byref(st), n)
        assert b > 0
        v = _lib.LayerWs()
        base = 1 << 20
        assert L.glmmoe_layer_workspace_view(C.byref(st), n, C.c_void_p(base), C.byref(v)) == 0
        assert v.bytes == b
        R = n * 8 + n
        # regions are 256-byte aligned, ordered, inside [base, base + bytes)
        regions = [v.logits, v.rpart, v.xsum, v.topk_ids, v.topk_w, v.expert_offsets, v.sorted_token_ids,
                   v.sorted_row, v.inv, v.tiles, v.ntiles, v.h, v.hsum, v.dpart]
        assert all(r % 256 == 0 for r in regions)
        assert regions == sorted(regions) and regions[0] == base
        assert v.dpart + R * 6144 * 4 <= base + b
        assert v.h + R * 2048 * 2 <= v.hsum
    # Unsupported layers size to 0 and are rejected.
    assert L.glmmoe_layer_workspace_bytes(C.byref(_layer(H=6000)), 4) == 0
    assert L.glmmoe_layer_workspace_bytes(C.byref(_layer(k=9)), 4) == 0
    bad = _layer()
    bad.sh_up_q = None          # a partial shared expert is an argument error
    assert L.glmmoe_layer_workspace_bytes(C.byref(bad), 4) == 0
    assert L.glmmoe_moe_layer_w4a16(C.byref(_layer()), C.c_void_p(16), 4, C.c_void_p(16),
                                    C.c_void_p(16), 16, None) == -3


def test_zero_token_calls_are_no_ops():
    # n == 0 returns GLMMOE_OK on every entry point without a device call (so
    # without a GPU here), with NULL data pointers; negative n stays an
    # argument error. (moe_dispatch at n == 0 writes its zero offsets: a GPU
    # test covers it.)
    L = _lib.lib()
    st = C.byref(_layer())
    assert L.glmmoe_moe_layer_w4a16(st, None, 0, None, None, 0, None) == 0
    assert L.glmmoe_moe_layer_w4a16_f32(st, None, 0, None, None, 0, None) == 0
    assert L.glmmoe_moe_layer_w4a16_noalloc(st, None, 0, None, None) == 0
    assert L.glmmoe_moe_route_w4a16(st, None, 0, None, None, None, 0, None) == 0
    assert L.glmmoe_expert_ffn_w4a16(st, None, 0, None, None, None, None, 0, None) == 0
    st8 = _lib.Fp8Layer()
    for name, _ in _lib.Layer._fields_:
        setattr(st8, name, getattr(_layer(), name))
    assert L.glmmoe_moe_layer_fp8(C.byref(st8), None, 0, None, None, 0, None) == 0
    assert L.glmmoe_expert_ffn_fp8(C.byref(st8), None, 0, None, None, None, None, 0, None) == 0
    assert L.glmmoe_quant_act_fp8(None, 0, 6144, None, None, None) == 0
    assert L.glmmoe_router_logits(None, None, 0, 6144, 256, None, None, None, 0, None) == 0
    assert L.glmmoe_router_logits_f32(None, None, None, None, 0, 6144, 256, None) == 0
    assert L.glmmoe_moe_router(None, None, 0, 256, 8, 1, 2.5, None, None, None) == 0
    assert L.glmmoe_ref_moe_expert_ffn_w4a16(None, None, None, None, None, None, None, None, None,
                                             0, 8, 6144, 2048, 256, 128, None, None) == 0
    assert L.glmmoe_ref_moe_expert_ffn(None, None, None, None, None, None, 0, 8, 64, 64, 16,
                                       None, None) == 0
    assert L.glmmoe_ref_gemm_w4a16(None, None, None, None, None, 0, 6144, 2048, 128, None) == 0
    assert L.glmmoe_ref_gemm_fp8(None, None, None, None, None, 0, 64, 64, None) == 0
    assert L.glmmoe_ref_silu_mul(None, None, None, 0, None) == 0
    assert L.glmmoe_ref_add_inplace(None, None, 0, None) == 0
    assert L.glmmoe_ref_gemm_q(18, None, None, None, None, 0, 6144, 64, 2352, None) == 0
    assert L.glmmoe_ref_moe_expert_ffn_q(18, 18, 23, None, None, None, None, None, None, 0, 8,
                                         6144, 2048, 256, 2352, 2352, 1088, None, None, None,
                                         None, None, None) == 0
    assert L.glmmoe_ref_quantize_act_q8(None, 0, 64, None, None, None) == 0
    assert L.glmmoe_ref_gemm_q_i8(18, None, None, None, None, None, 0, 256, 8, 98, None) == 0
    assert L.glmmoe_ref_moe_expert_ffn_q_i8(18, 18, 23, None, None, None, None, None, None, None,
                                            0, 8, 6144, 2048, 256, 2352, 2352, 1088, None, None,
                                            None, None, None, None, None, None) == 0
    # negative counts are errors
    assert L.glmmoe_moe_layer_w4a16(st, None, -1, None, None, 0, None) == -1
    assert L.glmmoe_moe_router(None, None, -1, 256, 8, 1, 2.5, None, None, None) == -1
    assert L.glmmoe_moe_dispatch(None, -1, 8, 256, C.c_void_p(16), None, None, None) == -1
    # dispatch at n == 0 needs only the offsets
    assert L.glmmoe_moe_dispatch(None, 0, 8, 256, None, None, None, None) == -1


def test_f32_layer_workspace_and_checks():
    # The fp32-activation layer: the layer's workspace plus the n x H bf16
    # copy of x at its end (256-byte aligned).
    L = _lib.lib()
    st = C.byref(_layer())
    for n in (1, 64, 300, 4096):
        lw = L.glmmoe_layer_workspace_bytes(st, n)
        assert L.glmmoe_layer_f32_workspace_bytes(st, n) == lw + (n * 6144 * 2 + 255) // 256 * 256
    assert L.glmmoe_layer_f32_workspace_bytes(C.byref(_layer(k=9)), 4) == 0
    d = C.c_void_p(16)
    assert L.glmmoe_moe_layer_w4a16_f32(st, None, 4, d, d, 1 << 30, None) == -1
    assert L.glmmoe_moe_layer_w4a16_f32(st, d, 4, d, d, L.glmmoe_layer_workspace_bytes(st, 4),
                                        None) == -3


def test_noalloc_entry_host_checks():
    # The no-allocation entry sizes the batch before any device call: a batch
    # whose workspace exceeds the library's scratch, or a bad layer, is
    # refused here (no GPU needed).
    L = _lib.lib()
    cap = L.glmmoe_noalloc_scratch_bytes()
    assert cap == 32 << 20
    assert L.glmmoe_layer_workspace_bytes(C.byref(_layer()), 64) <= cap   # decode fits
    big = 256
    assert L.glmmoe_layer_workspace_bytes(C.byref(_layer()), big) > cap
    assert L.glmmoe_moe_layer_w4a16_noalloc(C.byref(_layer()), C.c_void_p(16), big, C.c_void_p(16),
                                            None) == -3
    assert L.glmmoe_moe_layer_w4a16_noalloc(C.byref(_layer(k=9)), C.c_void_p(16), 4, C.c_void_p(16),
                                            None) == -1


def test_cpp_header_compiles_against_the_library(tmp_path):
    src = tmp_path / "use.cpp"
    src.write_text(
        '#define GLMMOE_GLMSERVE_NAMESPACE\n'
        '#include "glmmoe/kernels.hpp"\n'
        'int main() {\n'
        '  // reference call sites, unchanged apart from the include\n'
        '  glmserve::cuda::moe_router(nullptr, nullptr, 1, 256, 8, true, 2.5f, nullptr, nullptr);\n'
        '  glmserve::cuda::moe_dispatch(nullptr, 1, 8, 256, nullptr, nullptr, nullptr);\n'
        '  const float* x = nullptr; float* y = nullptr; const uint8_t* q = nullptr;\n'
        '  const float* sc = nullptr; const int* ids = nullptr; const float* w = nullptr;\n'
        '  glmserve::cuda::moe_expert_ffn_w4a16(x, ids, w, q, sc, q, sc, q, sc, 1, 8, 6144, 2048,\n'
        '                                       256, 128, y);\n'
        '  glmserve::cuda::moe_expert_ffn(x, ids, w, sc, sc, sc, 1, 8, 6144, 2048, 256, y);\n'
        '  glmserve::cuda::gemm_w4a16(x, q, sc, nullptr, y, 1, 6144, 2048, 128);\n'
        '  glmserve::cuda::gemm_fp8(x, q, sc, nullptr, y, 1, 6144, 2048);\n'
        '  glmserve::cuda::silu_mul(x, x, y, 2048);\n'
        '  glmserve::cuda::add_inplace(y, x, 6144);\n'
        '  float* hbuf = nullptr; int* disp = nullptr;\n'
        '  glmserve::cuda::gemm_q(18, x, q, nullptr, y, 1, 6144, 2048, 6144 / 256 * 98);\n'
        '  glmserve::cuda::moe_expert_ffn_q(18, 18, 23, x, ids, w, q, q, q, 1, 8, 6144, 2048, 256,\n'
        '                                   2352, 2352, 1088, hbuf, hbuf, y, disp);\n'
        '  int8_t* xq = nullptr; float* xs = nullptr;\n'
        '  if (glmserve::cuda::qtype_has_i8(18)) {\n'
        '    glmserve::cuda::quantize_act_q8(x, 1, 6144, xq, xs);\n'
        '    glmserve::cuda::gemm_q_i8(18, xq, xs, q, nullptr, y, 1, 6144, 2048, 2352);\n'
        '    glmserve::cuda::moe_expert_ffn_q_i8(18, 18, 23, xq, xs, ids, w, q, q, q, 1, 8, 6144,\n'
        '                                        2048, 256, 2352, 2352, 1088, hbuf, xq, xs, hbuf,\n'
        '                                        y, disp);\n'
        '  }\n'
        '  glmmoe_w4a16_layer L{};\n'
        '  glmserve::cuda::moe_layer_w4a16(L, x, 1, y, nullptr, 0);   // fp32 s.normed\n'
        '  return (int)glmserve::cuda::moe_layer_workspace_bytes(L, 1) +\n'
        '         (int)glmserve::cuda::moe_layer_f32_workspace_bytes(L, 1);\n'
        '}\n')
    exe = tmp_path / "use"
    r = subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                        str(exe), _lib.LIB_PATH, "-Wl,-rpath," + os.path.dirname(_lib.LIB_PATH)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_fp8_host_checks_and_workspace():
    L = _lib.lib()
    dummy = C.c_void_p(16)
    assert L.glmmoe_fp8_packed_bytes(2048, 6144) == 2048 * 6144
    assert L.glmmoe_pack_fp8(None, 1, 128, 128, dummy, None) == -1
    assert L.glmmoe_pack_fp8(dummy, 1, 96, 128, dummy, None) == -2
    assert L.glmmoe_pack_fp8(dummy, 1, 128, 200, dummy, None) == -2
    assert L.glmmoe_quant_act_fp8(dummy, 4, 100, dummy, dummy, None) == -2
    assert L.glmmoe_quant_act_fp8(None, 4, 128, dummy, dummy, None) == -1
    st = _lib.Fp8Layer()
    src = _layer()
    for name, _ in _lib.Layer._fields_:
        setattr(st, name, getattr(src, name))
    for n in (1, 8192):
        b = L.glmmoe_fp8_layer_workspace_bytes(C.byref(st), n)
        v = _lib.Fp8Ws()
        base = 1 << 20
        assert L.glmmoe_fp8_layer_workspace_view(C.byref(st), n, C.c_void_p(base), C.byref(v)) == 0
        assert v.bytes == b
        R = n * 9
        regions = [v.logits, v.rpart, v.xq, v.xscale, v.topk_ids, v.topk_w, v.expert_offsets,
                   v.sorted_token_ids, v.sorted_row, v.inv, v.tiles, v.ntiles, v.hq, v.hscale,
                   v.dpart]
        assert all(r % 256 == 0 for r in regions) and regions == sorted(regions)
        assert v.xscale - v.xq >= n * 6144 and v.hscale - v.hq >= R * 2048
        assert v.dpart + R * 6144 * 4 <= base + b
    assert L.glmmoe_moe_layer_fp8(C.byref(st), dummy, 4, dummy, dummy, 16, None) == -3
