"""Host-side mirror of glmserve's MoE launch API (cuda/kernels.cuh) over torch tensors.

Names, argument order and meaning follow the reference launchers; tensors are
device tensors and `stream` is a torch.cuda.Stream or None (current stream).
Unlike the reference (void return, errors printed), failures raise GlmMoeError.
"""
import torch

import ctypes

from ._lib import Fp8Layer, Fp8Ws, GlmMoeError, Layer, LayerWs, check, lib


def _p(t):
    return None if t is None else t.data_ptr()


def _s(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _need(t, dtype, numel, name):
    if t is None or not t.is_cuda or t.dtype != dtype or not t.is_contiguous() or t.numel() < numel:
        raise GlmMoeError(f"{name}: expected contiguous cuda {dtype} with >= {numel} elements")


def router_logits(x, wr, logits, xsum=None, stream=None):
    """logits[n,E] = x[n,H] . wr[E,H]^T (bf16 in, fp32 out, fixed order); replaces
    gemm_linear on the router (src/model_gpu.cpp:1448)."""
    n, H = x.shape
    E = wr.shape[0]
    _need(x, torch.bfloat16, n * H, "x")
    _need(wr, torch.bfloat16, E * H, "wr")
    _need(logits, torch.float32, n * E, "logits")
    if xsum is not None:
        _need(xsum, torch.float32, n * (H // 128), "xsum")
    nb = lib().glmmoe_router_logits_workspace_bytes(n, H, E)
    ws = torch.empty(nb, dtype=torch.uint8, device=x.device) if nb else None
    check(lib().glmmoe_router_logits(_p(x), _p(wr), n, H, E, _p(logits), _p(xsum), _p(ws), nb,
                                     _s(stream)), "router_logits")


def router_logits_f32(x, W, bias, y, stream=None):
    """y[n,E] = bf16(x)[n,H] . bf16(W)[E,H]^T (+ bias): gemm_fp32's arguments
    (cuda/kernels.cuh:37-38) for the router call of src/model_gpu.cpp:1448."""
    n, H = x.shape
    E = W.shape[0]
    _need(x, torch.float32, n * H, "x")
    _need(W, torch.float32, E * H, "W")
    _need(y, torch.float32, n * E, "y")
    if bias is not None:
        _need(bias, torch.float32, E, "bias")
    check(lib().glmmoe_router_logits_f32(_p(x), _p(W), _p(bias), _p(y), n, H, E, _s(stream)),
          "router_logits_f32")


def moe_router(logits, e_bias, n, E, topk, norm_topk, routed_scale, topk_ids, topk_weights,
               stream=None):
    """cuda/kernels.cuh:243-245."""
    _need(logits, torch.float32, n * E, "logits")
    if e_bias is not None:
        _need(e_bias, torch.float32, E, "e_bias")
    _need(topk_ids, torch.int32, n * topk, "topk_ids")
    _need(topk_weights, torch.float32, n * topk, "topk_weights")
    check(lib().glmmoe_moe_router(_p(logits), _p(e_bias), n, E, topk, int(bool(norm_topk)),
                                  float(routed_scale), _p(topk_ids), _p(topk_weights),
                                  _s(stream)), "moe_router")


def moe_dispatch(topk_ids, n, topk, E, expert_offsets, sorted_token_ids, sorted_row, stream=None):
    """cuda/kernels.cuh:249-250."""
    _need(topk_ids, torch.int32, n * topk, "topk_ids")
    _need(expert_offsets, torch.int32, E + 1, "expert_offsets")
    _need(sorted_token_ids, torch.int32, n * topk, "sorted_token_ids")
    _need(sorted_row, torch.int32, n * topk, "sorted_row")
    check(lib().glmmoe_moe_dispatch(_p(topk_ids), n, topk, E, _p(expert_offsets),
                                    _p(sorted_token_ids), _p(sorted_row), _s(stream)),
          "moe_dispatch")


def pack_w4a16(qweight, scales, n_mats, rows, K, group_size=128, stream=None):
    """Reference W4 layout ([n_mats, rows, K/2] u8 + [n_mats, rows, K/g] fp32|bf16 scales)
    -> native packed (q, scales) tensors."""
    L = lib()
    if scales.dtype not in (torch.float32, torch.bfloat16):
        raise GlmMoeError("scales must be float32 or bfloat16")
    _need(qweight, torch.uint8, n_mats * rows * K // 2, "qweight")
    pq = torch.empty(n_mats * L.glmmoe_w4_packed_bytes(rows, K), dtype=torch.uint8,
                     device=qweight.device)
    ps = torch.empty(n_mats * L.glmmoe_w4_packed_scale_bytes(rows, K) // 2, dtype=torch.bfloat16,
                     device=qweight.device)
    check(L.glmmoe_pack_w4a16(_p(qweight), _p(scales), 1 if scales.dtype == torch.bfloat16 else 0,
                              n_mats, rows, K, group_size, _p(pq), _p(ps), _s(stream)),
          "pack_w4a16")
    return pq, ps


class _MoELayer:
    """One MoE layer's device-resident expert weights in a native packed format.

    The weight tensors are kept alive by this object; `struct` is the layer
    descriptor handed to the C-ABI.
    """
    _struct = Layer
    _view = LayerWs
    _fn = dict(ws_bytes="glmmoe_layer_workspace_bytes", ws_view="glmmoe_layer_workspace_view",
               layer="glmmoe_moe_layer_w4a16", ffn="glmmoe_expert_ffn_w4a16")

    def __init__(self, hidden, moe_inter, n_experts, topk, router_w, e_bias, gate, up, down,
                 shared=None, norm_topk=True, routed_scale=2.5):
        """gate/up/down: (packed_q, scales) pairs of stacked experts; shared: a
        3-tuple of such pairs or None. router_w: [E, H] bf16; e_bias: [E] fp32 or None."""
        self.hidden, self.moe_inter, self.n_experts, self.topk = hidden, moe_inter, n_experts, topk
        self.keep = [router_w, e_bias, gate, up, down, shared]
        st = self._struct()
        st.hidden, st.moe_inter, st.n_experts, st.topk = hidden, moe_inter, n_experts, topk
        st.norm_topk, st.routed_scale = int(bool(norm_topk)), float(routed_scale)
        st.router_w, st.e_bias = _p(router_w), _p(e_bias)
        st.gate_q, st.gate_s = _p(gate[0]), _p(gate[1])
        st.up_q, st.up_s = _p(up[0]), _p(up[1])
        st.down_q, st.down_s = _p(down[0]), _p(down[1])
        if shared is not None:
            (sgq, sgs), (suq, sus), (sdq, sds) = shared
            st.sh_gate_q, st.sh_gate_s = _p(sgq), _p(sgs)
            st.sh_up_q, st.sh_up_s = _p(suq), _p(sus)
            st.sh_down_q, st.sh_down_s = _p(sdq), _p(sds)
        self.struct = st

    def _call(self, key, *args):
        return getattr(lib(), self._fn[key])(*args)

    def _ref(self):
        return ctypes.byref(self.struct)

    def workspace_bytes(self, n):
        b = self._call("ws_bytes", self._ref(), n)
        if b == 0:
            raise GlmMoeError("layer shape not supported")
        return b

    def alloc_workspace(self, n, device="cuda"):
        return torch.empty(self.workspace_bytes(n), dtype=torch.uint8, device=device)

    def workspace_view(self, n, ws):
        v = self._view()
        check(self._call("ws_view", self._ref(), n, _p(ws), ctypes.byref(v)), "workspace_view")
        return v

    def forward(self, x, out, ws, stream=None):
        """x: [n, H] bf16; out: [n, H] fp32."""
        n = x.shape[0]
        _need(x, torch.bfloat16, n * self.hidden, "x")
        _need(out, torch.float32, n * self.hidden, "out")
        check(self._call("layer", self._ref(), _p(x), n, _p(out), _p(ws), ws.numel(),
                         _s(stream)), self._fn["layer"])

    def route(self, x, topk_ids, topk_w, ws, stream=None):
        """The layer's routing alone (router logits + top-k) into topk_ids / topk_w."""
        if self._fn["layer"] != "glmmoe_moe_layer_w4a16":
            raise GlmMoeError("route: W4A16 layers only")
        n = x.shape[0]
        _need(x, torch.bfloat16, n * self.hidden, "x")
        _need(topk_ids, torch.int32, n * self.topk, "topk_ids")
        _need(topk_w, torch.float32, n * self.topk, "topk_w")
        check(lib().glmmoe_moe_route_w4a16(self._ref(), _p(x), n, _p(topk_ids), _p(topk_w), _p(ws),
                                           ws.numel(), _s(stream)), "glmmoe_moe_route_w4a16")

    def expert_ffn(self, x, topk_ids, topk_w, out, ws, stream=None):
        n = x.shape[0]
        _need(x, torch.bfloat16, n * self.hidden, "x")
        _need(out, torch.float32, n * self.hidden, "out")
        _need(topk_ids, torch.int32, n * self.topk, "topk_ids")
        _need(topk_w, torch.float32, n * self.topk, "topk_w")
        check(self._call("ffn", self._ref(), _p(x), n, _p(topk_ids), _p(topk_w), _p(out), _p(ws),
                         ws.numel(), _s(stream)), self._fn["ffn"])


class W4A16MoELayer(_MoELayer):
    """W4A16 experts: (packed_q, packed bf16 scales) from pack_w4a16."""

    def forward_noalloc(self, x, out, stream=None):
        """forward on the library's per-GPU scratch (glmmoe_moe_layer_w4a16_noalloc)."""
        n = x.shape[0]
        _need(x, torch.bfloat16, n * self.hidden, "x")
        _need(out, torch.float32, n * self.hidden, "out")
        check(lib().glmmoe_moe_layer_w4a16_noalloc(self._ref(), _p(x), n, _p(out), _s(stream)),
              "glmmoe_moe_layer_w4a16_noalloc")

    def alloc_workspace_f32(self, n, device="cuda"):
        """Workspace of forward_f32 (the layer's plus the bf16 copy of x)."""
        b = lib().glmmoe_layer_f32_workspace_bytes(self._ref(), n)
        if b == 0:
            raise GlmMoeError("layer shape not supported")
        return torch.empty(b, dtype=torch.uint8, device=device)

    def forward_f32(self, x, out, ws, stream=None):
        """x: [n, H] fp32 (rounded to bf16 inside); out: [n, H] fp32."""
        n = x.shape[0]
        _need(x, torch.float32, n * self.hidden, "x")
        _need(out, torch.float32, n * self.hidden, "out")
        check(lib().glmmoe_moe_layer_w4a16_f32(self._ref(), _p(x), n, _p(out), _p(ws), ws.numel(),
                                               _s(stream)), "glmmoe_moe_layer_w4a16_f32")


class FP8MoELayer(_MoELayer):
    """FP8 experts: (packed e4m3 from pack_fp8, fp32 [.., rows/128, K/128] block scales)."""
    _struct = Fp8Layer
    _view = Fp8Ws
    _fn = dict(ws_bytes="glmmoe_fp8_layer_workspace_bytes",
               ws_view="glmmoe_fp8_layer_workspace_view", layer="glmmoe_moe_layer_fp8",
               ffn="glmmoe_expert_ffn_fp8")


def pack_fp8(w, n_mats, rows, K, out=None, stream=None):
    """Row-major e4m3 [n_mats, rows, K] (uint8) -> the native tile layout (into
    `out`, a uint8 tensor or view of n_mats * glmmoe_fp8_packed_bytes bytes)."""
    _need(w, torch.uint8, n_mats * rows * K, "w")
    nbytes = n_mats * lib().glmmoe_fp8_packed_bytes(rows, K)
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _need(out, torch.uint8, nbytes, "out")
    check(lib().glmmoe_pack_fp8(_p(w), n_mats, rows, K, _p(out), _s(stream)), "pack_fp8")
    return out


def quant_act_fp8(x, stream=None):
    """x [n, K] bf16 -> (q [n, K] uint8 e4m3, scale [n, K/128] fp32)."""
    n, K = x.shape
    _need(x, torch.bfloat16, n * K, "x")
    q = torch.empty((n, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((n, K // 128), dtype=torch.float32, device=x.device)
    check(lib().glmmoe_quant_act_fp8(_p(x), n, K, _p(q), _p(s), _s(stream)), "quant_act_fp8")
    return q, s


def ws_tensor(ws_base, view_ptr, ws, dtype, numel):
    """A typed torch view of one workspace region (for tests)."""
    off = view_ptr - ws.data_ptr()
    nbytes = numel * torch.empty((), dtype=dtype).element_size()
    return ws[off:off + nbytes].view(dtype)


# ---- Reference signatures (cuda/kernels.cuh argument lists, fp32 activations) ----

def ref_gemm_w4a16(x, qweight, scales, bias, y, group_size=128, stream=None):
    """gemm_w4a16 (cuda/kernels.cuh:50-52): y[n, out] = x[n, in] . W^T (+ bias), W from
    qweight [out, ceil(in/2)] u8 and fp32 scales [out, ceil(in/g)]."""
    n, in_ = x.shape
    out = qweight.shape[0]
    _need(x, torch.float32, n * in_, "x")
    _need(qweight, torch.uint8, out * ((in_ + 1) // 2), "qweight")
    _need(scales, torch.float32, out * ((in_ + group_size - 1) // group_size), "scales")
    _need(y, torch.float32, n * out, "y")
    check(lib().glmmoe_ref_gemm_w4a16(_p(x), _p(qweight), _p(scales), _p(bias), _p(y), n, in_, out,
                                      group_size, _s(stream)), "ref_gemm_w4a16")


def ref_gemm_fp8(x, w, w_scale, bias, y, stream=None):
    """gemm_fp8 (cuda/kernels.cuh:55-57): e4m3 W [out, in], optional fp32 scale per row."""
    n, in_ = x.shape
    out = w.shape[0]
    _need(x, torch.float32, n * in_, "x")
    _need(w, torch.uint8, out * in_, "w")
    _need(y, torch.float32, n * out, "y")
    check(lib().glmmoe_ref_gemm_fp8(_p(x), _p(w), _p(w_scale), _p(bias), _p(y), n, in_, out,
                                    _s(stream)), "ref_gemm_fp8")


def ref_silu_mul(g, u, out, stream=None):
    check(lib().glmmoe_ref_silu_mul(_p(g), _p(u), _p(out), g.numel(), _s(stream)), "ref_silu_mul")


def ref_add_inplace(y, x, stream=None):
    check(lib().glmmoe_ref_add_inplace(_p(y), _p(x), y.numel(), _s(stream)), "ref_add_inplace")


def ref_moe_expert_ffn(x, topk_ids, topk_weights, gate_w, up_w, down_w, out, stream=None):
    """moe_expert_ffn (cuda/kernels.cuh:252-257): fp32 experts gate/up [E, I, H], down
    [E, H, I]; out [n, H] overwritten."""
    n, H = x.shape
    E, I, _ = gate_w.shape
    k = topk_ids.shape[1]
    check(lib().glmmoe_ref_moe_expert_ffn(_p(x), _p(topk_ids), _p(topk_weights), _p(gate_w),
                                          _p(up_w), _p(down_w), n, k, H, I, E, _p(out),
                                          _s(stream)), "ref_moe_expert_ffn")


class RefW4Experts:
    """Reference-layout W4A16 routed experts registered with their packed copy, for
    glmmoe_ref_moe_expert_ffn_w4a16 (cuda/kernels.cuh:259-268 argument list)."""

    def __init__(self, gate_q, gate_s, up_q, up_s, down_q, down_s, hidden, moe_inter,
                 group_size=128):
        E = gate_q.shape[0]
        self.raw = (gate_q, gate_s, up_q, up_s, down_q, down_s)
        self.hidden, self.moe_inter, self.E, self.group_size = hidden, moe_inter, E, group_size
        self.packed = (pack_w4a16(gate_q, gate_s, E, moe_inter, hidden, group_size),
                       pack_w4a16(up_q, up_s, E, moe_inter, hidden, group_size),
                       pack_w4a16(down_q, down_s, E, hidden, moe_inter, group_size))
        st = Layer()
        st.hidden, st.moe_inter, st.n_experts, st.topk = hidden, moe_inter, E, 1
        st.gate_q, st.gate_s = _p(self.packed[0][0]), _p(self.packed[0][1])
        st.up_q, st.up_s = _p(self.packed[1][0]), _p(self.packed[1][1])
        st.down_q, st.down_s = _p(self.packed[2][0]), _p(self.packed[2][1])
        self.struct = st
        check(lib().glmmoe_ref_register_w4a16(_p(gate_q), _p(gate_s), _p(up_q), _p(up_s),
                                              _p(down_q), _p(down_s), ctypes.byref(st)),
              "ref_register_w4a16")

    def release(self):
        gq, gs, uq, us, dq, ds = self.raw
        check(lib().glmmoe_ref_unregister_w4a16(_p(gq), _p(gs), _p(uq), _p(us), _p(dq), _p(ds)),
              "ref_unregister_w4a16")

    def workspace_bytes(self, n, topk):
        return lib().glmmoe_ref_workspace_bytes(n, topk, self.hidden, self.moe_inter, self.E)

    @staticmethod
    def set_workspace(ws):
        check(lib().glmmoe_ref_set_workspace(_p(ws), 0 if ws is None else ws.numel()),
              "ref_set_workspace")

    def ffn(self, x, topk_ids, topk_weights, out, stream=None):
        n = x.shape[0]
        gq, gs, uq, us, dq, ds = self.raw
        check(lib().glmmoe_ref_moe_expert_ffn_w4a16(
            _p(x), _p(topk_ids), _p(topk_weights), _p(gq), _p(gs), _p(uq), _p(us), _p(dq), _p(ds),
            n, topk_ids.shape[1], self.hidden, self.moe_inter, self.E, self.group_size, _p(out),
            _s(stream)), "ref_moe_expert_ffn_w4a16")


def ref_gemm_q(qtype, x, qweight, bias, y, row_bytes, stream=None):
    """gemm_q (cuda/kernels.cuh:63-66): GGUF rows of W [out, in] at qweight + o * row_bytes."""
    n, in_ = x.shape
    out = y.shape[1]
    _need(x, torch.float32, n * in_, "x")
    _need(y, torch.float32, n * out, "y")
    check(lib().glmmoe_ref_gemm_q(qtype, _p(x), _p(qweight), _p(bias), _p(y), n, in_, out,
                                  row_bytes, _s(stream)), "ref_gemm_q")


def ref_moe_expert_ffn_q(types, x, topk_ids, topk_w, gate_q, up_q, down_q, moe_inter, E,
                         row_bytes, h_act, dpart, out, dispatch=None, stream=None):
    """moe_expert_ffn_q (cuda/kernels.cuh:117-123). types / row_bytes: (gate, up, down)."""
    n, H = x.shape
    k = topk_ids.shape[1]
    check(lib().glmmoe_ref_moe_expert_ffn_q(
        types[0], types[1], types[2], _p(x), _p(topk_ids), _p(topk_w), _p(gate_q), _p(up_q),
        _p(down_q), n, k, H, moe_inter, E, row_bytes[0], row_bytes[1], row_bytes[2], _p(h_act),
        _p(dpart), _p(out), _p(dispatch), None, _s(stream)), "ref_moe_expert_ffn_q")


def ref_qtype_has_i8(qtype):
    """qtype_has_i8 (cuda/kernels.cuh:74)."""
    return bool(lib().glmmoe_ref_qtype_has_i8(qtype))


def ref_quantize_act_q8(x, xq, xs, stream=None):
    """quantize_act_q8 (cuda/kernels.cuh:77-78): x [n, in] fp32 -> xq int8, xs [n, in/32]."""
    n, in_ = x.shape
    _need(x, torch.float32, n * in_, "x")
    _need(xq, torch.int8, n * in_, "xq")
    _need(xs, torch.float32, n * in_ // 32, "xs")
    check(lib().glmmoe_ref_quantize_act_q8(_p(x), n, in_, _p(xq), _p(xs), _s(stream)),
          "ref_quantize_act_q8")


def ref_gemm_q_i8(qtype, xq, xs, qweight, bias, y, row_bytes, stream=None):
    """gemm_q_i8 (cuda/kernels.cuh:81-83)."""
    n, in_ = xq.shape
    out = y.shape[1]
    _need(xq, torch.int8, n * in_, "xq")
    _need(xs, torch.float32, n * in_ // 32, "xs")
    _need(y, torch.float32, n * out, "y")
    check(lib().glmmoe_ref_gemm_q_i8(qtype, _p(xq), _p(xs), _p(qweight), _p(bias), _p(y), n, in_,
                                     out, row_bytes, _s(stream)), "ref_gemm_q_i8")


def ref_moe_expert_ffn_q_i8(types, xq, xs, topk_ids, topk_w, gate_q, up_q, down_q, moe_inter, E,
                            row_bytes, h_act, hq, hs, dpart, out, dispatch=None, stream=None):
    """moe_expert_ffn_q_i8 (cuda/kernels.cuh:128-135). types / row_bytes: (gate, up, down)."""
    n, H = xq.shape
    k = topk_ids.shape[1]
    _need(xq, torch.int8, n * H, "xq")
    _need(hq, torch.int8, n * k * moe_inter, "hq")
    _need(hs, torch.float32, n * k * moe_inter // 32, "hs")
    check(lib().glmmoe_ref_moe_expert_ffn_q_i8(
        types[0], types[1], types[2], _p(xq), _p(xs), _p(topk_ids), _p(topk_w), _p(gate_q),
        _p(up_q), _p(down_q), n, k, H, moe_inter, E, row_bytes[0], row_bytes[1], row_bytes[2],
        _p(h_act), _p(hq), _p(hs), _p(dpart), _p(out), _p(dispatch), None, _s(stream)),
        "ref_moe_expert_ffn_q_i8")
