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
