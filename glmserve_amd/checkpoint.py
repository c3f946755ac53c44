"""Checkpoint ingestion: one MoE layer of a glmserve W4 safetensors checkpoint
onto the device as a W4A16MoELayer.

The W4 format is the one `tools/convert_hf_to_glmserve.py:216-252` writes and
`src/model_glm52.cpp:157-196` reads:
  ``<linear>.qweight``  U8  [out, in/2]   two nibbles per byte, column 2j in the
                                          low nibble, value = nibble - 8
  ``<linear>.scales``   F32 [out, in/g]   per-row, per-group scales
so w[r, c] = (nibble(r, c) - 8) * scales[r, c / g], with g = in / groups.

Names of MoE layer i (prefix p = "model.layers.{i}."), as `load_layer`
looks them up (`src/model_glm52.cpp:278-301`):
  router   p + "mlp.gate" or p + "mlp.router"                 [E, H] (any float dtype)
  bias     p + "mlp.gate.e_score_correction_bias" or p + "mlp.e_score_correction_bias"
  experts  p + "mlp.experts.{e}.{gate,up,down}_proj"         W4 (or float, quantized here)
  shared   p + "mlp.shared_experts.*" or p + "mlp.shared_expert.*"   (optional)
Routing constants come from config.json (num_experts_per_tok, norm_topk_prob,
routed_scaling_factor, `src/config.cpp:60-68`) or keyword arguments.

Files are read with safetensors' own loader (no pickled objects are ever
loaded). Expert weights stored as plain float tensors are quantized with
`quantize_w4`, the converter's rule.
"""
import json
import os

import torch

from ._lib import GlmMoeError
from .ops import W4A16MoELayer, pack_w4a16

GROUP = 128   # the int4 group size the kernels take


def quantize_w4(w, group=GROUP):
    """The converter's W4 quantizer (tools/convert_hf_to_glmserve.py:229-247):
    per row and group s = max|x| / 7 (1.0 for an all-zero group), q = clip(rint(x / s), -8, 7)
    + 8, two columns per byte (even column in the low nibble). Returns (qweight u8
    [out, in/2], scales fp32 [out, in/g]) on w's device."""
    w = w.float()
    out, K = w.shape
    if K % group or K % 2:
        raise GlmMoeError(f"quantize_w4: in_features {K} must be a multiple of {group}")
    x = w.view(out, K // group, group)
    s = x.abs().amax(dim=2) / 7.0
    s = torch.where(s > 0, s, torch.ones_like(s))
    q = torch.clamp(torch.round(x / s[:, :, None]), -8, 7).to(torch.int16) + 8
    q = q.view(out, K).to(torch.uint8)
    packed = q[:, 0::2] | (q[:, 1::2] << 4)
    return packed.contiguous(), s.contiguous()


def dequant_w4(qweight, scales):
    """fp32 weights of a W4 linear (src/tensor.cpp:53-63 semantics)."""
    out = qweight.shape[0]
    K = qweight.shape[1] * 2
    g = K // scales.shape[1]
    q = torch.empty(out, K, dtype=torch.int16, device=qweight.device)
    q[:, 0::2] = (qweight & 0xF).to(torch.int16)
    q[:, 1::2] = (qweight >> 4).to(torch.int16)
    return (q.float() - 8.0) * scales.float().repeat_interleave(g, dim=1)


class _Store:
    """Tensor lookup over one file, several shards or a directory of them."""

    def __init__(self, path):
        from safetensors import safe_open
        if os.path.isdir(path):
            files = sorted(os.path.join(path, f) for f in os.listdir(path)
                           if f.endswith(".safetensors"))
            cfg = os.path.join(path, "config.json")
            self.config = json.load(open(cfg)) if os.path.exists(cfg) else {}
        else:
            files = [path]
            self.config = {}
        if not files:
            raise GlmMoeError(f"no .safetensors files under {path}")
        self._where = {}
        self._handles = []
        for f in files:
            h = safe_open(f, framework="pt", device="cpu")
            self._handles.append(h)
            for name in h.keys():
                self._where[name] = h

    def has(self, name):
        return name in self._where

    def get(self, name):
        if name not in self._where:
            raise GlmMoeError(f"missing tensor: {name}")
        return self._where[name].get_tensor(name)


def _linear_w4(st, base, rows, K):
    """(qweight u8 [rows, K/2], scales fp32 [rows, K/g]) of one linear, quantizing a
    float `.weight` on the way."""
    if st.has(base + ".qweight"):
        q = st.get(base + ".qweight")
        s = st.get(base + ".scales").float()
        if q.dtype != torch.uint8 or tuple(q.shape) != (rows, K // 2):
            raise GlmMoeError(f"{base}.qweight: expected U8 [{rows}, {K // 2}], got "
                              f"{q.dtype} {list(q.shape)}")
        if s.dim() != 2 or s.shape[0] != rows or K % s.shape[1] or K // s.shape[1] != GROUP:
            raise GlmMoeError(f"{base}.scales: expected [{rows}, {K // GROUP}] (group {GROUP}), "
                              f"got {list(s.shape)}")
        return q, s
    w = st.get(base + ".weight")
    if tuple(w.shape) != (rows, K):
        raise GlmMoeError(f"{base}.weight: expected [{rows}, {K}], got {list(w.shape)}")
    return quantize_w4(w)


def read_layer(path, layer, hidden=None, moe_inter=None, n_experts=None):
    """Host tensors of MoE layer `layer`: dict with router_w [E, H] fp32, e_bias [E]
    fp32 or None, gate/up/down = (q [E, rows, K/2] u8, s [E, rows, K/g] fp32), shared =
    the same triple for the shared expert (E = 1) or None, and config."""
    st = _Store(path) if not isinstance(path, _Store) else path
    p = f"model.layers.{layer}."
    rname = p + "mlp.gate" if (st.has(p + "mlp.gate.weight") or st.has(p + "mlp.gate.qweight")) \
        else p + "mlp.router"
    if st.has(rname + ".qweight"):
        router = dequant_w4(st.get(rname + ".qweight"), st.get(rname + ".scales").float())
    else:
        router = st.get(rname + ".weight").float()
    E, H = router.shape
    if n_experts is not None and n_experts != E:
        raise GlmMoeError(f"router has {E} experts, expected {n_experts}")
    if hidden is not None and hidden != H:
        raise GlmMoeError(f"router width {H}, expected hidden {hidden}")
    e_bias = None
    for bn in (p + "mlp.gate.e_score_correction_bias", p + "mlp.e_score_correction_bias"):
        if st.has(bn):
            e_bias = st.get(bn).float()
            break
    # moe_inter from the first expert's gate projection.
    g0 = p + "mlp.experts.0.gate_proj"
    I = moe_inter or (st.get(g0 + ".qweight").shape[0] if st.has(g0 + ".qweight")
                      else st.get(g0 + ".weight").shape[0])

    def stack(prefixes, rows, K):
        qs, ss = zip(*[_linear_w4(st, pre, rows, K) for pre in prefixes])
        return torch.stack(qs).contiguous(), torch.stack(ss).contiguous()

    ex = [p + f"mlp.experts.{e}." for e in range(E)]
    gate = stack([e + "gate_proj" for e in ex], I, H)
    up = stack([e + "up_proj" for e in ex], I, H)
    down = stack([e + "down_proj" for e in ex], H, I)
    shared = None
    for sb in (p + "mlp.shared_experts.", p + "mlp.shared_expert."):
        if st.has(sb + "gate_proj.qweight") or st.has(sb + "gate_proj.weight"):
            shared = (stack([sb + "gate_proj"], I, H), stack([sb + "up_proj"], I, H),
                      stack([sb + "down_proj"], H, I))
            break
    return dict(router_w=router, e_bias=e_bias, gate=gate, up=up, down=down, shared=shared,
                hidden=H, moe_inter=I, n_experts=E, config=st.config)


def load_layer(path, layer, topk=None, norm_topk=None, routed_scale=None, device="cuda"):
    """W4A16MoELayer for MoE layer `layer` of a checkpoint: one .safetensors file,
    or a directory of shards with config.json. Routing constants default to
    config.json, else to top-8 / normalized / 2.5. The router weights are used in
    bf16 (the layer's router GEMM is bf16 x bf16 in a fixed fp32 order)."""
    t = read_layer(path, layer)
    cfg = t["config"]
    topk = topk if topk is not None else int(cfg.get("num_experts_per_tok", 8))
    norm_topk = norm_topk if norm_topk is not None else bool(cfg.get("norm_topk_prob", True))
    routed_scale = routed_scale if routed_scale is not None else float(
        cfg.get("routed_scaling_factor", 2.5))
    H, I, E = t["hidden"], t["moe_inter"], t["n_experts"]
    if t["shared"] is not None and t["shared"][0][0].shape[1] != I:
        raise GlmMoeError("shared expert intermediate size must equal moe_intermediate_size")

    def dev_pack(qs, rows, K):
        q, s = qs
        return pack_w4a16(q.to(device), s.to(device), q.shape[0], rows, K, GROUP)

    gate = dev_pack(t["gate"], I, H)
    up = dev_pack(t["up"], I, H)
    down = dev_pack(t["down"], H, I)
    shared = None
    if t["shared"] is not None:
        shared = (dev_pack(t["shared"][0], I, H), dev_pack(t["shared"][1], I, H),
                  dev_pack(t["shared"][2], H, I))
    router_w = t["router_w"].to(torch.bfloat16).to(device).contiguous()
    e_bias = t["e_bias"].to(device).contiguous() if t["e_bias"] is not None else None
    return W4A16MoELayer(H, I, E, topk, router_w, e_bias, gate, up, down, shared,
                         norm_topk=norm_topk, routed_scale=routed_scale)
