"""Checkpoint ingestion (glmserve_amd/checkpoint.py): the converter's W4
quantizer (tools/convert_hf_to_glmserve.py:229-247), the W4 safetensors layout
read back layer by layer (src/model_glm52.cpp:157-196, 278-301), and a layer
built from such a file run on the GPU against the oracle."""
import os

import numpy as np
import pytest
import torch

from glmserve_amd.checkpoint import dequant_w4, quantize_w4, read_layer


def test_quantize_w4_known_answer():
    # Row 0, group 0: max |x| = 7 -> s = 1, q = rint(x) + 8 with ties to even.
    # Row 0, group 1: all zero -> s = 1.0, every nibble 8.
    # Row 1, group 0: max |x| = 14 -> s = 2; -16 / 2 = -8 (the clip edge), 5 / 2 = 2.5 -> 2.
    # Row 1, group 1: max |x| = 0.7 -> s = 0.1; 0.7 / 0.1 = 7 (well, 6.99.. or 7.00..) -> 7.
    w = torch.zeros(2, 256)
    w[0, 0:6] = torch.tensor([7.0, -7.0, 3.5, -3.49, 0.0, 2.5])
    w[1, 0:4] = torch.tensor([14.0, -14.0, 5.0, -3.0])
    w[1, 128:130] = torch.tensor([0.7, -0.35])
    q, s = quantize_w4(w)
    assert q.dtype == torch.uint8 and tuple(q.shape) == (2, 128)
    assert s.dtype == torch.float32 and tuple(s.shape) == (2, 2)
    assert s[0, 0] == 1.0 and s[0, 1] == 1.0 and s[1, 0] == 2.0
    assert abs(float(s[1, 1]) - 0.1) < 1e-7
    nib = lambda r, c: int((q[r, c // 2] >> (4 * (c % 2))) & 0xF)
    # 7 -> 15, -7 -> 1, 3.5 -> 4 (even) -> 12, -3.49 -> -3 -> 5, 0 -> 8, 2.5 -> 2 -> 10
    assert [nib(0, c) for c in range(6)] == [15, 1, 12, 5, 8, 10]
    assert all(nib(0, c) == 8 for c in range(128, 256))
    # 14 -> 7 -> 15, -14 -> -7 -> 1, 5 -> 2.5 -> 2 -> 10, -3 -> -1.5 -> -2 -> 6
    assert [nib(1, c) for c in range(4)] == [15, 1, 10, 6]
    assert nib(1, 128) == 15 and nib(1, 129) in (4, 5)   # -0.35 / 0.1 = -3.5 -> -4 (even)
    # even column in the low nibble
    assert int(q[0, 0]) == 15 | (1 << 4)


def test_quantize_dequant_round_trip():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(64, 512, generator=g) * 0.05
    q, s = quantize_w4(w)
    d = dequant_w4(q, s)
    step = s.repeat_interleave(128, dim=1)
    # |w - dq| <= s / 2 except where the clip at -8 binds (x / s < -8.5 never
    # happens: |x| <= 7 s).
    assert torch.all((w - d).abs() <= step / 2 + 1e-7)
    # the group maximum is represented exactly: |x| = 7 s -> nibble 15 or 1
    amax = w.view(64, 4, 128).abs().amax(2)
    assert torch.allclose(amax, s * 7.0)


def _write_checkpoint(path, H=256, I=128, E=4, layer=3, seed=5, float_experts=(2,)):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)
    p = f"model.layers.{layer}."
    t = {p + "mlp.gate.weight": (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16),
         p + "mlp.gate.e_score_correction_bias": torch.rand(E, generator=g) * 0.2 - 0.1}
    full = {}
    def lin(base, rows, K, as_float):
        w = 0.02 * torch.randn(rows, K, generator=g)
        full[base] = w
        if as_float:
            t[base + ".weight"] = w.to(torch.bfloat16)
            full[base] = w.to(torch.bfloat16).float()
        else:
            q, s = quantize_w4(w)
            t[base + ".qweight"], t[base + ".scales"] = q, s
    for e in range(E):
        for name, rows, K in (("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)):
            lin(p + f"mlp.experts.{e}.{name}", rows, K, e in float_experts)
    for name, rows, K in (("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)):
        lin(p + f"mlp.shared_experts.{name}", rows, K, False)
    os.makedirs(path, exist_ok=True)
    # two shards, so the lookup crosses files
    keys = sorted(t)
    save_file({k: t[k].contiguous() for k in keys[: len(keys) // 2]}, os.path.join(path, "a.safetensors"))
    save_file({k: t[k].contiguous() for k in keys[len(keys) // 2:]}, os.path.join(path, "b.safetensors"))
    with open(os.path.join(path, "config.json"), "w") as f:
        f.write('{"num_experts_per_tok": 2, "norm_topk_prob": true, "routed_scaling_factor": 1.5}')
    return t, full


def test_read_layer_layout(tmp_path):
    t, full = _write_checkpoint(str(tmp_path))
    r = read_layer(str(tmp_path), 3)
    assert (r["hidden"], r["moe_inter"], r["n_experts"]) == (256, 128, 4)
    assert r["config"]["num_experts_per_tok"] == 2
    p = "model.layers.3."
    assert torch.equal(r["router_w"], t[p + "mlp.gate.weight"].float())
    assert torch.equal(r["e_bias"], t[p + "mlp.gate.e_score_correction_bias"])
    gq, gs = r["gate"]
    assert tuple(gq.shape) == (4, 128, 128) and tuple(gs.shape) == (4, 128, 2)
    # a W4 expert is copied as stored
    assert torch.equal(gq[1], t[p + "mlp.experts.1.gate_proj.qweight"])
    assert torch.equal(gs[1], t[p + "mlp.experts.1.gate_proj.scales"])
    # a float expert is quantized with the converter's rule
    q2, s2 = quantize_w4(t[p + "mlp.experts.2.down_proj.weight"])
    dq, ds = r["down"]
    assert torch.equal(dq[2], q2) and torch.equal(ds[2], s2)
    sq, ss = r["shared"][2]
    assert tuple(sq.shape) == (1, 256, 64)


@pytest.mark.gpu
def test_load_layer_matches_oracle(tmp_path, oracle):
    from glmserve_amd.checkpoint import load_layer
    from moe_cases import bits_to_f32, rel_err
    t, full = _write_checkpoint(str(tmp_path))
    L = load_layer(str(tmp_path), 3)
    n, H, E, k = 5, 256, 4, 2
    x = (torch.randn(n, H, generator=torch.Generator().manual_seed(9))).to(torch.bfloat16)
    xd = x.cuda()
    ws = L.alloc_workspace(n)
    out = torch.empty(n, H, dtype=torch.float32, device="cuda")
    L.forward(xd, out, ws)
    torch.cuda.synchronize()
    r = read_layer(str(tmp_path), 3)
    deq = lambda qs, e: oracle.dequant_int4_rows(qs[0][e].numpy(), qs[1][e].numpy(),
                                                 qs[0].shape[2] * 2, 128)
    gate = [deq(r["gate"], e) for e in range(E)]
    up = [deq(r["up"], e) for e in range(E)]
    down = [deq(r["down"], e) for e in range(E)]
    sh = [deq(r["shared"][i], 0) for i in range(3)]
    xf = bits_to_f32(x.view(torch.int16).numpy().view(np.uint16))
    wr = bits_to_f32(r["router_w"].to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    ref, _, _ = oracle.moe_forward(xf, E, k, gate, up, down, sh, router_w=wr,
                             e_bias=r["e_bias"].numpy(), norm_topk=True, routed_scale=1.5)
    assert rel_err(out.cpu().numpy(), ref) < 2e-2


def test_quantize_w4_matches_oracle(oracle):
    # The oracle restates the converter in C (orc_quantize_w4_rows, itself pinned
    # against the reference's golden cases in test_oracle.py); the product's
    # torch quantizer must give the same bytes and scales. The division x / s
    # rounds the same way in both (one IEEE fp32 division).
    g = torch.Generator().manual_seed(11)
    w = torch.randn(33, 1024, generator=g) * 0.03
    w[5, 128:256] = 0.0                      # an all-zero group
    w[7, 3] = 1.0                            # a large outlier
    q, s = quantize_w4(w)
    rq, rs = oracle.quantize_w4_rows(w.numpy(), 128)
    assert np.array_equal(q.numpy(), rq)
    assert np.array_equal(s.numpy().view(np.uint32), rs.view(np.uint32))
    d = dequant_w4(q, s).numpy()
    assert np.array_equal(d, oracle.dequant_int4_rows(rq, rs, 1024, 128))
