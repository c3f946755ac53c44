"""GPU parity of the reference-signature entry points (cuda/kernels.cuh argument
lists, fp32 activations) against the CPU oracle.

gemm_w4a16 / gemm_fp8 / moe_expert_ffn compute in fp32 like the reference, so
they match an fp64 product of the oracle's dequantized weights to ~1e-5;
moe_expert_ffn_w4a16 runs the bf16 grouped kernels (x rounded to bf16, scales
packed as bf16) and is held to the W4A16 tolerance, 2e-2.
"""
import numpy as np
import pytest
import torch

from glmserve_amd import ops
from glmserve_amd._lib import GlmMoeError
from moe_cases import rel_err

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-5
TOL_W4A16 = 2e-2


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("n,in_,out,g,with_bias", [
    (1, 6144, 2048, 128, False),   # the shared expert's gate at decode
    (13, 2048, 6144, 128, True),   # its down projection, a ragged token block
    (9, 264, 40, 8, True),         # staged path, rows not a multiple of 16
    (3, 250, 37, 50, False),       # odd shapes: one K per lane step
])
def test_ref_gemm_w4a16(oracle, n, in_, out, g, with_bias):
    gen = _gen(in_ + out + n)
    q = torch.randint(0, 256, (out, (in_ + 1) // 2), dtype=torch.uint8, generator=gen)
    s = torch.rand(out, (in_ + g - 1) // g, generator=gen) * 0.02
    x = torch.randn(n, in_, generator=gen)
    b = torch.randn(out, generator=gen) if with_bias else None
    W = oracle.dequant_int4_rows(q.numpy(), s.numpy(), in_, g)
    ref = x.double().numpy() @ W.astype(np.float64).T
    if with_bias:
        ref += b.double().numpy()
    y = torch.full((n, out), float("nan"), device="cuda")
    ops.ref_gemm_w4a16(x.cuda(), q.cuda(), s.cuda(), None if b is None else b.cuda(), y, g)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), ref) < TOL_F32


@pytest.mark.parametrize("n,in_,out,with_scale", [
    (2, 6144, 512, True),
    (5, 200, 33, False),
    (3, 100, 20, True),            # in % 8 != 0: one K per lane step
])
def test_ref_gemm_fp8(oracle, n, in_, out, with_scale):
    gen = _gen(7 * in_ + out)
    w = torch.randint(0, 256, (out, in_), dtype=torch.uint8, generator=gen)
    w[(w == 0x7F) | (w == 0xFF)] = 0x3C   # the NaN codes are not weights
    sc = torch.rand(out, generator=gen) + 0.5 if with_scale else None
    x = torch.randn(n, in_, generator=gen)
    dec = np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float64)
    W = dec[w.numpy()]
    if with_scale:
        W = W * sc.double().numpy()[:, None]
    ref = x.double().numpy() @ W.T
    y = torch.full((n, out), float("nan"), device="cuda")
    ops.ref_gemm_fp8(x.cuda(), w.cuda(), None if sc is None else sc.cuda(), None, y)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), ref) < TOL_F32


def test_ref_silu_mul_and_add_inplace():
    gen = _gen(3)
    n = 100003
    g = torch.randn(n, generator=gen) * 4
    u = torch.randn(n, generator=gen)
    out = torch.empty(n, device="cuda")
    ops.ref_silu_mul(g.cuda(), u.cuda(), out)
    gd, ud = g.double(), u.double()
    ref = gd / (1 + torch.exp(-gd)) * ud
    torch.cuda.synchronize()
    assert torch.allclose(out.cpu().double(), ref, rtol=1e-6, atol=1e-7)
    y = torch.randn(n, generator=gen)
    yd = y.cuda()
    ops.ref_add_inplace(yd, u.cuda())
    torch.cuda.synchronize()
    assert torch.equal(yd.cpu(), y + u)


def _routing(oracle, n, E, k, seed):
    gen = np.random.default_rng(seed)
    logits = gen.standard_normal((n, E)).astype(np.float32)
    e_bias = gen.uniform(-0.1, 0.1, E).astype(np.float32)
    ids, w = oracle.router_topk(logits, e_bias, k, True, 2.5)
    return logits, e_bias, ids, w


def test_ref_moe_expert_ffn_fp32(oracle):
    # configs[0] geometry with fp32 experts (moe_expert_ffn, cuda/moe_expert.cu:32-130).
    H, I, E, k, n = 256, 128, 16, 4, 7
    gen = _gen(11)
    gate = torch.randn(E, I, H, generator=gen) * 0.02
    up = torch.randn(E, I, H, generator=gen) * 0.02
    down = torch.randn(E, H, I, generator=gen) * 0.02
    x = torch.randn(n, H, generator=gen)
    logits, eb, ids, w = _routing(oracle, n, E, k, 5)
    ref, rids, rw = oracle.moe_forward(x.numpy(), E, k, list(gate.numpy()), list(up.numpy()),
                                       list(down.numpy()), None, logits=logits, e_bias=eb,
                                       norm_topk=True, routed_scale=2.5)
    assert np.array_equal(rids, ids)
    out = torch.full((n, H), float("nan"), device="cuda")
    ops.ref_moe_expert_ffn(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                           gate.cuda(), up.cuda(), down.cuda(), out)
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), ref) < 1e-4


@pytest.mark.parametrize("H,I,E,k,n", [
    (256, 128, 16, 4, 64),     # configs[0]: the LDS-ring decode kernels
    (2048, 512, 8, 4, 5),      # streaming gate/up (16 K-groups), ring down
])
def test_ref_moe_expert_ffn_w4a16(oracle, H, I, E, k, n):
    # The reference's argument list and weight layout (cuda/kernels.cuh:259-268):
    # raw qweight / fp32 scales, registered once with their packed copy.
    gen = _gen(H + I + n)
    def raw(rows, K):
        q = torch.randint(0, 256, (E, rows, K // 2), dtype=torch.uint8, generator=gen)
        s = torch.rand(E, rows, K // 128, generator=gen) * 0.01 + 1e-3
        return q, s
    (gq, gs), (uq, us), (dq, ds) = raw(I, H), raw(I, H), raw(H, I)
    dev = [t.cuda() for t in (gq, gs, uq, us, dq, ds)]
    experts = ops.RefW4Experts(*dev, hidden=H, moe_inter=I)
    x = torch.randn(n, H, generator=gen)
    logits, eb, ids, w = _routing(oracle, n, E, k, 9)
    out = torch.full((n, H), float("nan"), device="cuda")
    ids_d, w_d = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    try:
        ops.RefW4Experts.set_workspace(None)
        with pytest.raises(GlmMoeError):
            experts.ffn(x.cuda(), ids_d, w_d, out)      # no workspace registered
        ws = torch.empty(experts.workspace_bytes(n, k), dtype=torch.uint8, device="cuda")
        ops.RefW4Experts.set_workspace(ws)
        experts.ffn(x.cuda(), ids_d, w_d, out)
        torch.cuda.synchronize()
    finally:
        ops.RefW4Experts.set_workspace(None)
        experts.release()
    with pytest.raises(GlmMoeError):
        experts.ffn(x.cuda(), ids_d, w_d, out)          # no longer registered
    deq = lambda q, s, K: [oracle.dequant_int4_rows(q[e].numpy(), s[e].numpy(), K, 128)
                           for e in range(E)]
    ref, rids, _ = oracle.moe_forward(x.numpy(), E, k, deq(gq, gs, H), deq(uq, us, H),
                                      deq(dq, ds, I), None, logits=logits, e_bias=eb,
                                      norm_topk=True, routed_scale=2.5)
    assert np.array_equal(rids, ids)
    assert rel_err(out.cpu().numpy(), ref) < TOL_W4A16
