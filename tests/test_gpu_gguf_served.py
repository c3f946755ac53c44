"""GGUF MoE parity at the served checkpoint's shape (H 6144, I 2048, E 256,
top-8; IQ3_XXS gate/up, IQ4_XS down: the types glmserve serves), for the fp32-
and int8-activation entry points (moe_expert_ffn_q / _i8, cuda/kernels.cuh:
116-136), at a decode batch (n = 64) and at n * topk = 2048 grouped rows, the
size from which the reference switches its MoE to tensor-core tiles
(GLMSERVE_MMA_MOE_MIN_TS, cuda/qgemm.cu:1563-1587).

The routing draws each token's 8 distinct experts from a fixed set of 24 of
the 256 (so the oracle dequantizes 24 experts, not 256; the kernels still
index the full E = 256 weight arrays). Every token is checked: the fp32 path
within 1e-4 of the oracle's fp32 forward on the dequantized weights (as the
small-shape tests), the int8 path within the reference's 3e-2
(tests/test_qgemm.cpp:351-352) of the same forward; grouped and token-major
runs of the int8 path are bit-identical below 2048 grouped rows, and within
1e-2 of each other from there (the grouped run then takes the matrix-core
kernels, whose h differs in fp32 rounding, which the int8 requantization of h
can turn into a code step; tests/test_gpu_gguf_i8.py checks that path link by
link against the oracle).
"""
import numpy as np
import pytest
import torch

from glmserve_amd import ops
from moe_cases import GGUF_TYPES, ORACLE_THREADS, random_gguf_rows, rel_err

pytestmark = pytest.mark.gpu
H, I, E, K = 6144, 2048, 256, 8
TYPES = (18, 18, 23)
USED = 24


def _row_bytes(qtype, n):
    be, bb, _ = GGUF_TYPES[qtype]
    return n // be * bb


RB = (_row_bytes(TYPES[0], H), _row_bytes(TYPES[1], H), _row_bytes(TYPES[2], I))


@pytest.fixture(scope="module")
def served(oracle):
    rng = np.random.default_rng(2024)
    used = np.sort(rng.choice(E, USED, replace=False))
    gq = torch.zeros(E * I, RB[0], dtype=torch.uint8, device="cuda")
    uq = torch.zeros(E * I, RB[1], dtype=torch.uint8, device="cuda")
    dq = torch.zeros(E * H, RB[2], dtype=torch.uint8, device="cuda")
    deq = {}
    for e in used:
        g = random_gguf_rows(TYPES[0], I, H, rng)
        u = random_gguf_rows(TYPES[1], I, H, rng)
        d = random_gguf_rows(TYPES[2], H, I, rng)
        gq[e * I:(e + 1) * I] = torch.from_numpy(g).cuda()
        uq[e * I:(e + 1) * I] = torch.from_numpy(u).cuda()
        dq[e * H:(e + 1) * H] = torch.from_numpy(d).cuda()
        deq[int(e)] = (oracle.gguf_dequant_rows(TYPES[0], g, I, H),
                       oracle.gguf_dequant_rows(TYPES[1], u, I, H),
                       oracle.gguf_dequant_rows(TYPES[2], d, H, I))
    torch.cuda.synchronize()
    return used, gq, uq, dq, deq


def _case(used, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, H)).astype(np.float32)
    ids = np.stack([rng.choice(used, K, replace=False) for _ in range(n)]).astype(np.int32)
    w = rng.uniform(0.05, 0.4, (n, K)).astype(np.float32)
    return x, ids, w


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n", [64, 256])
def test_served_shape_fp32_activations(oracle, served, n):
    used, gq, uq, dq, deq = served
    x, ids, w = _case(used, n, 10 + n)
    ref = oracle.moe_forward_streamed(x, ids, w, lambda e: deq[e], nthreads=ORACLE_THREADS)
    outs = []
    for grouped in (False, True):
        h_act = torch.empty(n * K * I, device="cuda")
        dpart = torch.empty(n * K * H, device="cuda")
        out = torch.full((n, H), float("nan"), device="cuda")
        disp = torch.full((3 * E + 1 + n * K,), -7, dtype=torch.int32, device="cuda") if grouped else None
        ops.ref_moe_expert_ffn_q(TYPES, _dev(x), _dev(ids), _dev(w), gq, uq, dq, I, E, RB, h_act,
                                 dpart, out, disp)
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        assert np.isfinite(o).all()
        assert rel_err(o, ref) < 1e-4, (grouped, rel_err(o, ref))
        outs.append(o)


@pytest.mark.parametrize("n", [64, 256])
def test_served_shape_int8_activations(oracle, served, n):
    used, gq, uq, dq, deq = served
    x, ids, w = _case(used, n, 20 + n)
    ref32 = oracle.moe_forward_streamed(x, ids, w, lambda e: deq[e], nthreads=ORACLE_THREADS)
    xq = torch.empty(n, H, dtype=torch.int8, device="cuda")
    xs = torch.empty(n, H // 32, device="cuda")
    ops.ref_quantize_act_q8(_dev(x), xq, xs)
    outs = []
    for grouped in (False, True):
        h_act = torch.empty(n * K, I, device="cuda")
        hq = torch.empty(n * K, I, dtype=torch.int8, device="cuda")
        hs = torch.empty(n * K, I // 32, device="cuda")
        dpart = torch.empty(n * K * H, device="cuda")
        out = torch.full((n, H), float("nan"), device="cuda")
        disp = torch.full((3 * E + 1 + n * K,), -7, dtype=torch.int32, device="cuda") if grouped else None
        ops.ref_moe_expert_ffn_q_i8(TYPES, xq, xs, _dev(ids), _dev(w), gq, uq, dq, I, E, RB, h_act, hq,
                                    hs, dpart, out, disp)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.isfinite(outs[0]).all()
    assert rel_err(outs[0], ref32) < 3e-2, rel_err(outs[0], ref32)
    if n * K < 2048:
        assert np.array_equal(outs[0], outs[1])
    else:
        # The grouped run takes the matrix-core kernels (exact int32 dots per
        # 32-block, fp32 sums in another order than the VALU kernels); the
        # requantization of h turns that into int8 flips of a few h values.
        assert rel_err(outs[1], outs[0]) < 1e-2
