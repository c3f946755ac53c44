"""GPU parity of the GGUF int8-activation twins (quantize_act_q8, gemm_q_i8,
moe_expert_ffn_q_i8; cuda/kernels.cuh:68-83, 124-135) against the CPU oracle.

quantize_act_q8 is compared bit for bit. gemm_q_i8 is held to 1e-5 of the
oracle's fp64 sum of the same integer fragment products (fp32 in the kernel),
and to the reference's own 2e-2 gate against the fp32 product
(tests/test_qgemm.cpp:130-153). The MoE layer is checked link by link: h_act
against the oracle's int8 gate/up, hq / hs bit for bit against the oracle's
quantizer applied to that h_act, out against the oracle's int8 down and
slot-order combine; then against the fp32 layer within the reference's 3e-2
(tests/test_qgemm.cpp:351-352), and the expert-grouped run equal to the
token-major one.
"""
import numpy as np
import pytest
import torch

from glmserve_amd import ops
from glmserve_amd._lib import GlmMoeError
from moe_cases import GGUF_TYPES, random_gguf_rows, rel_err

pytestmark = pytest.mark.gpu
I8_TYPES = [8, 11, 12, 13, 14, 18, 23]


def _row_bytes(qtype, n):
    be, bb, _ = GGUF_TYPES[qtype]
    return n // be * bb


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _quant(x):
    n, k = x.shape
    xq = torch.empty(n, k, dtype=torch.int8, device="cuda")
    xs = torch.empty(n, k // 32, device="cuda")
    ops.ref_quantize_act_q8(x, xq, xs)
    return xq, xs


def test_qtype_has_i8():
    assert [t for t in range(40) if ops.ref_qtype_has_i8(t)] == I8_TYPES


@pytest.mark.parametrize("n,in_", [(1, 32), (3, 96), (7, 6144), (33, 2048)])
def test_quantize_act_q8_bit_exact(oracle, n, in_):
    rng = np.random.default_rng(n * 1000 + in_)
    x = (rng.standard_normal((n, in_)) * rng.uniform(1e-3, 30, (n, 1))).astype(np.float32)
    x[0, :32] = 0.0                                   # an all-zero block
    if in_ >= 64:
        x[-1, 32:64] = np.float32(2.5) * np.arange(-16, 16, dtype=np.float32)  # ties
    xq, xs = _quant(_dev(x))
    torch.cuda.synchronize()
    q, s = oracle.quant_act_q8(x)
    assert np.array_equal(xq.cpu().numpy(), q)
    assert np.array_equal(xs.cpu().numpy(), s)


@pytest.mark.parametrize("qtype", I8_TYPES)
@pytest.mark.parametrize("n", [1, 5, 13])
def test_gemm_q_i8(oracle, qtype, n):
    rng = np.random.default_rng(700 + qtype + n)
    in_, out = 1024, 40
    w = random_gguf_rows(qtype, out, in_, rng)
    x = rng.standard_normal((n, in_)).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32)
    xq, xs = _quant(_dev(x))
    y = torch.full((n, out), float("nan"), device="cuda")
    ops.ref_gemm_q_i8(qtype, xq, xs, _dev(w), _dev(b), y, _row_bytes(qtype, in_))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle.gemm_q_i8(qtype, xq.cpu().numpy(), xs.cpu().numpy(), w, out,
                           _row_bytes(qtype, in_)) + b
    assert rel_err(got, ref) < 1e-5
    W = oracle.gguf_dequant_rows(qtype, w, out, in_).astype(np.float64)
    assert rel_err(got, x.astype(np.float64) @ W.T + b) < 2e-2


def test_i8_rejects():
    x = torch.zeros(2, 48, device="cuda")
    with pytest.raises(GlmMoeError):
        _quant(x)                                     # in % 32 != 0
    xq = torch.zeros(2, 256, dtype=torch.int8, device="cuda")
    xs = torch.zeros(2, 8, device="cuda")
    w = torch.zeros(4, 256 * 2, dtype=torch.uint8, device="cuda")
    y = torch.empty(2, 4, device="cuda")
    with pytest.raises(GlmMoeError):
        ops.ref_gemm_q_i8(1, xq, xs, w, None, y, 512)   # F16 has no int8 form


def _silu(v):
    # exp(-v) overflows to inf for v < -88 in float32, which gives the right
    # limit (v / inf = -0); the warning it raises is expected.
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("types,n", [((18, 18, 23), 6), ((12, 12, 14), 6), ((8, 8, 8), 6),
                                     ((11, 13, 12), 6), ((18, 18, 23), 20)])
def test_moe_expert_ffn_q_i8(oracle, types, n):
    # n = 20: 80 routed rows over 8 experts, so the grouped run uses 8-row tiles
    H, I, E, k = 512, 256, 8, 4
    rng = np.random.default_rng(sum(types) + 99)
    gq = random_gguf_rows(types[0], E * I, H, rng)
    uq = random_gguf_rows(types[1], E * I, H, rng)
    dq = random_gguf_rows(types[2], E * H, I, rng)
    rb = (_row_bytes(types[0], H), _row_bytes(types[1], H), _row_bytes(types[2], I))
    x = rng.standard_normal((n, H)).astype(np.float32)
    logits = rng.standard_normal((n, E)).astype(np.float32)
    eb = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    deq = lambda t, q, rows, K: [oracle.gguf_dequant_rows(t, q[e * rows:(e + 1) * rows], rows, K)
                                 for e in range(E)]
    ref32, ids, w = oracle.moe_forward(x, E, k, deq(types[0], gq, I, H), deq(types[1], uq, I, H),
                                       deq(types[2], dq, H, I), None, logits=logits, e_bias=eb,
                                       norm_topk=True, routed_scale=2.5)
    xq, xs = _quant(_dev(x))
    outs = []
    for grouped in (False, True):
        h_act = torch.empty(n * k, I, device="cuda")
        hq = torch.empty(n * k, I, dtype=torch.int8, device="cuda")
        hs = torch.empty(n * k, I // 32, device="cuda")
        dpart = torch.empty(n * k * H, device="cuda")
        out = torch.full((n, H), float("nan"), device="cuda")
        disp = (torch.full((3 * E + 1 + n * k,), -7, dtype=torch.int32, device="cuda")
                if grouped else None)
        ops.ref_moe_expert_ffn_q_i8(types, xq, xs, _dev(ids), _dev(w), _dev(gq), _dev(uq),
                                    _dev(dq), I, E, rb, h_act, hq, hs, dpart, out, disp)
        torch.cuda.synchronize()
        outs.append((h_act.cpu().numpy(), hq.cpu().numpy(), hs.cpu().numpy(),
                     out.cpu().numpy()))
    h_g, hq_g, hs_g, out_g = outs[0]
    # link 1: gate/up from the oracle's int8 sums
    xq_h, xs_h = xq.cpu().numpy(), xs.cpu().numpy()
    h_ref = np.empty((n * k, I))
    for r in range(n * k):
        e, t = ids.reshape(-1)[r], r // k
        g = oracle.gemm_q_i8(types[0], xq_h[t:t + 1], xs_h[t:t + 1], gq[e * I:(e + 1) * I], I,
                             rb[0])[0]
        u = oracle.gemm_q_i8(types[1], xq_h[t:t + 1], xs_h[t:t + 1], uq[e * I:(e + 1) * I], I,
                             rb[1])[0]
        h_ref[r] = _silu(g) * u
    assert rel_err(h_g, h_ref) < 1e-5
    # link 2: the requantization of h_act
    q, s = oracle.quant_act_q8(h_g)
    assert np.array_equal(hq_g, q) and np.array_equal(hs_g, s)
    # link 3: down on (hq, hs) and the slot-order combine
    ref = np.zeros((n, H))
    for r in range(n * k):
        e, t = ids.reshape(-1)[r], r // k
        y = oracle.gemm_q_i8(types[2], hq_g[r:r + 1], hs_g[r:r + 1], dq[e * H:(e + 1) * H], H,
                             rb[2])[0]
        ref[t] += w.reshape(-1)[r] * y
    assert rel_err(out_g, ref) < 1e-5
    assert rel_err(out_g, ref32) < 3e-2
    # grouped tiles: per row the same sums in the same order
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)


def test_gemm_q_i8_unaligned_rows(oracle):
    # Q8_0 rows of 3 blocks (102 B) are not 4-byte aligned: the byte-load decode
    # serves them.
    rng = np.random.default_rng(6)
    n, in_, out = 5, 96, 19
    w = random_gguf_rows(8, out, in_, rng)
    x = rng.standard_normal((n, in_)).astype(np.float32)
    xq, xs = _quant(_dev(x))
    y = torch.full((n, out), float("nan"), device="cuda")
    ops.ref_gemm_q_i8(8, xq, xs, _dev(w), None, y, _row_bytes(8, in_))
    torch.cuda.synchronize()
    ref = oracle.gemm_q_i8(8, xq.cpu().numpy(), xs.cpu().numpy(), w, out, _row_bytes(8, in_))
    assert rel_err(y.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("types", [(18, 18, 23), (8, 8, 8), (23, 23, 18)])
def test_moe_expert_ffn_q_i8_matrix_cores(oracle, types):
    # n * topk = 2048 routed rows with the grouping scratch: the matrix-core
    # phases (v_mfma_i32_32x32x32_i8 per 32-block, then the fp32 rescale; the
    # reference's tensor-core policy, cuda/qgemm.cu:1563-1587) on the types
    # whose scale is uniform over each 32-block. Link by link as above:
    # h_act against the oracle's fp64 sums of the same integer products
    # (1e-5), (hq, hs) bit for bit against the oracle's quantizer of that
    # h_act, out against the oracle's int8 down and slot-order combine (1e-5);
    # then the fp32 layer within 3e-2, and the token-major run (no grouping:
    # the VALU kernels): h_act within 1e-5, the output within 1e-2 (after the
    # requantization of h, see below).
    H, I, E, k, n = 512, 256, 8, 4, 512
    rng = np.random.default_rng(sum(types) + 123)
    gq = random_gguf_rows(types[0], E * I, H, rng)
    uq = random_gguf_rows(types[1], E * I, H, rng)
    dq = random_gguf_rows(types[2], E * H, I, rng)
    rb = (_row_bytes(types[0], H), _row_bytes(types[1], H), _row_bytes(types[2], I))
    x = rng.standard_normal((n, H)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (n, k)).astype(np.float32)
    deq = lambda t, q, rows, K: [oracle.gguf_dequant_rows(t, q[e * rows:(e + 1) * rows], rows, K)
                                 for e in range(E)]
    G, U, D = deq(types[0], gq, I, H), deq(types[1], uq, I, H), deq(types[2], dq, H, I)
    ref32 = oracle.moe_forward_streamed(x, ids, w, lambda e: (G[e], U[e], D[e]))
    xq, xs = _quant(_dev(x))
    outs = []
    for grouped in (True, False):
        h_act = torch.full((n * k, I), float("nan"), device="cuda")
        hq = torch.empty(n * k, I, dtype=torch.int8, device="cuda")
        hs = torch.empty(n * k, I // 32, device="cuda")
        dpart = torch.empty(n * k * H, device="cuda")
        out = torch.full((n, H), float("nan"), device="cuda")
        disp = (torch.full((3 * E + 1 + n * k,), -7, dtype=torch.int32, device="cuda")
                if grouped else None)
        ops.ref_moe_expert_ffn_q_i8(types, xq, xs, _dev(ids), _dev(w), _dev(gq), _dev(uq),
                                    _dev(dq), I, E, rb, h_act, hq, hs, dpart, out, disp)
        torch.cuda.synchronize()
        outs.append((h_act.cpu().numpy(), hq.cpu().numpy(), hs.cpu().numpy(),
                     out.cpu().numpy()))
    h_g, hq_g, hs_g, out_g = outs[0]
    assert np.isfinite(h_g).all() and np.isfinite(out_g).all()
    xq_h, xs_h = xq.cpu().numpy(), xs.cpu().numpy()
    flat = ids.reshape(-1)
    h_ref = np.empty((n * k, I))
    for e in range(E):
        rows = np.nonzero(flat == e)[0]
        t = rows // k
        g = oracle.gemm_q_i8(types[0], xq_h[t], xs_h[t], gq[e * I:(e + 1) * I], I, rb[0])
        u = oracle.gemm_q_i8(types[1], xq_h[t], xs_h[t], uq[e * I:(e + 1) * I], I, rb[1])
        h_ref[rows] = _silu(g) * u
    assert rel_err(h_g, h_ref) < 1e-5
    q, s = oracle.quant_act_q8(h_g)
    assert np.array_equal(hq_g, q) and np.array_equal(hs_g, s)
    ref = np.zeros((n, H))
    for e in range(E):
        rows = np.nonzero(flat == e)[0]
        y = oracle.gemm_q_i8(types[2], hq_g[rows], hs_g[rows], dq[e * H:(e + 1) * H], H, rb[2])
        for j, r in enumerate(rows):
            ref[r // k] += w.reshape(-1)[r] * y[j]
    assert rel_err(out_g, ref) < 1e-5
    assert rel_err(out_g, ref32) < 3e-2
    # Across the two paths h_act differs by fp32 summation order (~1e-7), which
    # moves a few h values across an int8 rounding boundary when h is
    # requantized; each path is exact against the oracle given its own h.
    assert rel_err(outs[1][0], h_g) < 1e-5
    assert rel_err(outs[1][3], out_g) < 1e-2
