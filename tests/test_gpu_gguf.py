"""GPU parity of the GGUF weight paths (gemm_q, moe_expert_ffn_q signatures)
against the CPU oracle, whose block decode is pinned bit-for-bit against the
reference's dequantizer (tests/test_oracle.py).

One-hot activations make each output a single weight (exact in fp32), so the
in-kernel decode is checked bit for bit; dense inputs are held to 1e-5 of an
fp64 product of the oracle's dequantized weights (fp32 sums, another order),
and the MoE layer to 1e-4 of the oracle's fp32 forward.
"""
import numpy as np
import pytest
import torch

from glmserve_amd import ops
from moe_cases import GGUF_TYPES, random_gguf_rows, rel_err

pytestmark = pytest.mark.gpu
TYPES = sorted(GGUF_TYPES)


def _row_bytes(qtype, n):
    be, bb, _ = GGUF_TYPES[qtype]
    return n // be * bb


@pytest.mark.parametrize("qtype", TYPES)
def test_gemm_q_decode_bit_exact(oracle, qtype):
    rng = np.random.default_rng(300 + qtype)
    in_, out = 512, 24
    w = random_gguf_rows(qtype, out, in_, rng)
    W = oracle.gguf_dequant_rows(qtype, w, out, in_)
    ks = np.concatenate([np.arange(0, 256), np.arange(256, 512, 7)])   # every block position
    x = np.zeros((len(ks), in_), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    y = torch.empty(len(ks), out, device="cuda")
    ops.ref_gemm_q(qtype, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), None, y,
                   _row_bytes(qtype, in_))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    # exact values (a weight that decodes to -0.0 comes back as +0.0 = 0 + 1 * w)
    assert np.isfinite(got).all() and np.array_equal(got, W[:, ks].T)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("in_", [1024, 1280])    # 1280: a partial last K chunk
def test_gemm_q_dense(oracle, qtype, in_):
    rng = np.random.default_rng(400 + qtype + in_)
    n, out = 11, 40
    w = random_gguf_rows(qtype, out, in_, rng)
    W = oracle.gguf_dequant_rows(qtype, w, out, in_).astype(np.float64)
    x = rng.standard_normal((n, in_)).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32)
    y = torch.full((n, out), float("nan"), device="cuda")
    ops.ref_gemm_q(qtype, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(),
                   torch.from_numpy(b).cuda(), y, _row_bytes(qtype, in_))
    torch.cuda.synchronize()
    ref = x.astype(np.float64) @ W.T + b
    assert rel_err(y.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("types", [(18, 18, 23), (12, 12, 14), (8, 8, 8), (11, 13, 0)])
@pytest.mark.parametrize("grouped", [False, True])
def test_moe_expert_ffn_q(oracle, types, grouped):
    # gate/up [E, I, H], down [E, H, I] of the given GGUF types; (18, 18, 23) is
    # the served checkpoint's IQ3_XXS gate/up + IQ4_XS down; (11, 13, 0) has
    # gate and up of different types.
    H, I, E, k, n = 512, 256, 8, 4, 6
    rng = np.random.default_rng(sum(types) + 7 * grouped)
    gq = random_gguf_rows(types[0], E * I, H, rng)
    uq = random_gguf_rows(types[1], E * I, H, rng)
    dq = random_gguf_rows(types[2], E * H, I, rng)
    deq = lambda t, q, rows, K: [oracle.gguf_dequant_rows(t, q[e * rows:(e + 1) * rows], rows, K)
                                 for e in range(E)]
    G, U, D = deq(types[0], gq, I, H), deq(types[1], uq, I, H), deq(types[2], dq, H, I)
    x = rng.standard_normal((n, H)).astype(np.float32)
    logits = rng.standard_normal((n, E)).astype(np.float32)
    eb = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    ref, ids, w = oracle.moe_forward(x, E, k, G, U, D, None, logits=logits, e_bias=eb,
                                     norm_topk=True, routed_scale=2.5)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    h_act = torch.empty(n * k * I, device="cuda")
    dpart = torch.empty(n * k * H, device="cuda")
    out = torch.full((n, H), float("nan"), device="cuda")
    disp = torch.full((3 * E + 1 + n * k,), -7, dtype=torch.int32, device="cuda") if grouped else None
    ops.ref_moe_expert_ffn_q(types, dev(x), dev(ids), dev(w), dev(gq), dev(uq), dev(dq), I, E,
                             (_row_bytes(types[0], H), _row_bytes(types[1], H),
                              _row_bytes(types[2], I)), h_act, dpart, out, disp)
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), ref) < 1e-4


@pytest.mark.parametrize("grouped", [False, True])
def test_moe_expert_ffn_q_out_of_range_ids(oracle, grouped):
    # Slots routed to an id outside [0, E) add nothing, in the ungrouped path
    # (one tile per routed row) as in the grouped one: the output equals the
    # oracle's with those slots' weights set to zero.
    types = (18, 18, 23)
    H, I, E, k, n = 512, 256, 8, 4, 40
    rng = np.random.default_rng(77 + grouped)
    gq = random_gguf_rows(types[0], E * I, H, rng)
    uq = random_gguf_rows(types[1], E * I, H, rng)
    dq = random_gguf_rows(types[2], E * H, I, rng)
    deq = lambda t, q, rows, K: [oracle.gguf_dequant_rows(t, q[e * rows:(e + 1) * rows], rows, K)
                                 for e in range(E)]
    G, U, D = deq(types[0], gq, I, H), deq(types[1], uq, I, H), deq(types[2], dq, H, I)
    x = rng.standard_normal((n, H)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (n, k)).astype(np.float32)
    bad = rng.random((n, k)) < 0.2
    ids_bad = np.where(bad, np.where(rng.random((n, k)) < 0.5, -1, E), ids).astype(np.int32)
    ref = oracle.moe_forward_streamed(x, ids, np.where(bad, 0.0, w).astype(np.float32),
                                      lambda e: (G[e], U[e], D[e]))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    h_act = torch.empty(n * k * I, device="cuda")
    dpart = torch.empty(n * k * H, device="cuda")
    out = torch.full((n, H), float("nan"), device="cuda")
    disp = torch.full((3 * E + 1 + n * k,), -7, dtype=torch.int32, device="cuda") if grouped else None
    ops.ref_moe_expert_ffn_q(types, dev(x), dev(ids_bad), dev(w), dev(gq), dev(uq), dev(dq), I, E,
                             (_row_bytes(types[0], H), _row_bytes(types[1], H),
                              _row_bytes(types[2], I)), h_act, dpart, out, disp)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, ref) < 1e-4


def test_gemm_q_unaligned_rows(oracle):
    # Q8_0 rows of 3 blocks (102 B) are not 4-byte aligned: the byte-load decode
    # serves them (the streamed kernels need dword-aligned rows).
    rng = np.random.default_rng(5)
    n, in_, out = 3, 96, 21
    w = random_gguf_rows(8, out, in_, rng)
    W = oracle.gguf_dequant_rows(8, w, out, in_).astype(np.float64)
    x = rng.standard_normal((n, in_)).astype(np.float32)
    y = torch.full((n, out), float("nan"), device="cuda")
    ops.ref_gemm_q(8, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), None, y,
                   _row_bytes(8, in_))
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), x.astype(np.float64) @ W.T) < 1e-5
