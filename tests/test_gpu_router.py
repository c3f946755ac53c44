"""GPU routing and dispatch through the reference-named entry points
(moe_router / moe_dispatch, cuda/kernels.cuh:243-250), bit-exact vs the oracle."""
import numpy as np
import pytest
import torch

import glmserve_amd as G

pytestmark = pytest.mark.gpu


def _route(logits, bias, k, norm=True, scale=2.5):
    n, E = logits.shape
    lg = torch.from_numpy(logits).cuda()
    b = None if bias is None else torch.from_numpy(bias).cuda()
    ids = torch.empty(n, k, dtype=torch.int32, device="cuda")
    w = torch.empty(n, k, dtype=torch.float32, device="cuda")
    G.moe_router(lg, b, n, E, k, norm, scale, ids, w)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy()


CASES = [
    # (n, E, k, norm, scale, bias) -- the reference test's shape first
    # (tests/test_moe_router.cpp:19-25: n=7, E=32, topk=4, norm, x2.5).
    (7, 32, 4, True, 2.5, "normal"),
    (64, 16, 4, True, 2.5, "uniform"),
    (64, 256, 8, True, 2.5, "uniform"),
    (33, 256, 8, False, 1.0, None),
    (5, 100, 8, True, 2.5, "uniform"),    # E not a multiple of 64
    (9, 512, 8, True, 2.5, "uniform"),    # largest supported E
    (3, 8, 8, True, 2.5, "uniform"),      # topk == E
    (1, 1, 1, True, 2.5, None),
]


@pytest.mark.parametrize("n,E,k,norm,scale,bias", CASES)
def test_router_matches_oracle(oracle, n, E, k, norm, scale, bias):
    rng = np.random.default_rng(n * 1000 + E)
    logits = rng.standard_normal((n, E)).astype(np.float32)
    b = None
    if bias == "normal":
        b = (0.05 * rng.standard_normal(E)).astype(np.float32)
    elif bias == "uniform":
        b = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    ids, w = _route(logits, b, k, norm, scale)
    rid, rw = oracle.router_topk(logits, b, k, norm, scale)
    assert np.array_equal(ids, rid)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))


def test_router_ties_and_specials(oracle):
    n, E, k = 6, 64, 8
    logits = np.zeros((n, E), np.float32)            # all scores equal -> lowest ids
    logits[1, ::7] = 3.0                             # ties among the raised ones
    logits[2] = -200.0                               # saturated scores, wsum tiny
    logits[3, 5] = np.nan                            # NaN never beats a number
    logits[4] = np.linspace(-1, 1, E, dtype=np.float32)[::-1]
    logits[5] = 1e30                                 # saturated high
    bias = np.zeros(E, np.float32)
    bias[10] = 0.5                                   # bias flips selection but not weight
    ids, w = _route(logits, bias, k)
    rid, rw = oracle.router_topk(logits, bias, k)
    assert np.array_equal(ids, rid)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert ids[0, 0] == 10 and list(ids[0, 1:]) == list(range(7))


@pytest.mark.parametrize("n,k,E,mode", [(1, 8, 256, "rand"), (64, 8, 256, "rand"),
                                        (4096, 8, 256, "rand"), (520, 8, 256, "skew"),
                                        (100, 4, 16, "one"), (37, 3, 5, "rand"),
                                        (8192, 8, 256, "rand")])
def test_dispatch_matches_oracle(oracle, n, k, E, mode):
    rng = np.random.default_rng(n + k + E)
    if mode == "rand":
        ids = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    elif mode == "skew":
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        p /= p.sum()
        ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(n)]).astype(np.int32)
    else:  # every token on the same experts
        ids = np.tile(np.arange(k, dtype=np.int32), (n, 1))
    d_ids = torch.from_numpy(ids).cuda()
    off = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda")
    st = torch.full((n * k,), -7, dtype=torch.int32, device="cuda")
    sr = torch.full((n * k,), -7, dtype=torch.int32, device="cuda")
    G.moe_dispatch(d_ids, n, k, E, off, st, sr)
    torch.cuda.synchronize()
    roff, rst, rsr = oracle.dispatch(ids, E)
    assert np.array_equal(off.cpu().numpy(), roff)
    assert np.array_equal(st.cpu().numpy(), rst)
    assert np.array_equal(sr.cpu().numpy(), rsr)


def test_router_logits_bit_exact(oracle):
    from moe_cases import bf16_bits
    rng = np.random.default_rng(5)
    # (n >= 256 with H % 128 == 0 runs the LDS-tiled kernel; the rest the small-batch one)
    for n, H, E in [(1, 6144, 256), (13, 6144, 256), (64, 256, 16), (3, 1000, 7), (37, 8192, 300),
                    (9, 6144, 1), (300, 6144, 256), (260, 8192, 300), (512, 256, 16), (257, 1024, 5),
                    (300, 1000, 7)]:
        x = bf16_bits(rng.standard_normal((n, H)))
        w = bf16_bits(0.02 * rng.standard_normal((E, H)))
        dx = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
        dw = torch.from_numpy(w.view(np.int16)).cuda().view(torch.bfloat16)
        lg = torch.empty(n, E, dtype=torch.float32, device="cuda")
        xs = torch.empty(n, max(1, H // 128), dtype=torch.float32, device="cuda") if H % 128 == 0 else None
        G.router_logits(dx, dw, lg, xs)
        torch.cuda.synchronize()
        ref = oracle.router_logits_bf16(x, w)
        assert np.array_equal(lg.cpu().numpy().view(np.uint32), ref.view(np.uint32)), (n, H, E)
        if xs is not None:
            # group sums: ascending sequential fp32 sum of each 128-channel group
            xf = (x.astype(np.uint32) << 16).view(np.float32).reshape(n, H // 128, 128)
            rx = np.cumsum(xf, axis=2, dtype=np.float32)[:, :, -1]
            assert np.array_equal(xs.cpu().numpy().view(np.uint32), rx.view(np.uint32)), (n, H)


def test_router_logits_f32_bit_exact(oracle):
    # gemm_fp32-shaped entry: fp32 x and W rounded to bf16 in the kernel, then
    # the fixed order; bit-exact vs the oracle's bf16 logits of the rounded
    # inputs, and + bias exactly as one fp32 add.
    rng = np.random.default_rng(11)
    for n, H, E in [(1, 6144, 256), (8, 6144, 256), (64, 6144, 256), (300, 6144, 256),
                    (5, 256, 16), (17, 8192, 300), (3, 128, 1)]:
        x = rng.standard_normal((n, H)).astype(np.float32)
        w = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
        x[0, :3] = [1.0 + 2.0 ** -8, -(1.0 + 3 * 2.0 ** -9), 3.4e38]   # ties to even; rounds up to inf
        bias = rng.uniform(-0.1, 0.1, E).astype(np.float32)
        dx, dw = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
        y = torch.full((n, E), float("nan"), dtype=torch.float32, device="cuda")
        yb = torch.full((n, E), float("nan"), dtype=torch.float32, device="cuda")
        G.router_logits_f32(dx, dw, None, y)
        G.router_logits_f32(dx, dw, torch.from_numpy(bias).cuda(), yb)
        torch.cuda.synchronize()
        ref = oracle.router_logits_bf16(oracle.f32_to_bf16(x), oracle.f32_to_bf16(w))
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (n, H, E)
        assert np.array_equal(yb.cpu().numpy().view(np.uint32), (ref + bias[None, :]).view(np.uint32)), (n, H, E)


@pytest.mark.parametrize("n", [256, 520, 1000, 4096])
def test_layer_routing_bit_exact_large_batches(oracle, n):
    """From 256 tokens the layer routes with MFMA logits plus an exact
    fixed-order recompute of every expert that can reach the top-k; ids,
    weights and the activation group sums must still equal the oracle's bit
    for bit. Duplicate router rows force exact ties between experts. The
    dispatch (one workgroup below 4096 ids, chunked from there) must give
    the stable counting sort."""
    from moe_cases import SynthLayer
    from glmserve_amd.ops import ws_tensor
    H, E, k, I = 1024, 64, 8, 128
    L = SynthLayer(H, E, k, I, seed=11)
    L.router_w[5] = L.router_w[3]
    L.router_w[40] = L.router_w[3]
    L.router_w[63] = L.router_w[17]
    x = L.x(n, seed=n)
    ws = L.layer.alloc_workspace(n)
    out = torch.empty(n, H, dtype=torch.float32, device="cuda")
    L.layer.forward(x, out, ws)
    torch.cuda.synchronize()
    v = L.layer.workspace_view(n, ws)
    ids = ws_tensor(None, v.topk_ids, ws, torch.int32, n * k).cpu().numpy().reshape(n, k)
    w = ws_tensor(None, v.topk_w, ws, torch.float32, n * k).cpu().numpy().reshape(n, k)
    xs = ws_tensor(None, v.xsum, ws, torch.float32, n * (H // 128)).cpu().numpy()
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    wb = L.router_w.view(torch.int16).cpu().numpy().view(np.uint16)
    logits = oracle.router_logits_bf16(xb, wb)
    rid, rw = oracle.router_topk(logits, L.e_bias.cpu().numpy(), k, True, 2.5)
    assert np.array_equal(ids, rid)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    xf = (xb.astype(np.uint32) << 16).view(np.float32).reshape(n, H // 128, 128)
    rx = np.cumsum(xf, axis=2, dtype=np.float32)[:, :, -1].reshape(-1)
    assert np.array_equal(xs.view(np.uint32), rx.view(np.uint32))
    offs = ws_tensor(None, v.expert_offsets, ws, torch.int32, E + 1).cpu().numpy()
    st = ws_tensor(None, v.sorted_token_ids, ws, torch.int32, n * k).cpu().numpy()
    flat = rid.reshape(-1)
    order = np.argsort(flat, kind="stable")
    assert np.array_equal(st, (order // k).astype(np.int32))
    ref_offs = np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]).astype(np.int32)
    assert np.array_equal(offs, ref_offs)


@pytest.mark.parametrize("H,E,k,n", [(1024, 64, 8, 1), (2048, 100, 6, 37), (8192, 512, 8, 9),
                                     (6144, 256, 8, 255), (6144, 256, 8, 64), (256, 16, 4, 8),
                                     (768, 40, 4, 17)])
def test_layer_routing_bit_exact_small_batches(oracle, H, E, k, n):
    """Below 256 tokens the layer's routing kernels (up to 8 tokens the
    router kernel plus the gate/up prologue; from 9 the chunk-partials
    kernel plus the fold / select / dispatch kernel). ids, weights, the
    activation group sums and the dispatch must equal the oracle's bit for
    bit, with duplicated router rows forcing exact ties, E not a multiple of
    64, E = 512 and the largest hidden size. From 9 tokens the logits come
    from per-chunk partials folded in a second kernel; they are compared
    too."""
    from moe_cases import SynthLayer
    from glmserve_amd.ops import ws_tensor
    L = SynthLayer(H, E, k, 128, seed=12)
    L.router_w[5] = L.router_w[3]
    L.router_w[E - 1] = L.router_w[3]
    x = L.x(n, seed=n + 3)
    ws = L.layer.alloc_workspace(n)
    ws.fill_(0xFF)
    out = torch.empty(n, H, dtype=torch.float32, device="cuda")
    L.layer.forward(x, out, ws)
    torch.cuda.synchronize()
    v = L.layer.workspace_view(n, ws)
    ids = ws_tensor(None, v.topk_ids, ws, torch.int32, n * k).cpu().numpy().reshape(n, k)
    w = ws_tensor(None, v.topk_w, ws, torch.float32, n * k).cpu().numpy().reshape(n, k)
    xs = ws_tensor(None, v.xsum, ws, torch.float32, n * (H // 128)).cpu().numpy()
    offs = ws_tensor(None, v.expert_offsets, ws, torch.int32, E + 1).cpu().numpy()
    st = ws_tensor(None, v.sorted_token_ids, ws, torch.int32, n * k).cpu().numpy()
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    wb = L.router_w.view(torch.int16).cpu().numpy().view(np.uint16)
    logits = oracle.router_logits_bf16(xb, wb)
    rid, rw = oracle.router_topk(logits, L.e_bias.cpu().numpy(), k, True, 2.5)
    lg = ws_tensor(None, v.logits, ws, torch.float32, n * E).cpu().numpy().reshape(n, E)
    assert np.array_equal(lg.view(np.uint32), logits.view(np.uint32))
    assert np.array_equal(ids, rid)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    xf = (xb.astype(np.uint32) << 16).view(np.float32).reshape(n, H // 128, 128)
    rx = np.cumsum(xf, axis=2, dtype=np.float32)[:, :, -1].reshape(-1)
    assert np.array_equal(xs.view(np.uint32), rx.view(np.uint32))
    # Stable counting sort of the (token, slot) rows by expert.
    flat = rid.reshape(-1)
    order = np.argsort(flat, kind="stable")
    assert np.array_equal(st, (order // k).astype(np.int32))
    ref_offs = np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]).astype(np.int32)
    assert np.array_equal(offs, ref_offs)


@pytest.mark.parametrize("n", [1, 9, 64, 300])
def test_route_entry_bit_exact(oracle, n):
    """glmmoe_moe_route_w4a16 (the router GEMM + top-k alone, no dispatch)
    through each routing path: the small-batch kernels (1 token), the chunk
    GEMV and fold / select kernels (9, 64) and the MFMA pass with the exact
    refinement (300). ids and weights equal the oracle's bit for bit, with
    duplicated router rows forcing exact ties."""
    from moe_cases import SynthLayer
    H, E, k = 6144, 256, 8
    L = SynthLayer(H, E, k, 2048, seed=21)
    L.router_w[7] = L.router_w[2]
    L.router_w[200] = L.router_w[2]
    x = L.x(n, seed=5 * n + 1)
    ws = L.layer.alloc_workspace(n)
    ws.fill_(0xFF)
    ids = torch.full((n, k), -1, dtype=torch.int32, device="cuda")
    w = torch.full((n, k), float("nan"), dtype=torch.float32, device="cuda")
    L.layer.route(x, ids, w, ws)
    torch.cuda.synchronize()
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    wb = L.router_w.view(torch.int16).cpu().numpy().view(np.uint16)
    logits = oracle.router_logits_bf16(xb, wb)
    rid, rw = oracle.router_topk(logits, L.e_bias.cpu().numpy(), k, True, 2.5)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
