"""Range safety of the expert paths, checked per token against the oracle.

The large-group W4A16 kernels (from 1024 grouped rows) compute on fp16
operands: x rows carry a power-of-2 scale, the intermediate h rows a
power-of-2 exponent per row, and the weight scales a fixed power-of-2 factor,
so activations and weights far outside the N(0, 1) / 0.01 magnitudes of the
other tests stay in fp16's normal range. The reference keeps h in fp32
(cuda/moe_expert.cu:143-222), so these batches must give finite outputs
within tolerance for every token, including tokens whose |h| exceeds fp16's
65504 and tokens whose |h| stays below 1e-5.

Metric: per token t, max|gpu_t - oracle_t| / max|oracle_t| (the global
metric of the other tests normalizes by the batch's largest output, which
hides a small token's error).
"""
import numpy as np
import pytest
import torch

from moe_cases import (SynthFp8Layer, SynthLayer, bits_to_f32, oracle_full_fp8, oracle_full_w4,
                       rel_err)

pytestmark = pytest.mark.gpu
TOL_W4A16 = 2e-2
TOL_FP8 = 4e-2
BIG, TINY = 200.0, 2e-4


def _row_rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.max(np.abs(got - ref), axis=1) / np.maximum(1e-300, np.max(np.abs(ref), axis=1))


def _outlier_batch(L, n, seed):
    """x N(0, 1) with every 7th token scaled by BIG and every 11th (not 7th) by
    TINY; returns x and the indices of both sets."""
    x = L.x(n, seed).float()
    big = np.arange(0, n, 7)
    tiny = np.array([t for t in range(3, n, 11) if t % 7])
    x[big] *= BIG
    x[tiny] *= TINY
    return x.to(torch.bfloat16), big, tiny


def _uniform_routing(L, n, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    ids = torch.rand(n, L.E, generator=g, device="cuda").topk(L.k, dim=1).indices
    w = (0.1 + torch.rand(n, L.k, generator=g, device="cuda") * 0.5).contiguous()
    return ids.to(torch.int32).contiguous(), w


def _h_extremes(L, oracle, x, ids, t_big, t_tiny):
    """max|h| of token t_big's and t_tiny's first routed expert (oracle
    arithmetic: fp32 dot products on the dequantized weights)."""
    out = []
    for t in (t_big, t_tiny):
        gt, up, _ = L.dequant_expert(oracle, int(ids[t, 0]))
        xf = bits_to_f32(x[t].view(torch.int16).cpu().numpy().view(np.uint16))
        g = gt @ xf
        u = up @ xf
        sig = 0.5 * (1.0 + np.tanh(0.5 * g))   # logistic, no overflow
        out.append(float(np.max(np.abs(g * sig * u))))
    return out


@pytest.fixture(scope="module")
def layer():
    return SynthLayer(6144, 256, 8, 2048, seed=1)


@pytest.mark.parametrize("n", [1024, 64])
def test_w4a16_outlier_rows_per_token(oracle, layer, n):
    # n = 1024: 9216 grouped rows, the large-group (fp16) kernels; n = 64:
    # the decode kernels (bf16 h), the same tokens for comparison.
    L = layer
    x, big, tiny = _outlier_batch(L, n, 5)
    ids, w = _uniform_routing(L, n, 6)
    ws = L.layer.alloc_workspace(n)
    out = torch.full((n, L.H), float("nan"), dtype=torch.float32, device="cuda")
    L.layer.expert_ffn(x, ids, w, out, ws)
    torch.cuda.synchronize()
    idn, wn = ids.cpu().numpy(), w.cpu().numpy()
    hb, ht = _h_extremes(L, oracle, x, idn, big[0], tiny[0])
    assert hb > 65504.0 and ht < 1e-5, (hb, ht)
    o = out.cpu().numpy()
    ref = oracle_full_w4(L, oracle, x, idn, wn)
    assert np.isfinite(o).all(), "every output finite"
    r = _row_rel_err(o, ref)
    worst = int(np.argmax(r))
    assert r.max() < TOL_W4A16, (worst, float(r[worst]), worst in big, worst in tiny)
    assert rel_err(o, ref) < TOL_W4A16


@pytest.mark.parametrize("n", [1024, 64])
def test_w4a16_small_weight_scales_per_token(oracle, n):
    # Every down-projection scale times 1e-4 (bf16 scales of about 1e-6,
    # below fp16's normal range 2^-14 / 2 = 3e-5 for the decode factor 2s):
    # the large-group kernels' weight decode stays exact.
    L = SynthLayer(6144, 256, 8, 2048, seed=8, down_scale_mul=1e-4)
    x = L.x(n, 9)
    ids, w = _uniform_routing(L, n, 10)
    ws = L.layer.alloc_workspace(n)
    out = torch.full((n, L.H), float("nan"), dtype=torch.float32, device="cuda")
    L.layer.expert_ffn(x, ids, w, out, ws)
    torch.cuda.synchronize()
    idn, wn = ids.cpu().numpy(), w.cpu().numpy()
    o = out.cpu().numpy()
    ref = oracle_full_w4(L, oracle, x, idn, wn)
    assert np.isfinite(o).all()
    assert _row_rel_err(o, ref).max() < TOL_W4A16


def test_fp8_outlier_rows_per_token(oracle):
    # The FP8 layer quantizes x and h per token and 128 channels with fp32
    # scales, so the same outlier tokens stay within its tolerance per token.
    L = SynthFp8Layer(6144, 256, 8, 2048, seed=3)
    n = 1024
    x, big, tiny = _outlier_batch(L, n, 7)
    ids, w = _uniform_routing(L, n, 8)
    ws = L.layer.alloc_workspace(n)
    out = torch.full((n, L.H), float("nan"), dtype=torch.float32, device="cuda")
    L.layer.expert_ffn(x, ids, w, out, ws)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    ref = oracle_full_fp8(L, oracle, x, ids.cpu().numpy(), w.cpu().numpy())
    assert np.isfinite(o).all()
    r = _row_rel_err(o, ref)
    worst = int(np.argmax(r))
    assert r.max() < TOL_FP8, (worst, float(r[worst]), worst in big, worst in tiny)
