"""GPU parity of the FP8 path against the CPU oracle.

Activation quantization (codes and scales) must be bit-exact; routing and
dispatch bit-exact; the layer output within 4e-2 of the oracle's fp32 forward
on dequantized weights with the same activation / h quantization rule
(metric: max|gpu - oracle| / max|oracle|).
"""
import numpy as np
import pytest
import torch

from moe_cases import SynthFp8Layer, bits_to_f32, oracle_full_fp8, rel_err
from test_gpu_layer import _check_routing, _ws_f32, _ws_i32

pytestmark = pytest.mark.gpu
TOL_FP8 = 4e-2


def _special_rows(K):
    """Rows exercising the quantizer's edge cases, one per 128-channel group."""
    rows = np.zeros((4, K), np.float32)
    g = 0
    # all-zero group (scale 1, codes 0) is group 0 of row 0.
    # amax exactly 448 -> scale 1: RNE ties between e4m3 neighbours.
    ties = np.array([448.0, 1.0625, 1.1875, -1.0625, 0.0078125 * 1.5, 0.0029296875, 17.0, 272.0],
                    np.float32)
    rows[0, 128:128 + len(ties)] = ties
    # huge and tiny magnitudes in one group; negative zero.
    rows[1, :4] = [3.0e4, -1.0e-3, 2.5e-6, -0.0]
    # values landing in the e4m3 subnormal range after scaling.
    rows[2, 256:384] = np.linspace(-1e-3, 1e-3, 128, dtype=np.float32)
    rows[2, 300] = 1.0
    # constant group (every element equals amax -> all codes 448).
    rows[3, 512:640] = -0.75
    return rows


def test_quant_act_bit_exact(oracle):
    from glmserve_amd import quant_act_fp8
    K = 6144
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    x = torch.randn(300, K, generator=g, device="cuda").to(torch.bfloat16)
    sp = torch.from_numpy(_special_rows(K)).to(torch.bfloat16).cuda()
    x = torch.cat([x, sp])
    q, s = quant_act_fp8(x)
    torch.cuda.synchronize()
    xf = bits_to_f32(x.view(torch.int16).cpu().numpy().view(np.uint16))
    rq, rs = oracle.quant_act_e4m3(xf)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32)), "scales"
    assert np.array_equal(q.cpu().numpy(), rq), "codes"
    assert not np.any((rq & 0x7F) == 0x7F)


def _check_full(out, ref):
    assert np.isfinite(out).all(), "every output element written and finite"
    assert rel_err(out, ref) < TOL_FP8


def _run(L, n, seed):
    x = L.x(n, seed)
    ws = L.layer.alloc_workspace(n)
    out = torch.empty(n, L.H, dtype=torch.float32, device="cuda")
    L.layer.forward(x, out, ws)
    torch.cuda.synchronize()
    v = L.layer.workspace_view(n, ws)
    logits = _ws_f32(ws, v.logits, n * L.E).view(n, L.E).cpu().numpy()
    ids = _ws_i32(ws, v.topk_ids, n * L.k).view(n, L.k).cpu().numpy()
    w = _ws_f32(ws, v.topk_w, n * L.k).view(n, L.k).cpu().numpy()
    offs = _ws_i32(ws, v.expert_offsets, L.E + 1).cpu().numpy()
    st = _ws_i32(ws, v.sorted_token_ids, n * L.k).cpu().numpy()
    sr = _ws_i32(ws, v.sorted_row, n * L.k).cpu().numpy()
    return x, out, ws, logits, ids, w, offs, st, sr


@pytest.mark.parametrize("n", [1, 7, 64, 300, 1500])
def test_fp8_tiny(oracle, n):
    # configs[0] geometry with FP8 experts; at 1500 tokens every expert has
    # several 128-row tiles, which run in expert-major item order.
    L = SynthFp8Layer(256, 16, 4, 128, seed=12)
    x, out, ws, logits, ids, w, offs, st, sr = _run(L, n, seed=8)
    ref_logits = _check_routing(oracle, L, x, logits, ids, w, offs, st, sr)
    ref, _, _ = L.oracle_forward(oracle, x, np.arange(n), ref_logits)
    _check_full(out.cpu().numpy(), ref)


@pytest.fixture(scope="module")
def fp8_full():
    return SynthFp8Layer(6144, 256, 8, 2048, seed=5)


def test_fp8_prefill_full_shape(oracle, fp8_full):
    # 8192 tokens, FP8 e4m3 experts with 128 x 128 block scales.
    L = fp8_full
    n = 8192
    x, out, ws, logits, ids, w, offs, st, sr = _run(L, n, seed=9)
    _check_routing(oracle, L, x, logits, ids, w, offs, st, sr)
    # every token against the oracle (experts streamed through it one at a time)
    _check_full(out.cpu().numpy(), oracle_full_fp8(L, oracle, x, ids, w))
    # The expert-FFN entry on the layer's own routing reproduces it bit for bit.
    v = L.layer.workspace_view(n, ws)
    ids_t = _ws_i32(ws, v.topk_ids, n * L.k).clone()
    w_t = _ws_f32(ws, v.topk_w, n * L.k).clone()
    ws2 = L.layer.alloc_workspace(n)
    out2 = torch.empty_like(out)
    L.layer.expert_ffn(x, ids_t, w_t, out2, ws2)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_fp8_decode_sizes(oracle, fp8_full):
    # Small batches run on the same 128-row tiles (mostly padding rows).
    L = fp8_full
    for n in (1, 33):
        x, out, ws, logits, ids, w, offs, st, sr = _run(L, n, seed=10 + n)
        _check_routing(oracle, L, x, logits, ids, w, offs, st, sr)
        _check_full(out.cpu().numpy(), oracle_full_fp8(L, oracle, x, ids, w))
