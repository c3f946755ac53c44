"""GPU checks of the boundary's drop-in forms.

- glmmoe_moe_layer_w4a16_f32 takes run_layer_step's fp32 s.normed unchanged
  (src/model_gpu.cpp:1446-1494): its output must equal, bit for bit, the bf16
  layer's on the same rows rounded to bf16 (round to nearest even), at batch
  sizes that take each router path (rounding inside the small-batch router
  kernel up to 255 tokens, a conversion launch from 256) and each expert path.
- Zero-token calls are no-ops; moe_dispatch at n == 0 writes E + 1 zero
  offsets, as the reference's kernel does (cuda/moe_dispatch.cu:23-26).
"""
import numpy as np
import pytest
import torch

from moe_cases import SynthLayer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    return SynthLayer(6144, 256, 8, 2048, seed=1)


@pytest.mark.parametrize("n", [1, 8, 9, 64, 200, 300, 1024])
def test_f32_layer_bit_identical_to_bf16_layer(layer, n):
    L = layer
    g = torch.Generator(device="cuda")
    g.manual_seed(100 + n)
    xf = torch.randn(n, L.H, generator=g, device="cuda") * 1.7
    xb = xf.to(torch.bfloat16)   # round to nearest even
    outs = []
    for f32 in (True, False):
        ws = L.layer.alloc_workspace_f32(n) if f32 else L.layer.alloc_workspace(n)
        ws.fill_(0xFF)
        out = torch.full((n, L.H), float("nan"), dtype=torch.float32, device="cuda")
        if f32:
            L.layer.forward_f32(xf, out, ws)
        else:
            L.layer.forward(xb, out, ws)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1]), n


def test_zero_token_dispatch_writes_zero_offsets():
    from glmserve_amd import moe_dispatch
    E = 256
    offs = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda")
    ids = torch.empty(0, dtype=torch.int32, device="cuda")
    st = torch.empty(0, dtype=torch.int32, device="cuda")
    sr = torch.empty(0, dtype=torch.int32, device="cuda")
    moe_dispatch(ids, 0, 8, E, offs, st, sr)
    torch.cuda.synchronize()
    assert np.array_equal(offs.cpu().numpy(), np.zeros(E + 1, np.int32))


def test_zero_token_layer_leaves_output_untouched(layer):
    L = layer
    out = torch.full((4, L.H), 3.0, dtype=torch.float32, device="cuda")
    x = torch.empty(0, L.H, dtype=torch.bfloat16, device="cuda")
    ws = L.layer.alloc_workspace(1)
    L.layer.forward(x, out, ws)
    L.layer.forward_f32(x.float(), out, ws)
    torch.cuda.synchronize()
    assert torch.all(out == 3.0)
