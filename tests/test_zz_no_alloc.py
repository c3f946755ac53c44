"""The no-allocation layer entry (glmmoe_moe_layer_w4a16_noalloc) against the
workspace entry (glmmoe_moe_layer_w4a16) through the C-ABI: the same kernels
on the library's per-GPU scratch, so the outputs are bit-identical. Two calls
in a row, the second with a smaller batch, so the second runs on what the
first left in the scratch."""
import pytest
import torch

from glmserve_amd import _lib
from moe_cases import SynthLayer

pytestmark = pytest.mark.gpu


def test_noalloc_matches_workspace_entry():
    L = SynthLayer(6144, 256, 8, 2048, seed=5)
    for n in (64, 8):
        x = L.x(n, 40 + n)
        ref = torch.full((n, L.H), float("nan"), dtype=torch.float32, device="cuda")
        L.layer.forward(x, ref, L.layer.alloc_workspace(n))
        got = torch.full((n, L.H), float("nan"), dtype=torch.float32, device="cuda")
        L.layer.forward_noalloc(x, got)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all(), n
        assert torch.equal(got, ref), n
    # A batch whose workspace does not fit the scratch is refused.
    big = 256
    assert L.layer.workspace_bytes(big) > _lib.lib().glmmoe_noalloc_scratch_bytes()
    x = L.x(big, 1)
    out = torch.empty(big, L.H, dtype=torch.float32, device="cuda")
    with pytest.raises(_lib.GlmMoeError, match="WORKSPACE"):
        L.layer.forward_noalloc(x, out)
