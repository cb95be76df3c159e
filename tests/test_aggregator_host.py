"""Host-side pieces of the VGGT-style aggregator (ress_amd/aggregator.py), on the CPU."""

import pytest
import torch

from ress_amd.aggregator import Aggregator


@pytest.mark.parametrize("hw", [(70, 84), (75, 90), (14, 14)])
def test_patch_embedding_gemm_matches_conv(hw):
    """The patch embedding runs as one GEMM over flattened patches; it must be the stride-14
    convolution (kernel = stride, no padding, trailing rows/columns that do not fill a
    patch dropped) with the module's own weight and bias, tokens in row-major patch order."""
    torch.manual_seed(0)
    m = Aggregator(depth=1, dim=48, num_heads=4)
    x = torch.randn(3, 3, *hw)
    ref = m.patch_embed(x).flatten(2).transpose(1, 2)
    got, h, w = m._embed_patches(x)
    assert (h, w) == (hw[0] // 14, hw[1] // 14)
    assert got.shape == ref.shape
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)
