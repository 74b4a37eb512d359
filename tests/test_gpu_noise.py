"""Weight noise's per-sample elements (mca_noise_sample_weights_*) against the reference's composed
expression w + (rand * 2 - 1) * noise_scale (morpho_op_wrap.hxx:55-64) evaluated by torch on the same
draw: bit for bit, for both dtypes and scales whose float32 rounding matters."""
import pytest
import torch

from morphocore_amd import _native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("scale", [0.05, 0.3, 1e-3, 0.1234567891])
def test_noise_sample_matches_torch_expression(dtype, scale):
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    w = torch.randn((7, 3, 5, 5), generator=g, dtype=dtype, device=dev)
    u = torch.rand((6, 7, 3, 5, 5), generator=g, dtype=dtype, device=dev)
    u[0, 0, 0, 0, :3] = torch.tensor([0.0, 2.0 ** -30, 0.5], dtype=dtype)
    want = w.unsqueeze(0) + (u * 2.0 - 1.0) * scale
    out = torch.empty_like(u)
    _native.noise_sample_weights(w, u, scale, out)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
