"""The float32 dilation / erosion backward that allocates nothing (C ABI
mca_morpho_backward_noalloc_f32) against the backward with a caller workspace
(mca_morpho_backward_f32) and the oracle, through the C ABI: two calls in a row on one GPU, the
second with a smaller problem (the scratch keeps the first call's contents)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu


def _case(op, merge, B, Cin, Cout, H, W, K, seed, with_indices, kind="randn"):
    from morphocore_amd import _native

    dev = torch.device("cuda")
    Cw = 1 if merge == O.IDENTITY else Cin
    if merge == O.IDENTITY:
        Cout = Cin
    x = seeded(seed, B, Cin, H, W, kind=kind)
    w = seeded(seed + 1, Cout, Cw, K, K, kind=kind, scale=0.3)
    go = seeded(seed + 2, B, Cout, H, W, kind=kind)
    geom = (B, Cin, Cout, Cw, H, W, K, K)
    xd, wd, god = x.to(dev), w.to(dev), go.to(dev)
    out = torch.empty((B, Cout, H, W), device=dev)
    idx = None
    if with_indices:
        idx = torch.empty(max(_native.indices_bytes(merge, geom), 1), dtype=torch.uint8, device=dev)
    _native.morpho_forward(op, merge, True, 0.0, xd, wd, 0, out, idx, geom)
    gi_a, gw_a = torch.empty_like(xd), torch.empty_like(wd)
    gi_b, gw_b = torch.full_like(xd, float("nan")), torch.full_like(wd, float("nan"))
    _native.morpho_backward(op, merge, True, 0.0, xd, wd, 0, idx, god, gi_a, gw_a, geom)
    _native.morpho_backward_noalloc(op, merge, True, 0.0, xd, wd, 0, idx, god, gi_b, gw_b, geom)
    torch.cuda.synchronize()
    want_gi, want_gw = O.morpho_backward(op, merge, O.REPLICATE, 0.0, x.numpy(), w.numpy(), go.numpy())
    for got, ref, want in ((gi_b, gi_a, want_gi), (gw_b, gw_a, want_gw)):
        got, ref = got.cpu().numpy(), ref.cpu().numpy()
        assert normwise_error(got, ref) <= TOL[np.float32]
        assert normwise_error(got, want) <= TOL[np.float32]
        if kind == "quant":
            assert np.array_equal(got, ref), "dyadic inputs: both backwards are exact"


@pytest.mark.parametrize("with_indices", [True, False])
@pytest.mark.parametrize("merge", [O.MAX, O.MIN, O.ADD, O.AVERAGE, O.IDENTITY])
def test_noalloc_backward_matches_workspace_backward_twice(merge, with_indices):
    op = O.EROSION if merge in (O.MIN, O.AVERAGE) else O.DILATION
    print(f"noalloc merge={merge} indices={with_indices}: 2x5x6x40x90 k5, then 1x3x4x17x30 k3", flush=True)
    _case(op, merge, 2, 5, 6, 40, 90, 5, 100 + merge, with_indices)
    _case(op, merge, 1, 3, 4, 17, 30, 3, 200 + merge, with_indices)


@pytest.mark.parametrize("K", [3, 5])
def test_noalloc_identity_row_bands_twice(K):
    """Identity planes whose width is a multiple of 8 (16-byte aligned buffers): the row-band gather
    and its per-band partial slots in the scratch, then a smaller plane."""
    print(f"noalloc identity row bands k{K}: 2x6x37x64, then 1x3x19x32", flush=True)
    _case(O.DILATION, O.IDENTITY, 2, 6, 6, 37, 64, K, 400 + K, True)
    _case(O.EROSION, O.IDENTITY, 1, 3, 3, 19, 32, K, 410 + K, True)


def test_noalloc_backward_dyadic_exact():
    _case(O.DILATION, O.ADD, 2, 4, 4, 33, 70, 3, 300, True, kind="quant")
    _case(O.DILATION, O.MAX, 1, 2, 3, 20, 20, 3, 310, False, kind="quant")
