"""Dilation / erosion in float16 and bfloat16 (mca_morpho_*_f16 / _bf16 and the torch operators; the
reference's TODO, morpho_op.cpp:7). The arithmetic is float32 with one rounding per stored result, so
the oracle is the float32 oracle on the same (exactly converted) values: forward values and saved
winners bit for bit after rounding the oracle's output to the 16-bit type; gradients within one unit
in the last place of the 16-bit type (norm-wise 1e-3 for float16, 8e-3 for bfloat16), since they are
rounded once from sums the float32 oracle forms in another order."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import normwise_error, seeded

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]
GTOL = {torch.float16: 1e-3, torch.bfloat16: 8e-3}
MERGES = ["sum", "mean", "max", "min", "identity"]


def _case(seed, dtype, B, Cin, Cout, H, W, K, merge):
    Cw = 1 if merge == "identity" else Cin
    if merge == "identity":
        Cout = Cin
    x = seeded(seed, B, Cin, H, W, kind="randn").to(dtype)
    w = seeded(seed + 1, Cout, Cw, K, K, kind="randn", scale=0.3).to(dtype)
    g = seeded(seed + 2, B, Cout, H, W, kind="randn").to(dtype)
    return x, w, g


@pytest.mark.parametrize("K", [3, 5, 4])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", ["dilation", "erosion"])
@pytest.mark.parametrize("dtype", DTYPES)
def test_16bit_matches_float32_oracle(dtype, op, merge, K):
    import morphocore_amd as mca

    dev = torch.device("cuda")
    x, w, g = _case(501 + K, dtype, 2, 3, 4, 19, 70, K, merge)
    for padding in ("replicate", "geodesic", "constant"):
        xd, wd = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
        f = mca.functional.dilation if op == "dilation" else mca.functional.erosion
        out = f(xd, wd, merge, padding, padding_value=0.25)
        out.backward(g.to(dev))
        assert out.dtype == dtype and xd.grad.dtype == dtype and wd.grad.dtype == dtype
        opc = O.DILATION if op == "dilation" else O.EROSION
        x32, w32, g32 = x.float().numpy(), w.float().numpy(), g.float().numpy()
        wk = w32 if op == "dilation" else np.ascontiguousarray(w32[:, :, ::-1, ::-1])
        ref, idx = O.morpho_forward(opc, O.MERGES[merge], O.PADDINGS[padding], 0.25, x32, wk, save_indices=merge in ("max", "min"))
        gx, gwk = O.morpho_backward(opc, O.MERGES[merge], O.PADDINGS[padding], 0.25, x32, wk, g32, indices=idx)
        gw = gwk if op == "dilation" else gwk[:, :, ::-1, ::-1]
        want = torch.from_numpy(ref).to(dtype)
        assert torch.equal(out.detach().cpu(), want), (op, merge, padding)
        for got, exp in ((xd.grad, gx), (wd.grad, gw)):
            exp16 = torch.from_numpy(np.ascontiguousarray(exp)).to(dtype).float().numpy()
            assert normwise_error(got.float().cpu().numpy(), exp16) <= GTOL[dtype], (op, merge, padding)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("merge", ["max", "sum", "identity"])
def test_16bit_saved_winners_match_float32(dtype, merge):
    # The C ABI forward saves the same winners as the float32 kernels on the converted values.
    from morphocore_amd import _native

    dev = torch.device("cuda")
    x, w, _ = _case(511, dtype, 2, 3, 4, 21, 66, 3, merge)
    xd, wd = x.to(dev), w.to(dev)
    geom = (2, 3, w.shape[0], w.shape[1], 21, 66, 3, 3)
    code = {"max": 0, "sum": 2, "identity": 5}[merge]
    nb = _native.indices_bytes(code, geom)
    i16 = torch.empty(nb, dtype=torch.uint8, device=dev)
    i32 = torch.empty(nb, dtype=torch.uint8, device=dev)
    o16 = torch.empty((2, w.shape[0], 21, 66), dtype=dtype, device=dev)
    o32 = torch.empty((2, w.shape[0], 21, 66), dtype=torch.float32, device=dev)
    _native.morpho_forward(0, code, True, 0.0, xd, wd, 0, o16, i16, geom)
    _native.morpho_forward(0, code, True, 0.0, xd.float(), wd.float(), 0, o32, i32, geom)
    torch.cuda.synchronize()
    assert torch.equal(i16, i32)
    assert torch.equal(o16, o32.to(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
def test_16bit_ties_and_specials(dtype):
    # Quantised values tie constantly; +-0, +-inf and NaN in the input.
    import morphocore_amd as mca

    dev = torch.device("cuda")
    x = seeded(521, 2, 3, 16, 40, kind="quant").to(dtype)
    x[0, 0, 2, 3:6] = float("nan")
    x[0, 1, 5, :] = float("inf")
    x[1, 2, 7, 1:9] = -float("inf")
    x[1, 0, 9, :] = -0.0
    w = torch.zeros(4, 3, 3, 3, dtype=dtype)
    for merge in ("max", "min", "sum"):
        out = mca.functional.dilation(x.to(dev), w.to(dev), merge, "geodesic")
        ref, _ = O.morpho_forward(O.DILATION, O.MERGES[merge], O.GEODESIC, 0.0, x.float().numpy(), w.float().numpy())
        got = out.cpu()
        want = torch.from_numpy(ref).to(dtype)
        assert torch.equal(torch.isnan(got), torch.isnan(want))
        same = got[~torch.isnan(got)] == want[~torch.isnan(want)]
        assert bool(same.all())
        assert torch.equal(torch.signbit(got[~torch.isnan(got)]), torch.signbit(want[~torch.isnan(want)]))


def test_16bit_rejected_by_smorph():
    import morphocore_amd as mca

    dev = torch.device("cuda")
    x = torch.zeros(1, 2, 8, 8, dtype=torch.float16, device=dev)
    w = torch.zeros(2, 2, 3, 3, dtype=torch.float16, device=dev)
    a = torch.zeros(2, 2, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="not implemented for 'Half'"):
        mca.functional.smorph(x, w, a)
