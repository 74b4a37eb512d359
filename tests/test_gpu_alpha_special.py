"""Smorph with special alpha values, against the oracle: negative zero (the alpha = 0 path takes it as
zero, as the reference's arithmetic does: every e is 1), magnitudes so small that every tap weighs
the same (+-1e-30), so large that the softmax is the hard extremum and every other tap's exponential
underflows (+-1e30), and +-88, whose scaled differences straddle the exponential's lower threshold.
Per-pair alphas mix them in one launch; forward values bit for bit, gradients within the contract,
with the pair statistics saved and recomputed."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu

SPECIAL = [-0.0, 1e-30, -1e-30, 1e30, -1e30, 88.0, -88.0, 0.0, 3.0]


@pytest.mark.parametrize("saved", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("merge", ["sum", "mean", "max", "min", "identity"])
@pytest.mark.parametrize("K", [3, 7])
def test_smorph_special_alphas(K, merge, dtype, saved, monkeypatch):
    import morphocore_amd  # noqa: F401

    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", "-1" if saved else "0")
    B, Cin, Cout, H, W = 2, 3, 3, 20, 70
    print(f"smorph special alphas {K}x{K} {merge} {dtype} saved={saved}", flush=True)
    x = seeded(901, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(902, Cout, 1 if merge == "identity" else Cin, K, K, dtype=dtype, kind="randn", scale=0.2)
    pairs = Cout if merge == "identity" else Cout * Cin
    alpha = torch.tensor([SPECIAL[p % len(SPECIAL)] for p in range(pairs)], dtype=dtype)
    alpha = alpha.reshape((Cout,) if merge == "identity" else (Cout, Cin))
    g = seeded(903, B, Cout, H, W, dtype=dtype, kind="randn")
    dev = torch.device("cuda")
    xd, wd, ad = (t.to(dev).requires_grad_(True) for t in (x, w, alpha))
    out = torch.ops.morphocore.smorph(xd, wd, ad, O.MERGES[merge])
    out.backward(g.to(dev))
    ref = O.smorph_forward(O.MERGES[merge], x.numpy(), w.numpy(), alpha.numpy())
    got = out.detach().cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)]), "forward differs"
    gx, gw, ga = O.smorph_backward(O.MERGES[merge], x.numpy(), w.numpy(), alpha.numpy(), g.numpy())
    for name, a, b in (("grad_input", xd.grad, gx), ("grad_weight", wd.grad, gw), ("grad_alpha", ad.grad, ga)):
        err = normwise_error(a.detach().cpu().numpy(), b)
        assert err <= TOL[dtype], f"{name}: {err}"
