"""Smorph gradients at the configs' real channel counts and structuring elements, against the
reference's own CPU extension (oracle/_ref, built from the reference sources; run in a child process
by tests/helpers.py: reference_run), on one batch element at the full spatial size:

* (1, 64, 256, 256) ~N(0, 1), w~ (64, 64, 7, 7) ~N(0, 0.1), merge mean, every alpha of its
  sweep, both backward paths (from the forward's saved pair statistics, and recomputing them);
* configs[4]'s smorph layer: (1, 64, 256, 256) ~U[0, 1), w~ (64, 64, 11, 11) ~N(0, 0.05), merge sum,
  alpha 5 (both paths).

Every output and gradient is compared element for element (norm-wise, the contract's 1e-6 for float32):
the forward output, grad_input, grad_weight of every (output, input) pair and tap, and grad_alpha of
every pair. This covers what conservation sums cannot: a permutation of taps or pairs inside the
kernels' slot reductions and packed LDS bins. Each case prints its name before the GPU work.
"""
import numpy as np
import pytest
import torch

from tests.helpers import REF_LIB, normwise_error, reference_run, seeded

pytestmark = pytest.mark.gpu

MEAN, SUM = 3, 2


@pytest.fixture(autouse=True)
def _ops():
    import morphocore_amd  # noqa: F401  (registers torch.ops.morphocore)
    if not __import__("os").path.exists(REF_LIB):
        pytest.skip("the reference's CPU extension (oracle/_ref) is not built")


def _gpu_smorph(x, wt, alpha, g, merge):
    dev = torch.device("cuda")
    xr = x.to(dev).requires_grad_(True)
    wr = wt.to(dev).requires_grad_(True)
    ar = alpha.to(dev).requires_grad_(True)
    out = torch.ops.morphocore.smorph(xr, wr, ar, merge)
    out.backward(g.to(dev))
    torch.cuda.synchronize()
    res = {"out": out.detach().cpu().numpy(), "grad_input": xr.grad.cpu().numpy(), "grad_weight": wr.grad.cpu().numpy(),
           "grad_alpha": ar.grad.cpu().numpy()}
    del out, xr, wr, ar
    torch.cuda.empty_cache()
    return res


def _compare(got, want, what):
    for k in ("out", "grad_input", "grad_weight", "grad_alpha"):
        err = normwise_error(got[k], want[k])
        print(f"  {what} {k}: {err:.3g}", flush=True)
        assert err <= 1e-6, f"{what}: {k} differs from the reference by {err}"


def _case(name, x, wt, alpha, g, merge, monkeypatch):
    print(name, "(GPU, saved statistics)", flush=True)
    saved = _gpu_smorph(x, wt, alpha, g, merge)
    print(name, "(GPU, recomputed statistics)", flush=True)
    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", "0")
    recomputed = _gpu_smorph(x, wt, alpha, g, merge)
    monkeypatch.delenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT")
    print(name, "(reference CPU extension)", flush=True)
    want = reference_run("smorph", x=x.numpy(), wt=wt.numpy(), alpha=alpha.numpy(), grad=g.numpy(), merge=np.array(merge))
    assert np.array_equal(saved["out"], recomputed["out"])
    _compare(saved, want, "saved")
    _compare(recomputed, want, "recomputed")


@pytest.mark.parametrize("a", [-20.0, -1.0, 0.0, 1.0, 20.0])
def test_config3_channels_against_the_reference(a, monkeypatch):
    x = seeded(70, 1, 64, 256, 256, kind="randn")
    wt = seeded(71, 64, 64, 7, 7, kind="randn", scale=0.1)
    g = seeded(72, 1, 64, 256, 256, kind="randn")
    _case(f"configs[2] channels, (1, 64, 256, 256) 7x7 mean, alpha {a}", x, wt, torch.full((64, 64), a), g, MEAN, monkeypatch)


def test_config5_smorph_channels_against_the_reference(monkeypatch):
    x = seeded(73, 1, 64, 256, 256)
    wt = seeded(74, 64, 64, 11, 11, kind="randn", scale=0.05)
    g = seeded(75, 1, 64, 256, 256, kind="randn")
    _case("configs[4] smorph layer channels, (1, 64, 256, 256) 11x11 sum, alpha 5", x, wt, torch.full((64, 64), 5.0), g, SUM, monkeypatch)
