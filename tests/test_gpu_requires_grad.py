"""Gradients requested for any subset of the operators' inputs: each subset's gradients equal the ones the
all-inputs run gives (the saved state and the backward do not depend on which inputs ask), the others
stay None, and a forward under no_grad or with no input requiring grad saves nothing and builds no
graph."""
import itertools

import pytest
import torch

import morphocore_amd as mca

pytestmark = pytest.mark.gpu

F = mca.functional
DEV = "cuda"


def _inputs(kind, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(2, 3, 20, 70, generator=g)
    if kind == "morpho":
        return {"x": x, "w": torch.randn(4, 3, 5, 5, generator=g) * 0.3}
    if kind == "smorph":
        return {"x": x, "w": torch.randn(4, 3, 5, 5, generator=g) * 0.3, "alpha": torch.randn(4, 3, generator=g) * 2}
    if kind == "scm":
        return {"x": x, "w": torch.randn(4, 3, 5, 5, generator=g) * 0.3, "alpha": torch.randn(4, 3, generator=g) * 2,
                "beta": torch.randn(4, generator=g)}
    if kind == "sigma":
        return {"x": x, "w": torch.randn(3, 1, 3, 3, generator=g) * 0.3, "alpha": torch.randn(3, 1, generator=g)}
    return {"x": x, "w1": torch.randn(3, 1, 3, 3, generator=g) * 0.3, "w2": torch.randn(3, 1, 3, 3, generator=g) * 0.3}


CASES = {
    "dilation max": ("morpho", lambda t: F.dilation(t["x"], t["w"], "max", "replicate")),
    "erosion sum": ("morpho", lambda t: F.erosion(t["x"], t["w"], "sum", "geodesic")),
    "smorph mean": ("smorph", lambda t: F.smorph(t["x"], t["w"], t["alpha"], channel_merge_mode="mean")),
    "smorph max": ("smorph", lambda t: F.smorph(t["x"], t["w"], t["alpha"], channel_merge_mode="max")),
    "smorph_scm": ("scm", lambda t: F.smorph(t["x"], t["w"], t["alpha"], t["beta"])),
    "opening": ("pair", lambda t: F.opening(t["x"], t["w1"], t["w2"], "identity", "geodesic")),
    "sigma_layer": ("sigma", lambda t: F.sigma_layer(t["x"], t["w"], t["alpha"], "identity", "replicate")),
}


@pytest.mark.parametrize("name", list(CASES))
def test_any_subset_of_inputs(name):
    kind, fn = CASES[name]
    base = _inputs(kind, 7)
    names = list(base)
    g = torch.Generator().manual_seed(8)
    full = {k: v.to(DEV).requires_grad_(True) for k, v in base.items()}
    out = fn(full)
    grad = torch.randn(out.shape, generator=g).to(DEV)
    out.backward(grad)
    want = {k: v.grad.clone() for k, v in full.items()}
    for r in range(1, len(names)):
        for subset in itertools.combinations(names, r):
            print(f"{name}: gradients of {subset}", flush=True)
            t = {k: v.to(DEV).requires_grad_(k in subset) for k, v in base.items()}
            o = fn(t)
            torch.testing.assert_close(o.detach(), out.detach(), rtol=0, atol=0)
            o.backward(grad)
            for k in names:
                if k in subset:
                    # Sums of floating-point atomics may differ in their last bits between two runs.
                    torch.testing.assert_close(t[k].grad, want[k], rtol=1e-6, atol=1e-6 * float(want[k].abs().max()))
                else:
                    assert t[k].grad is None


@pytest.mark.parametrize("name", list(CASES))
def test_no_graph_without_gradients(name):
    kind, fn = CASES[name]
    t = {k: v.to(DEV) for k, v in _inputs(kind, 9).items()}
    out = fn(t)
    assert out.grad_fn is None and not out.requires_grad
    with torch.no_grad():
        t2 = {k: v.clone().requires_grad_(True) for k, v in t.items()}
        out2 = fn(t2)
    assert out2.grad_fn is None
    torch.testing.assert_close(out, out2, rtol=0, atol=0)
