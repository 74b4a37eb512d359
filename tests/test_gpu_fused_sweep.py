"""Seeded sweep of the fused operators (opening_closing, sigma_identity) against the compositions of
the single operators they replace, on random shapes (ragged tiles, images smaller than the element,
one channel, wide and tall planes), paddings, sizes and dtypes: forward bit for bit, gradients within
1e-6 (float32) / 1e-12 (float64) norm-wise."""
import numpy as np
import pytest
import torch

from tests.helpers import TOL, normwise_error

pytestmark = pytest.mark.gpu

ops = None


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        yield dict(B=int(rng.integers(1, 4)), C=int(rng.integers(1, 10)), H=int(rng.integers(1, 80)), W=int(rng.integers(1, 200)),
                   K=int(rng.choice([3, 5, 7])), padding=int(rng.integers(0, 4)), pv=float(rng.normal()),
                   dtype=[torch.float32, torch.float64][int(rng.integers(0, 2))], seed=int(rng.integers(0, 1 << 30)))


def _tensors(c, dev):
    g = torch.Generator().manual_seed(c["seed"])
    mk = lambda *s, scale=1.0: (torch.randn(*s, generator=g, dtype=torch.float64) * scale).to(c["dtype"]).to(dev)  # noqa: E731
    x = mk(c["B"], c["C"], c["H"], c["W"])
    w1 = mk(c["C"], 1, c["K"], c["K"], scale=0.3)
    w2 = mk(c["C"], 1, c["K"], c["K"], scale=0.3)
    gout = mk(c["B"], c["C"], c["H"], c["W"])
    soft = torch.sigmoid(mk(c["C"]))
    return x, w1, w2, gout, soft


def _grads(outs, params, g):
    outs.backward(g)
    return [p.grad.detach().clone() for p in params]


@pytest.mark.parametrize("case", list(_cases(100, 2024)), ids=lambda c: f"{c['B']}x{c['C']}x{c['H']}x{c['W']}k{c['K']}p{c['padding']}")
@pytest.mark.parametrize("first", [0, 1], ids=["closing", "opening"])
def test_opening_closing_sweep(case, first):
    import morphocore_amd  # noqa: F401

    dev = torch.device("cuda")
    ops = torch.ops.morphocore
    x, w1, w2, g, _ = _tensors(case, dev)
    p, pv = case["padding"], case["pv"]
    second = 1 - first
    res = []
    for fused in (True, False):
        xd, a, b = (t.clone().requires_grad_(True) for t in (x, w1, w2))
        if fused:
            out = ops.opening_closing(xd, a, b, first, p, pv, True, 0.0)
        else:
            f1 = ops.erosion if first == 1 else ops.dilation
            f2 = ops.erosion if second == 1 else ops.dilation
            out = f2(f1(xd, a, 5, p, pv, True, 0.0), b, 5, p, pv, True, 0.0)
        res.append([out.detach()] + _grads(out, [xd, a, b], g))
    assert torch.equal(res[0][0], res[1][0])
    for u, v in zip(res[0][1:], res[1][1:]):
        assert normwise_error(u.cpu().numpy(), v.cpu().numpy()) <= TOL[case["dtype"]]


@pytest.mark.parametrize("case", list(_cases(100, 4048)), ids=lambda c: f"{c['B']}x{c['C']}x{c['H']}x{c['W']}k{c['K']}p{c['padding']}")
def test_sigma_identity_sweep(case):
    import morphocore_amd  # noqa: F401

    dev = torch.device("cuda")
    ops = torch.ops.morphocore
    x, w1, _, g, soft = _tensors(case, dev)
    p, pv = case["padding"], case["pv"]
    res = []
    for fused in (True, False):
        xd, wd, sd = (t.clone().requires_grad_(True) for t in (x, w1, soft))
        if fused:
            out = ops.sigma_identity(xd, wd.flip((-2, -1)), wd, sd, p, pv, True, 0.0)
        else:
            e = ops.erosion(xd, wd.flip((-2, -1)), 5, p, pv, True, 0.0)
            d = ops.dilation(xd, wd, 5, p, pv, True, 0.0)
            s = sd.view(1, -1, 1, 1)
            out = e * (1.0 - s) + d * s
            fin = lambda t: torch.where(torch.isfinite(t), t, torch.zeros_like(t))  # noqa: E731
            scale = ((g * fin(e).detach()).abs() + (g * fin(d).detach()).abs()).double().sum(dim=(0, 2, 3))
        res.append([out.detach()] + _grads(out, [xd, wd, sd], g))
    assert torch.equal(res[0][0], res[1][0])
    for u, v in zip(res[0][1:3], res[1][1:3]):
        assert normwise_error(u.cpu().numpy(), v.cpu().numpy()) <= TOL[case["dtype"]]
    # The gradient of soft sums over every pixel in another order: within the rounding of that many
    # terms, relative to the sum of their magnitudes.
    diff = (res[0][3].double() - res[1][3].double()).abs()
    assert bool((diff <= 8 * TOL[case["dtype"]] * scale + 1e-300).all())
