"""Seeded sweep of the fused operators (opening_closing, sigma_identity) on random shapes (ragged
tiles, images smaller than the element, one channel, wide and tall planes), paddings, sizes and dtypes,
against the oracle's composition of the reference's single operators (functional/opening.py:96-101,
functional/closing.py:96-101, functional/sigma_layer.py:73-83), stage by stage: forward bit for bit,
gradients within 1e-6 (float32) / 1e-12 (float64) norm-wise. The composition of the HIP single
operators, which the product runs where the fused kernels do not apply, is held to the same oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error

pytestmark = pytest.mark.gpu

IDENTITY = 5


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        yield dict(B=int(rng.integers(1, 4)), C=int(rng.integers(1, 10)), H=int(rng.integers(1, 80)), W=int(rng.integers(1, 200)),
                   K=int(rng.choice([3, 5, 7])), padding=int(rng.integers(0, 4)), pv=float(rng.normal()),
                   dtype=[torch.float32, torch.float64][int(rng.integers(0, 2))], seed=int(rng.integers(0, 1 << 30)))


def _tensors(c):
    g = torch.Generator().manual_seed(c["seed"])
    mk = lambda *s, scale=1.0: (torch.randn(*s, generator=g, dtype=torch.float64) * scale).to(c["dtype"])  # noqa: E731
    x = mk(c["B"], c["C"], c["H"], c["W"])
    w1 = mk(c["C"], 1, c["K"], c["K"], scale=0.3)
    w2 = mk(c["C"], 1, c["K"], c["K"], scale=0.3)
    gout = mk(c["B"], c["C"], c["H"], c["W"])
    soft = torch.sigmoid(mk(c["C"]))
    return x, w1, w2, gout, soft


def _grads(outs, params, g):
    outs.backward(g)
    return [p.grad.detach().cpu().numpy() for p in params]


def _check(got, want, dtype):
    assert np.array_equal(got[0], want[0]), "forward"
    for name, u, v in zip(("grad_input", "grad_first", "grad_second"), got[1:], want[1:]):
        assert normwise_error(u, v) <= TOL[dtype], name


def _oracle_pair(first, p, pv, x, w1, w2, g):
    second = 1 - first
    mid, _ = O.morpho_forward(first, IDENTITY, p, pv, x, w1)
    out, _ = O.morpho_forward(second, IDENTITY, p, pv, mid, w2)
    gmid, gw2 = O.morpho_backward(second, IDENTITY, p, pv, mid, w2, g)
    gx, gw1 = O.morpho_backward(first, IDENTITY, p, pv, x, w1, gmid)
    return out, gx, gw1, gw2


@pytest.mark.parametrize("case", list(_cases(100, 2024)), ids=lambda c: f"{c['B']}x{c['C']}x{c['H']}x{c['W']}k{c['K']}p{c['padding']}")
@pytest.mark.parametrize("first", [0, 1], ids=["closing", "opening"])
def test_opening_closing_sweep(case, first):
    import morphocore_amd  # noqa: F401

    dev = torch.device("cuda")
    ops = torch.ops.morphocore
    x, w1, w2, g = (t for t in _tensors(case)[:4])
    p, pv = case["padding"], case["pv"]
    want = _oracle_pair(first, p, pv, x.numpy(), w1.numpy(), w2.numpy(), g.numpy())
    second = 1 - first
    for fused in (True, False):
        xd, a, b = (t.to(dev).requires_grad_(True) for t in (x, w1, w2))
        if fused:
            out = ops.opening_closing(xd, a, b, first, p, pv, True, 0.0)
        else:
            f1 = ops.erosion if first == 1 else ops.dilation
            f2 = ops.erosion if second == 1 else ops.dilation
            out = f2(f1(xd, a, IDENTITY, p, pv, True, 0.0), b, IDENTITY, p, pv, True, 0.0)
        _check([out.detach().cpu().numpy()] + _grads(out, [xd, a, b], g.to(dev)), want, case["dtype"])


@pytest.mark.parametrize("case", list(_cases(100, 4048)), ids=lambda c: f"{c['B']}x{c['C']}x{c['H']}x{c['W']}k{c['K']}p{c['padding']}")
def test_sigma_identity_sweep(case):
    import morphocore_amd  # noqa: F401

    dev = torch.device("cuda")
    ops = torch.ops.morphocore
    x, w, _, g, soft = _tensors(case)
    p, pv = case["padding"], case["pv"]
    # The oracle's composition: erosion (flipped element) and dilation, then torch's blend
    # e * (1 - s) + d * s, each product and the sum rounded in the dtype; its backward routes
    # g * (1 - s) through the erosion and g * s through the dilation.
    xn, wn, gn = x.numpy(), w.numpy(), g.numpy()
    wf = np.ascontiguousarray(wn[:, :, ::-1, ::-1])
    s = soft.numpy().reshape(1, -1, 1, 1)
    one = s.dtype.type(1)
    e, _ = O.morpho_forward(O.EROSION, IDENTITY, p, pv, xn, wf)
    d, _ = O.morpho_forward(O.DILATION, IDENTITY, p, pv, xn, wn)
    out = e * (one - s) + d * s
    gxe, gwe = O.morpho_backward(O.EROSION, IDENTITY, p, pv, xn, wf, (gn * (one - s)).astype(xn.dtype))
    gxd, gwd = O.morpho_backward(O.DILATION, IDENTITY, p, pv, xn, wn, (gn * s).astype(xn.dtype))
    want = [out, gxe + gxd, gwd + gwe[:, :, ::-1, ::-1]]
    gsoft = (gn.astype(np.float64) * (d.astype(np.float64) - e.astype(np.float64))).sum(axis=(0, 2, 3))
    scale = (np.abs(gn * e).astype(np.float64) + np.abs(gn * d).astype(np.float64)).sum(axis=(0, 2, 3))
    for fused in (True, False):
        xd, wd, sd = (t.to(dev).requires_grad_(True) for t in (x, w, soft))
        if fused:
            res = ops.sigma_identity(xd, wd.flip((-2, -1)), wd, sd, p, pv, True, 0.0)
        else:
            sv = sd.view(1, -1, 1, 1)
            res = ops.erosion(xd, wd.flip((-2, -1)), IDENTITY, p, pv, True, 0.0) * (1.0 - sv) + ops.dilation(xd, wd, IDENTITY, p, pv, True,
                                                                                                          0.0) * sv
        got = [res.detach().cpu().numpy()] + _grads(res, [xd, wd, sd], g.to(dev))
        _check(got[:3], want, case["dtype"])
        # The gradient of soft sums over every pixel in another order: within the rounding of that many
        # terms, relative to the sum of their magnitudes.
        assert bool((np.abs(got[3].astype(np.float64) - gsoft) <= 8 * TOL[case["dtype"]] * scale + 1e-300).all()), "grad_soft"
