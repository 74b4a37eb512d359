"""The compositions of the reference's API on the GPU: opening, closing and sigma_layer (functional
and nn; reference morphocore/functional/{opening,closing,sigma_layer}.py, morphocore/nn/{opening,
closing,sigma_layer}.py) against the oracle composed the same way, and the algebraic properties the
reference's own tests check for the shared structuring element (tests/functional/
test_opening_closing_sharing.py)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _flip(w):
    return np.ascontiguousarray(w[:, :, ::-1, ::-1])


def _oracle_stage(op, merge, padding, x, w, g=None):
    """One stage through the oracle with the functional layer's transform (erosion flips w)."""
    wk = w if op == O.DILATION else _flip(w)
    out, idx = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], 0.25, x, wk, save_indices=merge in ("max", "min"))
    if g is None:
        return out, None
    gx, gwk = O.morpho_backward(op, O.MERGES[merge], O.PADDINGS[padding], 0.25, x, wk, g, indices=idx)
    return out, (gx, gwk if op == O.DILATION else _flip(gwk))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("padding", ["replicate", "geodesic", "constant"])
@pytest.mark.parametrize("merge", ["sum", "max", "identity"])
@pytest.mark.parametrize("kind", ["opening", "closing"])
def test_opening_closing_against_oracle(kind, merge, padding, dtype):
    import morphocore_amd as mca

    dev = torch.device("cuda")
    B, Cin, H, W, K = 2, 3, 17, 70, 5
    Cmid = Cin if merge == "identity" else 4
    x = seeded(121, B, Cin, H, W, dtype=dtype, kind="randn")
    w1 = seeded(122, Cmid, 1 if merge == "identity" else Cin, K, K, dtype=dtype, kind="randn", scale=0.3)
    w2 = seeded(123, Cmid, 1, K, K, dtype=dtype, kind="randn", scale=0.3)
    g = seeded(124, B, Cmid, H, W, dtype=dtype, kind="randn")
    xd, w1d, w2d = (t.to(dev).requires_grad_(True) for t in (x, w1, w2))
    if kind == "opening":
        out = mca.functional.opening(xd, w1d, w2d, merge, padding, padding_value=0.25)
        first, second = O.EROSION, O.DILATION
    else:
        out = mca.functional.closing(xd, w1d, w2d, merge, padding, padding_value=0.25)
        first, second = O.DILATION, O.EROSION
    out.backward(g.to(dev))
    y1, _ = _oracle_stage(first, merge, padding, x.numpy(), w1.numpy())
    y2, (gy1, gw2) = _oracle_stage(second, "identity", padding, y1, w2.numpy(), g.numpy())
    _, (gx, gw1) = _oracle_stage(first, merge, padding, x.numpy(), w1.numpy(), gy1)
    assert np.array_equal(_np(out), y2)
    for got, want in ((xd.grad, gx), (w1d.grad, gw1), (w2d.grad, gw2)):
        assert normwise_error(_np(got), want) <= TOL[dtype]


@pytest.mark.parametrize("merge", ["sum", "max", "identity"])
def test_sigma_layer_against_oracle(merge):
    import morphocore_amd as mca

    dev = torch.device("cuda")
    B, Cin, H, W, K = 2, 3, 15, 66, 3
    Cout = Cin if merge == "identity" else 4
    x = seeded(125, B, Cin, H, W, kind="randn")
    w = seeded(126, Cout, 1 if merge == "identity" else Cin, K, K, kind="randn", scale=0.3)
    alpha = seeded(127, Cout, 1 if merge == "identity" else Cin, kind="randn")
    g = seeded(128, B, Cout, H, W, kind="randn")
    xd, wd, ad = (t.to(dev).requires_grad_(True) for t in (x, w, alpha))
    out = mca.functional.sigma_layer(xd, wd, ad, merge)
    out.backward(g.to(dev))
    e, _ = _oracle_stage(O.EROSION, merge, "replicate", x.numpy(), w.numpy())
    d, _ = _oracle_stage(O.DILATION, merge, "replicate", x.numpy(), w.numpy())
    # The blend in torch on the CPU, with the oracle's stage outputs.
    ac = alpha.clone().requires_grad_(True)
    ec, dc = torch.from_numpy(e).requires_grad_(True), torch.from_numpy(d).requires_grad_(True)
    soft = torch.sigmoid(ac.mean(dim=1)).view(1, -1, 1, 1)
    ref = ec * (1.0 - soft) + dc * soft
    ref.backward(g)
    assert normwise_error(_np(out), ref.detach().numpy()) <= 1e-6
    assert normwise_error(_np(ad.grad), ac.grad.numpy()) <= 1e-6
    _, (gex, gew) = _oracle_stage(O.EROSION, merge, "replicate", x.numpy(), w.numpy(), ec.grad.numpy())
    _, (gdx, gdw) = _oracle_stage(O.DILATION, merge, "replicate", x.numpy(), w.numpy(), dc.grad.numpy())
    assert normwise_error(_np(xd.grad), gex + gdx) <= 1e-6
    assert normwise_error(_np(wd.grad), gew + gdw) <= 1e-6


def _trained_like(layer):
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(torch.randn_like(p) * 0.5)
    return layer


def _violation_pct(y, x, sense):
    if sense == "anti":
        return (y > x + 1e-5).float().mean().item() * 100
    return (y < x - 1e-5).float().mean().item() * 100


@pytest.mark.parametrize("cls,sense", [("Opening", "anti"), ("Closing", "ext")])
def test_shared_structuring_element_properties(cls, sense):
    """With one structuring element and geodesic padding the layer is an algebraic opening (closing):
    anti-extensive (extensive) and idempotent; any padding leaves the interior property intact; the
    opt-out of sharing loses idempotence; the gradient reaches the shared weight (reference
    tests/functional/test_opening_closing_sharing.py:35-84)."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    Layer = getattr(mca.nn, cls)
    torch.manual_seed(0)
    layer = Layer(3, 3, 5).to(dev)
    assert layer.erosion.weight is layer.dilation.weight and len(list(layer.parameters())) == 1
    assert tuple(layer.erosion.weight.shape) == (3, 1, 5, 5)
    layer = _trained_like(Layer(3, 3, 5, padding_mode="geodesic").to(dev))
    x = torch.randn(2, 3, 20, 70, device=dev)
    y = layer(x)
    assert _violation_pct(y, x, sense) == 0.0
    assert (layer(y) - y).abs().max().item() < 1e-5
    free = _trained_like(Layer(3, 3, 5, padding_mode="geodesic", share_weights=False).to(dev))
    y = free(x)
    assert (free(y) - y).abs().max().item() > 1e-3
    for padding_mode in ("zero", "geodesic", "constant", "replicate"):
        layer = _trained_like(Layer(3, 3, 5, padding_mode=padding_mode).to(dev))
        y = layer(x)
        inner = (slice(None), slice(None), slice(4, -4), slice(4, -4))
        assert _violation_pct(y[inner], x[inner], sense) == 0.0, padding_mode
    layer = _trained_like(Layer(3, 3, 5).to(dev))
    layer(torch.randn(2, 3, 16, 16, device=dev)).sum().backward()
    grad = layer.erosion.weight.grad
    assert grad is not None and torch.isfinite(grad).all() and grad.abs().sum() > 0
    assert Layer(3, 8, 5, share_weights=False).to(dev)(torch.randn(2, 3, 16, 16, device=dev)).shape == (2, 8, 16, 16)


def test_sigma_layer_module_follows_training_mode():
    import morphocore_amd as mca

    dev = torch.device("cuda")
    torch.manual_seed(0)
    m = _trained_like(mca.nn.SigmaLayer(3, 3, 3, noise_scale=0.5).to(dev))
    x = torch.randn(2, 3, 12, 12, device=dev)
    m.eval()
    assert torch.equal(m(x), m(x))
    m.train()
    torch.manual_seed(1)
    first = m(x)
    torch.manual_seed(2)
    second = m(x)
    assert not torch.equal(first, second)
    first.sum().backward()
    assert torch.isfinite(m.alpha.grad).all()
