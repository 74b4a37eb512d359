"""Fused opening / closing with per-channel merges (mca_morpho_pair_* and torch.ops.morphocore.
opening_closing) against the reference's composition of two operators (functional/opening.py:96-101,
functional/closing.py:96-101): the oracle run stage by stage for values and gradients, and a numpy
brute force of the strict first-tap rule (morpho_op_cpu_kernels.hxx:254-263) for the saved taps.
Forward values and taps bit for bit; gradients within 1e-6 (float32) / 1e-12 (float64) norm-wise,
and bit for bit on dyadic inputs, whose sums are exact."""
import numpy as np
import pytest
import torch

from morphocore_amd import _native
from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu

PADDINGS = ["zero", "geodesic", "constant", "replicate"]
PV = 0.25


def _np(t):
    return t.detach().cpu().numpy()


def _other(op):
    return O.EROSION if op == O.DILATION else O.DILATION


def _first_taps(op, padding, x, wk):
    """Strict first-tap scan of every pixel (identity merge) in numpy: (values, taps)."""
    B, C, H, W = x.shape
    KH, KW = wk.shape[-2:]
    ph, pw = KH // 2, KW // 2
    fill = O.fill_value(op, O.PADDINGS[padding], PV, x.dtype)
    ys, xs = np.arange(H)[:, None], np.arange(W)[None, :]
    best = np.full(x.shape, -np.inf if op == O.DILATION else np.inf, dtype=x.dtype)
    arg = np.zeros(x.shape, dtype=np.int64)
    for kh in range(KH):
        for kw in range(KW):
            yy, xx = ys + ph - kh, xs + pw - kw
            inb = (yy >= 0) & (yy < H) & (xx >= 0) & (xx < W)
            v = x[:, :, np.clip(yy, 0, H - 1), np.clip(xx, 0, W - 1)]
            if padding != "replicate":
                v = np.where(inb, v, x.dtype.type(fill))
            wv = wk[None, :, 0, kh, kw, None, None]
            v = v + wv if op == O.DILATION else v - wv
            better = v > best if op == O.DILATION else v < best
            best = np.where(better, v, best)
            arg = np.where(better, kh * KW + kw, arg)
    return best, arg


def _oracle_pair(first, padding, x, w1, w2, g):
    """The composition through the oracle: values, then the two backwards chained."""
    second = _other(first)
    e, _ = O.morpho_forward(first, O.IDENTITY, O.PADDINGS[padding], PV, x, w1)
    out, _ = O.morpho_forward(second, O.IDENTITY, O.PADDINGS[padding], PV, e, w2)
    ge, gw2 = O.morpho_backward(second, O.IDENTITY, O.PADDINGS[padding], PV, e, w2, g)
    gx, gw1 = O.morpho_backward(first, O.IDENTITY, O.PADDINGS[padding], PV, x, w1, ge)
    return e, out, gx, gw1, gw2


def _run_pair(first, padding, x, w1, w2, g, sample=None):
    """Fused forward and backward through the C ABI; w1 / w2 as the operators receive them."""
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    B, C, H, W = x.shape
    K = w1.shape[-1]
    pg = (B, C, H, W, K, K)
    second = _other(first)
    f1 = O.fill_value(first, O.PADDINGS[padding], PV, x.dtype)
    f2 = O.fill_value(second, O.PADDINGS[padding], PV, x.dtype)
    if sample is None:
        k1, k2, wbs = torch.from_numpy(w1).to(dev), torch.from_numpy(w2).to(dev), 0
    else:
        k1, k2, wbs = torch.from_numpy(sample[0]).to(dev), torch.from_numpy(sample[1]).to(dev), C * K * K
    out = torch.empty_like(xd)
    taps = torch.empty((2, B, C, H, W), dtype=torch.uint8, device=dev)
    _native.morpho_pair_forward(first, padding == "replicate", f1, f2, xd, k1, k2, wbs, out, taps[0], taps[1], pg)
    gd = torch.from_numpy(g).to(dev)
    gx = torch.empty_like(xd)
    gw1 = torch.empty((C, 1, K, K), dtype=xd.dtype, device=dev)
    gw2 = torch.empty_like(gw1)
    _native.morpho_pair_backward(first, taps[0], taps[1], gd, gx, gw1, gw2, pg)
    torch.cuda.synchronize()
    return _np(out), _np(taps), _np(gx), _np(gw1), _np(gw2)


def _case(seed, dtype, B, C, H, W, K, kind="randn"):
    x = seeded(seed, B, C, H, W, dtype=dtype, kind=kind).numpy()
    w1 = seeded(seed + 1, C, 1, K, K, dtype=dtype, kind=kind, scale=0.3 if kind == "randn" else 1.0).numpy()
    w2 = seeded(seed + 2, C, 1, K, K, dtype=dtype, kind=kind, scale=0.3 if kind == "randn" else 1.0).numpy()
    g = seeded(seed + 3, B, C, H, W, dtype=dtype, kind=kind).numpy()
    return x, w1, w2, g


@pytest.mark.parametrize("K", [3, 5, 7])
@pytest.mark.parametrize("padding", PADDINGS)
@pytest.mark.parametrize("first", [O.EROSION, O.DILATION], ids=["opening", "closing"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_pair_matches_composition(dtype, first, padding, K):
    x, w1, w2, g = _case(301 + K, dtype, 2, 3, 37, 150, K)
    out, taps, gx, gw1, gw2 = _run_pair(first, padding, x, w1, w2, g)
    e, want, wgx, wgw1, wgw2 = _oracle_pair(first, padding, x, w1, w2, g)
    assert np.array_equal(out, want)
    be, t1 = _first_taps(first, padding, x, w1)
    bo, t2 = _first_taps(_other(first), padding, be, w2)
    assert np.array_equal(be, e) and np.array_equal(bo, want)
    assert np.array_equal(taps[0], t1) and np.array_equal(taps[1], t2)
    for got, exp in ((gx, wgx), (gw1, wgw1), (gw2, wgw2)):
        assert normwise_error(got, exp) <= TOL[dtype]


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (1, 2, 2, 3), (2, 1, 5, 4), (1, 2, 16, 58), (1, 1, 17, 63), (3, 2, 33, 125)])
@pytest.mark.parametrize("K", [3, 7])
def test_pair_small_and_ragged_shapes(shape, K):
    x, w1, w2, g = _case(311, torch.float32, *shape, K)
    for first in (O.EROSION, O.DILATION):
        for padding in ("replicate", "geodesic"):
            out, taps, gx, gw1, gw2 = _run_pair(first, padding, x, w1, w2, g)
            e, want, wgx, wgw1, wgw2 = _oracle_pair(first, padding, x, w1, w2, g)
            assert np.array_equal(out, want)
            assert np.array_equal(taps[0], _first_taps(first, padding, x, w1)[1])
            for got, exp in ((gx, wgx), (gw1, wgw1), (gw2, wgw2)):
                assert normwise_error(got, exp) <= 1e-6


@pytest.mark.parametrize("first", [O.EROSION, O.DILATION], ids=["opening", "closing"])
def test_pair_dyadic_gradients_exact(first):
    # Quantised inputs (multiples of 1/16) tie often and sum exactly: every gradient bit for bit.
    x, w1, w2, g = _case(321, torch.float32, 2, 4, 40, 130, 5, kind="quant")
    for padding in PADDINGS:
        out, taps, gx, gw1, gw2 = _run_pair(first, padding, x, w1, w2, g)
        e, want, wgx, wgw1, wgw2 = _oracle_pair(first, padding, x, w1, w2, g)
        assert np.array_equal(out, want)
        assert np.array_equal(taps[1], _first_taps(_other(first), padding, e, w2)[1])
        assert np.array_equal(gx, wgx) and np.array_equal(gw1, wgw1) and np.array_equal(gw2, wgw2)


def test_pair_per_sample_weights():
    # One element per batch element (weight noise), weight_batch_stride apart.
    x, w1, w2, g = _case(331, torch.float64, 3, 2, 20, 70, 3)
    rng = np.random.default_rng(5)
    s1 = (w1[None] + rng.uniform(-0.1, 0.1, (3,) + w1.shape)).astype(np.float64)
    s2 = (w2[None] + rng.uniform(-0.1, 0.1, (3,) + w2.shape)).astype(np.float64)
    for first in (O.EROSION, O.DILATION):
        out, taps, gx, gw1, gw2 = _run_pair(first, "constant", x, w1, w2, g, sample=(s1, s2))
        e, _ = O.morpho_forward(first, O.IDENTITY, O.CONSTANT, PV, x, w1, sample_weight=s1)
        want, _ = O.morpho_forward(_other(first), O.IDENTITY, O.CONSTANT, PV, e, w2, sample_weight=s2)
        ge, wgw2 = O.morpho_backward(_other(first), O.IDENTITY, O.CONSTANT, PV, e, w2, g, sample_weight=s2)
        wgx, wgw1 = O.morpho_backward(first, O.IDENTITY, O.CONSTANT, PV, x, w1, ge, sample_weight=s1)
        assert np.array_equal(out, want)
        for got, exp in ((gx, wgx), (gw1, wgw1), (gw2, wgw2)):
            assert normwise_error(got, exp) <= 1e-12


def test_pair_nan_and_inf_inputs():
    x, w1, w2, g = _case(341, torch.float32, 1, 2, 24, 90, 5)
    x[0, 0, 3:6, 10:20] = np.nan
    x[0, 1, 12, :] = np.inf
    x[0, 1, 20, 40:60] = -np.inf
    for first in (O.EROSION, O.DILATION):
        for padding in ("replicate", "zero"):
            out, taps, gx, gw1, gw2 = _run_pair(first, padding, x, w1, w2, g)
            e, want, wgx, wgw1, wgw2 = _oracle_pair(first, padding, x, w1, w2, g)
            assert np.array_equal(out, want, equal_nan=True)
            assert np.array_equal(taps[0], _first_taps(first, padding, x, w1)[1])
            assert np.array_equal(gx, wgx, equal_nan=True)
            for got, exp in ((gw1, wgw1), (gw2, wgw2)):
                assert normwise_error(got, exp) <= 1e-6


class _CountingOps:
    """Forwards to torch.ops.morphocore and counts opening_closing calls."""

    def __init__(self):
        self.calls = 0

    def __getattr__(self, name):
        op = getattr(torch.ops.morphocore, name)
        if name != "opening_closing":
            return op

        def counted(*args):
            self.calls += 1
            return op(*args)

        return counted


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("kind", ["opening", "closing"])
def test_functional_fused_equals_composition(kind, dtype, monkeypatch):
    import morphocore_amd as mca
    from morphocore_amd.functional import _pair

    counter = _CountingOps()
    monkeypatch.setattr(_pair, "ops", counter)
    dev = torch.device("cuda")
    x = seeded(351, 2, 4, 29, 100, dtype=dtype, kind="randn").to(dev)
    w1 = seeded(352, 4, 1, 5, 5, dtype=dtype, kind="randn", scale=0.3).to(dev)
    w2 = seeded(353, 4, 1, 5, 5, dtype=dtype, kind="randn", scale=0.3).to(dev)
    g = seeded(354, 2, 4, 29, 100, dtype=dtype, kind="randn").to(dev)
    F = mca.functional
    first, second = (F.erosion, F.dilation) if kind == "opening" else (F.dilation, F.erosion)
    fused = F.opening if kind == "opening" else F.closing
    grads = []
    for use_fused in (True, False):
        xd, w1d, w2d = (t.clone().requires_grad_(True) for t in (x, w1, w2))
        if use_fused:
            out = fused(xd, w1d, w2d, 'identity', 'constant', padding_value=PV)
        else:
            out = second(first(xd, w1d, 'identity', 'constant', padding_value=PV), w2d, 'identity', 'constant', padding_value=PV)
        out.backward(g)
        grads.append([out.detach(), xd.grad, w1d.grad, w2d.grad])
    assert counter.calls == 1
    assert torch.equal(grads[0][0], grads[1][0])
    for a, b in zip(grads[0][1:], grads[1][1:]):
        assert normwise_error(_np(a), _np(b)) <= TOL[dtype]


@pytest.mark.parametrize("kind", ["opening", "closing"])
@pytest.mark.parametrize("dropout,noise", [(0.3, 0.0), (0.0, 0.2), (0.3, 0.2)])
def test_fused_draws_like_composition(kind, dropout, noise):
    # Seeded training runs draw the same dropout masks and noise as the two separate operator calls.
    import morphocore_amd as mca

    dev = torch.device("cuda")
    x = seeded(361, 2, 3, 21, 80, kind="randn").to(dev)
    w1 = seeded(362, 3, 1, 3, 3, kind="randn", scale=0.3).to(dev)
    w2 = seeded(363, 3, 1, 3, 3, kind="randn", scale=0.3).to(dev)
    F = mca.functional
    first, second = (F.erosion, F.dilation) if kind == "opening" else (F.dilation, F.erosion)
    fused = F.opening if kind == "opening" else F.closing
    kw = dict(weight_dropout=dropout, training=True, noise_scale=noise)
    torch.manual_seed(7)
    a = fused(x, w1, w2, 'identity', 'replicate', **kw)
    torch.manual_seed(7)
    b = second(first(x, w1, 'identity', 'replicate', **kw), w2, 'identity', 'replicate', **kw)
    assert torch.equal(a, b)


@pytest.mark.parametrize("kind", ["Opening", "Closing"])
def test_nn_shared_weight_fused(kind):
    import morphocore_amd as mca

    dev = torch.device("cuda")
    torch.manual_seed(3)
    m = getattr(mca.nn, kind)(3, 3, 5, padding_mode='geodesic').to(dev)
    with torch.no_grad():
        m.erosion.weight.copy_(seeded(371, 3, 1, 5, 5, kind="randn", scale=0.3))
    x = seeded(372, 2, 3, 30, 70, kind="randn").to(dev)
    g = seeded(373, 2, 3, 30, 70, kind="randn").to(dev)
    out = m(x)
    out.backward(g)
    fused_grad = m.erosion.weight.grad.clone()
    m.zero_grad()
    a, b = (m.erosion, m.dilation) if kind == "Opening" else (m.dilation, m.erosion)
    ref = b(a(x))
    ref.backward(g)
    assert torch.equal(out, ref)
    assert normwise_error(_np(fused_grad), _np(m.erosion.weight.grad)) <= 1e-6
