"""Fused sigma_layer with the 'identity' merge (mca_morpho_sigma_* and torch.ops.morphocore.
sigma_identity) against the reference's composition (functional/sigma_layer.py:73-83): the oracle's
erosion and dilation blended with numpy in the operand dtype (each product and the sum rounded, as
torch's three elementwise operations do) for the output, bit for bit; the saved taps against a brute
force of the strict first-tap rule; gradients against the oracle's two backwards with g (1 - soft) and
g soft, within 1e-6 (float32) / 1e-12 (float64) norm-wise."""
import numpy as np
import pytest
import torch

from morphocore_amd import _native
from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded
from tests.test_gpu_pair import PADDINGS, PV, _first_taps, _np

pytestmark = pytest.mark.gpu


def _oracle_sigma(padding, x, w, soft, g):
    we = np.ascontiguousarray(w[:, :, ::-1, ::-1])
    e, _ = O.morpho_forward(O.EROSION, O.IDENTITY, O.PADDINGS[padding], PV, x, we)
    d, _ = O.morpho_forward(O.DILATION, O.IDENTITY, O.PADDINGS[padding], PV, x, w)
    s = soft.reshape(1, -1, 1, 1)
    oms = (x.dtype.type(1) - s).astype(x.dtype)
    out = (e * oms).astype(x.dtype) + (d * s).astype(x.dtype)
    gxe, gwe = O.morpho_backward(O.EROSION, O.IDENTITY, O.PADDINGS[padding], PV, x, we, (g * oms).astype(x.dtype))
    gxd, gwd = O.morpho_backward(O.DILATION, O.IDENTITY, O.PADDINGS[padding], PV, x, w, (g * s).astype(x.dtype))
    terms = np.stack([(g * e).astype(np.float64).sum(axis=(0, 2, 3)), (g * d).astype(np.float64).sum(axis=(0, 2, 3))])
    return out.astype(x.dtype), e, d, we, gxe + gxd, gwe, gwd, terms


def _run_sigma(padding, x, w, soft, g, sample=None):
    dev = torch.device("cuda")
    B, C, H, W = x.shape
    K = w.shape[-1]
    pg = (B, C, H, W, K, K)
    xd = torch.from_numpy(x).to(dev)
    we = np.ascontiguousarray(w[:, :, ::-1, ::-1])
    if sample is None:
        ke, kd, wbs = torch.from_numpy(we).to(dev), torch.from_numpy(w).to(dev), 0
    else:
        ke, kd, wbs = torch.from_numpy(sample[0]).to(dev), torch.from_numpy(sample[1]).to(dev), C * K * K
    sd = torch.from_numpy(soft).to(dev)
    fe = O.fill_value(O.EROSION, O.PADDINGS[padding], PV, x.dtype)
    fd = O.fill_value(O.DILATION, O.PADDINGS[padding], PV, x.dtype)
    out = torch.empty_like(xd)
    taps = torch.empty((2, B, C, H, W), dtype=torch.uint8, device=dev)
    _native.morpho_sigma_forward(padding == "replicate", fe, fd, xd, ke, kd, wbs, sd, out, taps[0], taps[1], pg)
    gx = torch.empty_like(xd)
    gwe = torch.empty((C, 1, K, K), dtype=xd.dtype, device=dev)
    gwd = torch.empty_like(gwe)
    terms = torch.empty((2, C), dtype=xd.dtype, device=dev)
    _native.morpho_sigma_backward(padding == "replicate", fe, fd, xd, ke, kd, wbs, sd, taps[0], taps[1], torch.from_numpy(g).to(dev), gx, gwe,
                                  gwd, terms, pg)
    torch.cuda.synchronize()
    return _np(out), _np(taps), _np(gx), _np(gwe), _np(gwd), _np(terms)


def _case(seed, dtype, B, C, H, W, K, kind="randn"):
    x = seeded(seed, B, C, H, W, dtype=dtype, kind=kind).numpy()
    w = seeded(seed + 1, C, 1, K, K, dtype=dtype, kind=kind, scale=0.3 if kind == "randn" else 1.0).numpy()
    soft = torch.sigmoid(seeded(seed + 2, C, dtype=dtype, kind="randn")).numpy()
    g = seeded(seed + 3, B, C, H, W, dtype=dtype, kind=kind).numpy()
    return x, w, soft, g


def _check(padding, x, w, soft, g, dtype, exact=False):
    out, taps, gx, gwe, gwd, terms = _run_sigma(padding, x, w, soft, g)
    want, e, d, we, wgx, wgwe, wgwd, wterms = _oracle_sigma(padding, x, w, soft, g)
    assert np.array_equal(out, want, equal_nan=True)
    assert np.array_equal(taps[0], _first_taps(O.EROSION, padding, x, we)[1])
    assert np.array_equal(taps[1], _first_taps(O.DILATION, padding, x, w)[1])
    if exact:
        assert np.array_equal(gx, wgx) and np.array_equal(gwe, wgwe) and np.array_equal(gwd, wgwd)
    for got, exp in ((gx, wgx), (gwe, wgwe), (gwd, wgwd)):
        assert normwise_error(got, exp) <= TOL[dtype]
    # The per-channel sums run over every pixel in a different order: relative to their magnitude.
    scale = np.abs(g.astype(np.float64) * np.where(np.isfinite(e), e, 0)).sum(axis=(0, 2, 3))
    assert np.all(np.abs(terms.astype(np.float64) - wterms) <= 4 * TOL[dtype] * (scale + 1e-30) + 1e-300)


@pytest.mark.parametrize("K", [3, 5, 7])
@pytest.mark.parametrize("padding", PADDINGS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sigma_matches_composition(dtype, padding, K):
    x, w, soft, g = _case(401 + K, dtype, 2, 3, 37, 150, K)
    _check(padding, x, w, soft, g, dtype)


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (1, 2, 2, 3), (2, 1, 5, 4), (1, 2, 16, 64), (1, 1, 17, 65), (3, 2, 33, 129)])
@pytest.mark.parametrize("K", [3, 7])
def test_sigma_small_and_ragged_shapes(shape, K):
    x, w, soft, g = _case(411, torch.float32, *shape, K)
    for padding in ("replicate", "geodesic", "zero"):
        _check(padding, x, w, soft, g, torch.float32)


def test_sigma_dyadic_gradients_exact():
    # Quantised inputs and soft = 1/4: every product and sum is exact, so every gradient is bit for bit.
    x, w, _, g = _case(421, torch.float32, 2, 4, 40, 130, 5, kind="quant")
    soft = np.full(4, 0.25, dtype=np.float32)
    for padding in PADDINGS:
        _check(padding, x, w, soft, g, torch.float32, exact=True)


def test_sigma_nan_and_inf_inputs():
    x, w, soft, g = _case(431, torch.float64, 1, 2, 24, 90, 3)
    x[0, 0, 3:6, 10:20] = np.nan
    x[0, 1, 12, :] = np.inf
    for padding in ("replicate", "geodesic"):
        out, taps, gx, gwe, gwd, terms = _run_sigma(padding, x, w, soft, g)
        want, e, d, we, wgx, wgwe, wgwd, wterms = _oracle_sigma(padding, x, w, soft, g)
        assert np.array_equal(out, want, equal_nan=True)
        for got, exp in ((gx, wgx), (gwe, wgwe), (gwd, wgwd)):
            assert normwise_error(got, exp) <= 1e-12
        assert np.array_equal(np.isnan(terms), np.isnan(wterms))


def test_sigma_per_sample_weights():
    x, w, soft, g = _case(441, torch.float64, 3, 2, 20, 70, 3)
    rng = np.random.default_rng(9)
    we = np.ascontiguousarray(w[:, :, ::-1, ::-1])
    se = (we[None] + rng.uniform(-0.1, 0.1, (3,) + w.shape)).astype(np.float64)
    sd = (w[None] + rng.uniform(-0.1, 0.1, (3,) + w.shape)).astype(np.float64)
    out, taps, gx, gwe, gwd, terms = _run_sigma("constant", x, w, soft, g, sample=(se, sd))
    e, _ = O.morpho_forward(O.EROSION, O.IDENTITY, O.CONSTANT, PV, x, we, sample_weight=se)
    d, _ = O.morpho_forward(O.DILATION, O.IDENTITY, O.CONSTANT, PV, x, w, sample_weight=sd)
    s = soft.reshape(1, -1, 1, 1)
    assert np.array_equal(out, e * (1 - s) + d * s)
    gxe, wgwe = O.morpho_backward(O.EROSION, O.IDENTITY, O.CONSTANT, PV, x, we, g * (1 - s), sample_weight=se)
    gxd, wgwd = O.morpho_backward(O.DILATION, O.IDENTITY, O.CONSTANT, PV, x, w, g * s, sample_weight=sd)
    for got, exp in ((gx, gxe + gxd), (gwe, wgwe), (gwd, wgwd)):
        assert normwise_error(got, exp) <= 1e-12
    assert normwise_error(terms, np.stack([(g * e).sum(axis=(0, 2, 3)), (g * d).sum(axis=(0, 2, 3))])) <= 1e-12


def _composition(F, x, w, alpha, padding, **kw):
    e = F.erosion(x, w, 'identity', padding, padding_value=PV, **kw)
    d = F.dilation(x, w, 'identity', padding, padding_value=PV, **kw)
    soft = torch.sigmoid(alpha.mean(dim=1)).view(1, -1, 1, 1)
    return e * (1.0 - soft) + d * soft


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("padding", ["replicate", "geodesic"])
def test_functional_sigma_fused_equals_composition(dtype, padding):
    import morphocore_amd as mca

    F = mca.functional
    dev = torch.device("cuda")
    x = seeded(451, 2, 4, 29, 100, dtype=dtype, kind="randn").to(dev)
    w = seeded(452, 4, 1, 5, 5, dtype=dtype, kind="randn", scale=0.3).to(dev)
    a = seeded(453, 4, 1, dtype=dtype, kind="randn").to(dev)
    g = seeded(454, 2, 4, 29, 100, dtype=dtype, kind="randn").to(dev)
    res = []
    for fused in (True, False):
        xd, wd, ad = (t.clone().requires_grad_(True) for t in (x, w, a))
        out = F.sigma_layer(xd, wd, ad, 'identity', padding, padding_value=PV) if fused else _composition(F, xd, wd, ad, padding)
        out.backward(g)
        res.append((out.detach(), xd.grad, wd.grad, ad.grad))
    assert torch.equal(res[0][0], res[1][0])
    for u, v in zip(res[0][1:], res[1][1:]):
        assert normwise_error(_np(u), _np(v)) <= TOL[dtype] * 4


@pytest.mark.parametrize("dropout,noise", [(0.3, 0.0), (0.0, 0.2), (0.3, 0.2)])
def test_sigma_draws_like_composition(dropout, noise):
    import morphocore_amd as mca

    F = mca.functional
    dev = torch.device("cuda")
    x = seeded(461, 2, 3, 21, 80, kind="randn").to(dev)
    w = seeded(462, 3, 1, 3, 3, kind="randn", scale=0.3).to(dev)
    a = seeded(463, 3, 1, kind="randn").to(dev)
    kw = dict(weight_dropout=dropout, training=True, noise_scale=noise)
    torch.manual_seed(11)
    u = F.sigma_layer(x, w, a, 'identity', 'replicate', padding_value=PV, **kw)
    torch.manual_seed(11)
    v = _composition(F, x, w, a, 'replicate', **kw)
    assert torch.equal(u, v)


def test_nn_sigma_layer_identity():
    import morphocore_amd as mca

    dev = torch.device("cuda")
    m = mca.nn.SigmaLayer(3, 3, 3, channel_merge_mode='identity', init_alpha=0.4).to(dev)
    with torch.no_grad():
        m.weight.copy_(seeded(471, 3, 1, 3, 3, kind="randn", scale=0.3))
    x = seeded(472, 2, 3, 30, 70, kind="randn").to(dev)
    out = m(x)
    ref = _composition(mca.functional, x, m.weight, m.alpha, 'replicate')
    assert torch.equal(out, ref)
