"""Parity of smorph with the SMOOTH channel merge (the smorph_scm operator: smorph with a beta,
reference smorph_scm.cpp:13-96, smorph_cpu_kernels.hxx:231-266) on the GPU against the CPU oracle,
whose restatement is pinned by the reference's own vectors and by closed forms (tests/test_oracle.py).

Forward values bit for bit (the pair outputs, the soft merge's extremum and sums are computed in the
reference's order with its exponential); gradients of x, w~, alpha and beta within the contract's
tolerance (1e-6 float32, 1e-12 float64, norm-wise). Rectangular, even and large elements, border
tiles, beta of both signs and zero, NaN inputs, the torch operator and the module; in float32 with
square 3x3 / 5x5 / 7x7 / 11x11 elements, also the forward that saves each pair's statistics and the
backward that reads them."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float64]


def _np(t):
    return t.detach().cpu().numpy()


def _saves(dtype, KH, KW):
    """Whether the configuration has the saved-statistics path (float32, square 3, 5, 7, 11)."""
    return dtype == torch.float32 and KH == KW and KH in (3, 5, 7, 11)


def _abi_case(x, w, alpha, beta, g, saved=False):
    """Forward and backward through the C ABI (`saved`: the forward saves the pair statistics and the
    backward reads them); returns out, merge statistics and the gradients."""
    from morphocore_amd import _native

    dev = torch.device("cuda")
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w.shape
    geom = (B, Cin, Cout, Cw, H, W, KH, KW)
    xd, wd, gd = x.to(dev), w.to(dev), g.to(dev)
    ad = alpha.reshape(-1).to(dev).contiguous()
    bd = beta.reshape(-1).to(dev).contiguous()
    out = torch.empty((B, Cout, H, W), dtype=x.dtype, device=dev)
    ms = torch.empty((2, B, Cout, H, W), dtype=x.dtype, device=dev)
    ps = None
    if saved:
        nbytes = _native.smorph_scm_stats_bytes(x.dtype, geom)
        assert nbytes == 12 * B * Cout * Cin * H * W
        ps = torch.full((nbytes // 4,), float("nan"), device=dev)
    _native.smorph_scm_forward(xd, wd, ad, bd, out, ms, geom, pair_stats=ps)
    gx, gw, ga, gb = torch.empty_like(xd), torch.empty_like(wd), torch.empty_like(ad), torch.empty_like(bd)
    _native.smorph_scm_backward(xd, wd, ad, bd, out, ms, gd, gx, gw, ga, gb, geom, pair_stats=ps)
    torch.cuda.synchronize()
    return _np(out), _np(ms), _np(gx), _np(gw), _np(ga).reshape(alpha.shape), _np(gb)


def _check(x, w, alpha, beta, g, exact_forward=True, saved=False):
    out, _, gx, gw, ga, gb = _abi_case(x, w, alpha, beta, g, saved)
    xn, wn, an, bn, gn = x.numpy(), w.numpy(), alpha.numpy(), beta.numpy(), g.numpy()
    ref = O.smorph_scm_forward(xn, wn, an, bn)
    if exact_forward:
        assert np.array_equal(out, ref, equal_nan=True), "forward differs"
    else:
        assert normwise_error(out, ref) <= TOL[x.dtype]
    rgx, rgw, rga, rgb = O.smorph_scm_backward(xn, wn, an, bn, gn)
    for got, want, name in ((gx, rgx, "grad_input"), (gw, rgw, "grad_weight"), (ga, rga, "grad_alpha"), (gb, rgb, "grad_beta")):
        err = normwise_error(got, want)
        assert err <= TOL[x.dtype], f"{name}: {err}"


@pytest.mark.parametrize("saved", [False, True], ids=["recomputed", "saved"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("beta", ["pos", "neg", "zero", "mixed", "large"])
@pytest.mark.parametrize("KH,KW", [(3, 3), (5, 5), (3, 5), (4, 2), (1, 5), (7, 7), (11, 11)])
def test_scm_parity(KH, KW, beta, dtype, saved):
    if saved and not _saves(dtype, KH, KW):
        pytest.skip("no saved-statistics path for this configuration")
    B, Cin, Cout, H, W = 2, 3, 4, 19, 70
    print(f"scm {KH}x{KW} beta={beta} {dtype} saved={saved}", flush=True)
    x = seeded(41, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(42, Cout, Cin, KH, KW, dtype=dtype, kind="randn", scale=0.1)
    alpha = seeded(43, Cout, Cin, dtype=dtype, kind="randn", scale=3.0)
    betas = {"pos": torch.full((Cout,), 2.0), "neg": torch.full((Cout,), -3.0), "zero": torch.zeros(Cout),
             "mixed": seeded(44, Cout, kind="randn", scale=5.0), "large": torch.tensor([20.0, -20.0, 40.0, -0.5])}
    g = seeded(45, B, Cout, H, W, dtype=dtype, kind="randn")
    _check(x, w, alpha, betas[beta].to(dtype), g, saved=saved)


@pytest.mark.parametrize("dtype", DTYPES)
def test_scm_shared_alpha_large_element_and_one_channel(dtype):
    """A shared (0-d) alpha, an 11x11 element over a ragged image, and a single input channel (whose
    soft merge returns the pair output itself)."""
    x = seeded(51, 1, 2, 33, 90, dtype=dtype, kind="randn")
    w = seeded(52, 3, 2, 11, 11, dtype=dtype, kind="randn", scale=0.1)
    g = seeded(53, 1, 3, 33, 90, dtype=dtype, kind="randn")
    _check(x, w, torch.full((3, 2), 1.5, dtype=dtype), torch.tensor([1.0, -1.0, 0.3], dtype=dtype), g)
    x1 = seeded(54, 2, 1, 20, 65, dtype=dtype, kind="randn")
    w1 = seeded(55, 2, 1, 5, 5, dtype=dtype, kind="randn", scale=0.1)
    g1 = seeded(56, 2, 2, 20, 65, dtype=dtype, kind="randn")
    _check(x1, w1, torch.full((2, 1), -2.0, dtype=dtype), torch.tensor([4.0, -4.0], dtype=dtype), g1)


@pytest.mark.parametrize("saved", [False, True], ids=["recomputed", "saved"])
@pytest.mark.parametrize("K,Cout", [(3, 160), (5, 64), (5, 65), (7, 3), (11, 2)])
def test_scm_float32_static_partials(K, Cout, saved):
    """The float32 static backwards' grad_weight / grad_alpha / grad_beta partials: summed in LDS (5x5
    with 64 output channels, 64 x 27 values, the most that fit) or added with atomics (3x3 with 160
    output channels, 5x5 with 65, 7x7 and 11x11), over border and interior tiles; recomputing or from
    the saved pair statistics (11x11: packed bins with the alpha and beta tail)."""
    B, Cin, H, W = 1, 2, 21, 140
    x = seeded(71 + K, B, Cin, H, W, kind="randn")
    w = seeded(72 + K, Cout, Cin, K, K, kind="randn", scale=0.1)
    alpha = seeded(73 + K, Cout, Cin, kind="randn", scale=2.0)
    beta = seeded(74 + K, Cout, kind="randn", scale=2.0)
    g = seeded(75 + K, B, Cout, H, W, kind="randn")
    _check(x, w, alpha, beta, g, saved=saved)


@pytest.mark.parametrize("saved", [False, True], ids=["recomputed", "saved"])
def test_scm_nan_input_propagates_like_the_reference(saved):
    """An in-image NaN reaches its pairs' outputs, the merged output and the gradients as in the
    oracle (positions of NaN identical, finite values within the tolerance)."""
    x = seeded(57, 1, 2, 16, 70, kind="randn")
    x[0, 1, 5, 30] = float("nan")
    w = seeded(58, 2, 2, 3, 3, kind="randn", scale=0.1)
    g = seeded(59, 1, 2, 16, 70, kind="randn")
    out, _, gx, gw, ga, gb = _abi_case(x, w, torch.full((2, 2), 2.0), torch.tensor([1.0, -1.0]), g, saved)
    ref = O.smorph_scm_forward(x.numpy(), w.numpy(), np.full((2, 2), 2.0, np.float32), np.array([1.0, -1.0], np.float32))
    assert np.isnan(ref).any()
    assert np.array_equal(out, ref, equal_nan=True)
    rgx, rgw, rga, rgb = O.smorph_scm_backward(x.numpy(), w.numpy(), np.full((2, 2), 2.0, np.float32), np.array([1.0, -1.0], np.float32),
                                               g.numpy())
    for got, want in ((gx, rgx), (gw, rgw), (ga, rga), (gb, rgb)):
        assert np.array_equal(np.isnan(got), np.isnan(want))


@pytest.mark.parametrize("dtype", DTYPES)
def test_scm_operator_and_functional(dtype):
    """torch.ops.morphocore.smorph_scm through functional.smorph(beta=...) with autograd: w~ blended
    from w, the gradients of w and alpha carried back through torch, beta's gradient from the
    kernel."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    B, Cin, Cout, H, W, K = 2, 3, 2, 15, 66, 5
    x = seeded(61, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(62, Cout, Cin, K, K, dtype=dtype, kind="randn", scale=0.2)
    alpha = seeded(63, Cout, Cin, dtype=dtype, kind="randn", scale=2.0)
    beta = torch.tensor([2.5, -1.5], dtype=dtype)
    g = seeded(64, B, Cout, H, W, dtype=dtype, kind="randn")
    xd, wd, ad, bd = (t.to(dev).requires_grad_(True) for t in (x, w, alpha, beta))
    out = mca.functional.smorph(xd, wd, ad, beta=bd)
    out.backward(g.to(dev))
    # The oracle on the blended weight; torch carries grad_w~ to w and alpha on the CPU.
    wc, ac = w.clone().requires_grad_(True), alpha.clone().requires_grad_(True)
    t = torch.tanh(ac).unsqueeze(-1).unsqueeze(-1)
    wt = t * ((1 - t) / 2 * wc.flip(dims=(-2, -1)) + (1 + t) / 2 * wc)
    ref = O.smorph_scm_forward(x.numpy(), wt.detach().numpy(), alpha.numpy(), beta.numpy())
    assert np.array_equal(_np(out), ref)
    rgx, rgwt, rga, rgb = O.smorph_scm_backward(x.numpy(), wt.detach().numpy(), alpha.numpy(), beta.numpy(), g.numpy())
    torch.autograd.backward([wt, ac], [torch.from_numpy(rgwt), torch.from_numpy(rga)])
    assert normwise_error(_np(xd.grad), rgx) <= TOL[dtype]
    assert normwise_error(_np(wd.grad), wc.grad.numpy()) <= TOL[dtype]
    assert normwise_error(_np(ad.grad), ac.grad.numpy()) <= TOL[dtype]
    assert normwise_error(_np(bd.grad), rgb) <= TOL[dtype]


def test_scm_no_grad_keeps_no_statistics_and_matches():
    import morphocore_amd as mca

    dev = torch.device("cuda")
    x = seeded(65, 1, 2, 12, 40, kind="randn").to(dev)
    w = seeded(66, 3, 2, 3, 3, kind="randn", scale=0.1).to(dev)
    a, b = torch.full((3, 2), 1.0, device=dev), torch.tensor([1.0, 0.0, -1.0], device=dev)
    with torch.no_grad():
        y0 = torch.ops.morphocore.smorph_scm(x, w, a, b)
    y1 = torch.ops.morphocore.smorph_scm(x, w, a, b.clone().requires_grad_(True))
    assert torch.equal(y0, y1)


@pytest.mark.parametrize("K", [3, 7, 11])
def test_scm_saved_statistics_abi(K):
    """mca_smorph_scm_forward_stats_f32 / mca_smorph_scm_backward_stats_f32 through the C ABI: the
    output and the soft merge's statistics are bit for bit the plain forward's; the saved pair
    statistics are bit for bit those the SUM merge's forward saves for the same pairs (the same
    per-pair computation), their W / S being the pair outputs the soft merge reads; the gradients
    match the oracle and the recomputing backward."""
    from morphocore_amd import _native

    dev = torch.device("cuda")
    B, Cin, Cout, H, W = 2, 3, 4, 21, 70
    x = seeded(81, B, Cin, H, W, kind="randn")
    w = seeded(82, Cout, Cin, K, K, kind="randn", scale=0.1)
    alpha = torch.where(torch.arange(Cout * Cin) % 2 == 0, 3.0, -2.0).reshape(Cout, Cin) + seeded(83, Cout, Cin, kind="randn", scale=0.1)
    beta = torch.tensor([2.0, -3.0, 0.0, 7.5])
    g = seeded(84, B, Cout, H, W, kind="randn")
    geom = (B, Cin, Cout, Cin, H, W, K, K)
    xd, wd, ad, bd, gd = x.to(dev), w.to(dev), alpha.reshape(-1).to(dev), beta.to(dev), g.to(dev)
    nbytes = _native.smorph_scm_stats_bytes(torch.float32, geom)
    assert nbytes == _native.smorph_stats_bytes(O.MERGES["sum"], torch.float32, geom)
    outs, mss, pss = [], [], []
    for saved in (False, True):
        out = torch.empty((B, Cout, H, W), device=dev)
        ms = torch.empty((2, B, Cout, H, W), device=dev)
        ps = torch.full((nbytes // 4,), float("nan"), device=dev) if saved else None
        _native.smorph_scm_forward(xd, wd, ad, bd, out, ms, geom, pair_stats=ps)
        outs.append(out)
        mss.append(ms)
        pss.append(ps)
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(mss[0], mss[1])
    sum_stats = torch.full((nbytes // 4,), float("nan"), device=dev)
    _native.smorph_forward(O.MERGES["sum"], xd, wd, ad, torch.empty((B, Cout, H, W), device=dev), geom, stats=sum_stats)
    assert torch.equal(pss[1], sum_stats)
    ref = O.smorph_scm_forward(x.numpy(), w.numpy(), alpha.numpy(), beta.numpy())
    assert np.array_equal(_np(outs[1]), ref)
    want = O.smorph_scm_backward(x.numpy(), w.numpy(), alpha.numpy(), beta.numpy(), g.numpy())
    grads = []
    for ps in (pss[1], None):
        gx, gw, ga, gb = torch.empty_like(xd), torch.empty_like(wd), torch.empty_like(ad), torch.empty_like(bd)
        _native.smorph_scm_backward(xd, wd, ad, bd, outs[1], mss[1], gd, gx, gw, ga, gb, geom, pair_stats=ps)
        grads.append([_np(t) for t in (gx, gw, ga.reshape(Cout, Cin), gb)])
    for got in grads:
        for name, a, b in zip(("grad_input", "grad_weight", "grad_alpha", "grad_beta"), got, want):
            assert normwise_error(a, b) <= 1e-6, name
    for a1, a0 in zip(*grads):
        assert normwise_error(a1, a0) <= 1e-6


def test_scm_saves_statistics_only_for_a_backward(monkeypatch):
    """The smorph_scm operator keeps the pair statistics (float32) only when a backward can follow and
    the per-call cap allows them; they live as long as the graph holds them; the outputs and
    gradients do not depend on them."""
    from morphocore_amd import _C, _native

    dev = torch.device("cuda")
    live = lambda: _C.saved_stats_live_bytes(torch.cuda.current_device())  # noqa: E731
    base = live()
    x = seeded(85, 1, 2, 12, 70, kind="randn").to(dev)
    w = seeded(86, 3, 2, 5, 5, kind="randn", scale=0.1).to(dev)
    a, b = torch.full((3, 2), 2.0, device=dev), torch.tensor([1.0, 0.0, -1.0], device=dev)
    g = seeded(87, 1, 3, 12, 70, kind="randn").to(dev)
    nbytes = _native.smorph_scm_stats_bytes(torch.float32, (1, 2, 3, 2, 12, 70, 5, 5))
    with torch.no_grad():
        y0 = torch.ops.morphocore.smorph_scm(x, w, a, b)
    assert live() == base
    grads = []
    for limit, held in (("-1", nbytes), ("0", 0)):
        monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", limit)
        xr, br = x.clone().requires_grad_(True), b.clone().requires_grad_(True)
        y = torch.ops.morphocore.smorph_scm(xr, w, a, br)
        assert live() == base + held
        assert torch.equal(y, y0)
        y.backward(g)
        grads.append((xr.grad, br.grad))
        del y
        assert live() == base
    for g1, g0 in zip(*grads):
        assert normwise_error(_np(g1), _np(g0)) <= 1e-6
