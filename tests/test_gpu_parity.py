"""Parity of the HIP kernels with the CPU oracle (oracle/), on the GPU.

Forward values of every merge and the packed indices are compared bit for bit; gradients and smorph
within the contract's tolerance (relative 1e-6 float32, 1e-12 float64, norm-wise: max |diff| over
max |expected| per tensor). Inputs are seeded and sized so the oracle finishes in seconds; the
reference's own test cases (odd shapes, even kernels, kernel larger than the image, every padding,
ties) are re-expressed here.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu

MERGES = ["max", "min", "sum", "mean", "identity"]
PADDINGS = ["zero", "geodesic", "constant", "replicate"]
DTYPES = [torch.float32, torch.float64]


def _mca():
    import morphocore_amd
    from morphocore_amd import _native
    return morphocore_amd, _native, None


def _np(t):
    return t.detach().cpu().numpy()


def _weight_shape(merge, cin, cout, kh, kw):
    return (cin, 1, kh, kw) if merge == "identity" else (cout, cin, kh, kw)


def kernel_forward(op, merge, padding, pv, x, w, save=False, sample_weight=None):
    """One call of the C ABI forward on the GPU (kernel-facing weight)."""
    _, native, _ = _mca()
    dev = torch.device("cuda")
    xd = x.to(dev).contiguous()
    wd = (w if sample_weight is None else sample_weight).to(dev).contiguous()
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w.shape
    out = torch.empty((B, Cout, H, W), dtype=x.dtype, device=dev)
    idx = torch.empty((B, Cout, H, W), dtype=torch.int32, device=dev) if save else None
    wbs = Cout * Cw * KH * KW if sample_weight is not None else 0
    native.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding] == O.REPLICATE, O.fill_value(op, O.PADDINGS[padding], pv, x.numpy().dtype), xd, wd, wbs,
                          out, idx, (B, Cin, Cout, Cw, H, W, KH, KW))
    torch.cuda.synchronize()
    return _np(out), (None if idx is None else _np(idx))


SHAPES = [
    # B, Cin, Cout, H, W, KH, KW
    (2, 3, 5, 19, 70, 3, 5),   # two column tiles, ragged rows
    (1, 2, 2, 7, 9, 4, 2),     # even kernel sizes
    (1, 1, 3, 3, 4, 5, 5),     # kernel larger than the image
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("padding", PADDINGS)
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_forward_bit_exact(op, merge, padding, dtype):
    for si, (B, Cin, Cout, H, W, KH, KW) in enumerate(SHAPES):
        if merge == "identity":
            Cout = Cin
        x = seeded(10 + si, B, Cin, H, W, dtype=dtype, kind="randn")
        w = seeded(20 + si, *_weight_shape(merge, Cin, Cout, KH, KW), dtype=dtype, kind="randn", scale=0.3)
        save = merge in ("max", "min")
        out, idx = kernel_forward(op, merge, padding, 0.25, x, w, save=save)
        ref, ref_idx = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], 0.25, x.numpy(), w.numpy(), save_indices=save)
        assert np.array_equal(out, ref), f"shape {si}: forward differs"
        assert np.array_equal(np.signbit(out), np.signbit(ref))
        if save:
            assert np.array_equal(idx, ref_idx), f"shape {si}: indices differ"


@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
@pytest.mark.parametrize("merge", ["max", "min", "sum", "identity"])
def test_forward_ties_and_signed_zeros(op, merge):
    """Quantised inputs with a zero structuring element: every window ties; the first tap and the
    first channel must win, and a zero result keeps the sign of the first zero tap."""
    B, Cin, Cout, H, W, K = 2, 4, 3, 21, 66, 5
    if merge == "identity":
        Cout = Cin
    x = seeded(1, B, Cin, H, W, kind="quant")
    x[:, :, ::3, ::2] = -0.0
    x[:, 1:, 5:9, 10:30] = 0.0
    w = torch.zeros(_weight_shape(merge, Cin, Cout, K, K))
    w[..., 0, 0] = -0.0
    for padding in PADDINGS:
        save = merge in ("max", "min")
        out, idx = kernel_forward(op, merge, padding, 0.0, x, w, save=save)
        ref, ref_idx = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], 0.0, x.numpy(), w.numpy(), save_indices=save)
        assert np.array_equal(out, ref)
        assert np.array_equal(np.signbit(out), np.signbit(ref)), padding
        if save:
            assert np.array_equal(idx, ref_idx), padding


def _backward_case(op, merge, padding, dtype, x, w, g, save_indices=True, pv=0.5):
    """Forward + backward through torch.ops.morphocore on the GPU vs the oracle."""
    _mca()
    dev = torch.device("cuda")
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    fn = torch.ops.morphocore.dilation if op == O.DILATION else torch.ops.morphocore.erosion
    out = fn(xd, wd, O.MERGES[merge], O.PADDINGS[padding], pv, save_indices, 0.0)
    out.backward(g.to(dev))
    ref, ref_idx = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], pv, x.numpy(), w.numpy(), save_indices=merge in ("max", "min"))
    gx, gw = O.morpho_backward(op, O.MERGES[merge], O.PADDINGS[padding], pv, x.numpy(), w.numpy(), g.numpy(), indices=ref_idx)
    return _np(out), ref, _np(xd.grad), gx, _np(wd.grad), gw


@pytest.mark.parametrize("merge,K,dtype", [("max", 3, torch.float32), ("min", 5, torch.float32), ("sum", 3, torch.float32),
                                           ("mean", 5, torch.float32), ("identity", 3, torch.float32),
                                           ("identity", 3, torch.float64), ("max", 11, torch.float32)])
def test_forward_backward_large_grid(merge, K, dtype):
    """Launches of at least 1024 workgroups, which take the forward's full launch shape (4 rows per
    wave, 4 or 2 output channels per workgroup, IDENTITY 8 channels per workgroup with a partial last
    group) rather than the small-grid one that the smaller cases here use: values and winners bit
    exact, gradients within tolerance."""
    B, Cin, Cout, H, W = 4, 2, 16, 256, 256
    if merge == "identity":
        B, Cin, H, W = 6, 20, 256, 320
        Cout = Cin
    x = seeded(41, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(42, *_weight_shape(merge, Cin, Cout, K, K), dtype=dtype, kind="randn", scale=0.2)
    g = seeded(43, B, Cout, H, W, dtype=dtype, kind="randn")
    out, ref, gx, rgx, gw, rgw = _backward_case(O.DILATION, merge, "replicate", dtype, x, w, g)
    assert np.array_equal(out, ref)
    assert normwise_error(gx, rgx) <= TOL[dtype]
    assert normwise_error(gw, rgw) <= TOL[dtype]
    if merge in ("max", "min"):
        kout, kidx = kernel_forward(O.DILATION, merge, "replicate", 0.5, x, w, save=True)
        _, ridx = O.morpho_forward(O.DILATION, O.MERGES[merge], O.REPLICATE, 0.5, x.numpy(), w.numpy(), save_indices=True)
        assert np.array_equal(kout, ref) and np.array_equal(kidx, ridx)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("padding", ["geodesic", "replicate", "constant"])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_backward_parity(op, merge, padding, dtype):
    B, Cin, Cout, H, W, KH, KW = 2, 3, 4, 23, 69, 5, 3
    if merge == "identity":
        Cout = Cin
    x = seeded(3, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(4, *_weight_shape(merge, Cin, Cout, KH, KW), dtype=dtype, kind="randn", scale=0.2)
    g = seeded(5, B, Cout, H, W, dtype=dtype, kind="randn")
    out, ref, gx, rgx, gw, rgw = _backward_case(op, merge, padding, dtype, x, w, g)
    assert np.array_equal(out, ref)
    assert normwise_error(gx, rgx) <= TOL[dtype]
    assert normwise_error(gw, rgw) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("merge", ["sum", "mean"])
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
@pytest.mark.parametrize(
    "shape",
    [
        (2, 3, 7, 37, 70, 5, 5),  # 16-row planes, grad_weight flushed in chunks of 3 output channels
        (2, 2, 3, 19, 130, 3, 3),  # 16-row planes, one chunk
        (1, 2, 5, 19, 66, 7, 7),  # 8-row planes
        (1, 2, 3, 30, 70, 11, 11),  # one shared tile per channel (planes do not fit)
        (2, 1, 1, 17, 64, 5, 1),  # single channels, one-column element
        (1, 4, 9, 20, 130, 1, 5),  # one-row element
    ],
)
def test_backward_parity_kernel_variants(shape, op, merge, dtype):
    """Per-pair merges through each backward kernel layout the launch can choose."""
    B, Cin, Cout, H, W, KH, KW = shape
    x = seeded(41, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(42, *_weight_shape(merge, Cin, Cout, KH, KW), dtype=dtype, kind="randn", scale=0.2)
    g = seeded(43, B, Cout, H, W, dtype=dtype, kind="randn")
    for padding in ("replicate", "geodesic"):
        out, ref, gx, rgx, gw, rgw = _backward_case(op, merge, padding, dtype, x, w, g)
        assert np.array_equal(out, ref), padding
        assert normwise_error(gx, rgx) <= TOL[dtype], padding
        assert normwise_error(gw, rgw) <= TOL[dtype], padding


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
@pytest.mark.parametrize(
    "shape",
    [
        (2, 3, 37, 70, 3, 3),  # gathered grad_input
        (1, 4, 19, 130, 5, 5),  # gathered grad_input
        (1, 2, 19, 66, 7, 7),  # scattered (shared tile per channel)
        (1, 2, 20, 70, 5, 3),  # scattered
        (1, 1, 3, 4, 5, 5),  # element larger than the image
    ],
)
def test_backward_parity_identity_variants(shape, op, dtype):
    B, C, H, W, KH, KW = shape
    x = seeded(44, B, C, H, W, dtype=dtype, kind="randn")
    w = seeded(45, *_weight_shape("identity", C, C, KH, KW), dtype=dtype, kind="randn", scale=0.2)
    g = seeded(46, B, C, H, W, dtype=dtype, kind="randn")
    for padding in PADDINGS:
        out, ref, gx, rgx, gw, rgw = _backward_case(op, "identity", padding, dtype, x, w, g)
        assert np.array_equal(out, ref), padding
        assert normwise_error(gx, rgx) <= TOL[dtype], padding
        assert normwise_error(gw, rgw) <= TOL[dtype], padding


@pytest.mark.parametrize("save_indices", [True, False])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_backward_exact_on_dyadic_inputs(op, merge, save_indices):
    """Quantised inputs, zero structuring element, integer gradients: every sum is exact, so the
    gradients must match bit for bit whatever the accumulation order."""
    B, Cin, Cout, H, W, K = 2, 3, 4, 20, 70, 5
    if merge == "identity":
        Cout = Cin
    x = seeded(6, B, Cin, H, W, kind="quant")
    w = torch.zeros(_weight_shape(merge, Cin, Cout, K, K))
    g = seeded(7, B, Cout, H, W, kind="quant") * 16 - 8
    # 'mean' scales by the rounded 1 / Cin, which makes its sums inexact: checked norm-wise.
    out, ref, gx, rgx, gw, rgw = _backward_case(op, merge, "replicate", torch.float32, x, w, g, save_indices=save_indices)
    assert np.array_equal(out, ref)
    if merge == "mean":
        assert normwise_error(gx, rgx) <= 1e-6 and normwise_error(gw, rgw) <= 1e-6
    else:
        assert np.array_equal(gx, rgx)
        assert np.array_equal(gw, rgw)


def test_backward_geodesic_minus_inf_weights():
    """Dropped taps (-inf) with geodesic padding: windows that see only -inf route to tap 0, as the
    strict-improvement scan leaves it (reference test_weight_dropout.py:107-139)."""
    x = seeded(8, 1, 2, 9, 11, kind="randn")
    w = seeded(9, 3, 2, 3, 3, kind="randn")
    w[:, :, 0, :] = -float("inf")
    w[0, 1] = -float("inf")
    g = seeded(10, 1, 3, 9, 11, kind="randn")
    for merge in ("max", "sum", "min"):
        out, ref, gx, rgx, gw, rgw = _backward_case(O.DILATION, merge, "geodesic", torch.float32, x, w, g)
        assert np.array_equal(out, ref)
        assert normwise_error(gx, rgx) <= 1e-6
        assert normwise_error(gw, rgw) <= 1e-6


def test_noise_matches_per_sample_weights():
    """Weight noise (morpho_op_wrap.hxx:55-64): the same draw, reproduced from the seed, fed to the
    oracle as per-sample weights, gives the same output and gradients."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    B, Cin, Cout, H, W, K = 3, 2, 4, 17, 20, 3
    x = seeded(11, B, Cin, H, W)
    w = seeded(12, Cout, Cin, K, K, kind="randn", scale=0.1)
    g = seeded(13, B, Cout, H, W, kind="randn")
    for merge in ("max", "sum"):
        xd = x.to(dev).requires_grad_(True)
        wd = w.to(dev).requires_grad_(True)
        torch.manual_seed(1234)
        out = mca.functional.dilation(xd, wd, merge, "geodesic", training=True, noise_scale=0.05)
        out.backward(g.to(dev))
        torch.manual_seed(1234)
        noise = (torch.rand((B, Cout, Cin, K, K), dtype=torch.float32, device=dev) * 2.0 - 1.0) * 0.05
        sample = (wd.detach().unsqueeze(0) + noise).cpu().numpy()
        ref, idx = O.morpho_forward(O.DILATION, O.MERGES[merge], O.GEODESIC, 0.0, x.numpy(), w.numpy(), save_indices=merge == "max",
                                    sample_weight=sample)
        gx, gw = O.morpho_backward(O.DILATION, O.MERGES[merge], O.GEODESIC, 0.0, x.numpy(), w.numpy(), g.numpy(), indices=idx,
                                   sample_weight=sample)
        assert np.array_equal(_np(out), ref)
        assert normwise_error(_np(xd.grad), gx) <= 1e-6
        assert normwise_error(_np(wd.grad), gw) <= 1e-6


def test_ranks_2d_3d():
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    x = seeded(14, 13, 4).to(dev)
    w = seeded(15, 5, 5, kind="randn").to(dev)
    out = mca.functional.dilation(x, w, "max", "geodesic")
    assert out.shape == (13, 4)
    ref, _ = O.morpho_forward(O.DILATION, O.MAX, O.GEODESIC, 0.0, _np(x)[None, None], _np(w)[None, None])
    assert np.array_equal(_np(out), ref[0, 0])
    x3 = seeded(16, 2, 10, 12).to(dev)
    w4 = seeded(17, 3, 2, 3, 3, kind="randn").to(dev)
    out3 = mca.functional.erosion(x3, w4, "sum")
    assert out3.shape == (3, 10, 12)


def test_functional_erosion_flips_weight():
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    x = seeded(18, 2, 3, 15, 16)
    w = seeded(19, 4, 3, 3, 5, kind="randn", scale=0.1)
    out = mca.functional.erosion(x.to(dev), w.to(dev), "min", "zero")
    ref, _ = O.morpho_forward(O.EROSION, O.MIN, O.ZERO, 0.0, x.numpy(), np.ascontiguousarray(w.flip((-2, -1)).numpy()))
    assert np.array_equal(_np(out), ref)


# ------------------------------------------------------------------------------------------------
# Smorph
# ------------------------------------------------------------------------------------------------

def _smorph_case(merge, x, w_tilde, alpha, g):
    _mca()
    dev = torch.device("cuda")
    xd = x.to(dev).requires_grad_(True)
    wd = w_tilde.to(dev).requires_grad_(True)
    ad = alpha.to(dev).requires_grad_(True)
    out = torch.ops.morphocore.smorph(xd, wd, ad, O.MERGES[merge])
    out.backward(g.to(dev))
    ref = O.smorph_forward(O.MERGES[merge], x.numpy(), w_tilde.numpy(), alpha.numpy())
    gx, gw, ga = O.smorph_backward(O.MERGES[merge], x.numpy(), w_tilde.numpy(), alpha.numpy(), g.numpy())
    return (_np(out), ref), (_np(xd.grad), gx), (_np(wd.grad), gw), (_np(ad.grad), ga)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("a", [-20.0, -1.0, 0.0, 1.0, 20.0])
@pytest.mark.parametrize("merge", MERGES)
def test_smorph_parity(merge, a, dtype):
    B, Cin, Cout, H, W, K = 2, 3, 4, 18, 67, 5
    if merge == "identity":
        Cout = Cin
    x = seeded(21, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(22, *_weight_shape(merge, Cin, Cout, K, K), dtype=dtype, kind="randn", scale=0.1)
    pairs = Cout if merge == "identity" else Cout * Cin
    alpha = (torch.full((pairs,), a, dtype=dtype) + seeded(23, pairs, dtype=dtype, kind="randn", scale=0.1 if a != 0 else 0.0))
    alpha = alpha.reshape((Cout,) if merge == "identity" else (Cout, Cin))
    g = seeded(24, B, Cout, H, W, dtype=dtype, kind="randn")
    for actual, expected in _smorph_case(merge, x, w, alpha, g):
        assert normwise_error(actual, expected) <= TOL[dtype]


@pytest.mark.parametrize("saved", [True, False], ids=["saved-stats", "recomputed"])
@pytest.mark.parametrize("a", [-20.0, 0.5, 20.0])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("K,H", [(3, 14), (7, 24), (11, 30)])
def test_smorph_static_interior_and_border_tiles(K, H, merge, a, saved, monkeypatch):
    """The float32 static smorph kernels at 3x3 / 7x7 / 11x11 on images wide and tall enough that
    some 64 x 4 tiles lie inside the image (the unmasked path) next to border tiles (masked), with a
    partial last tile in both directions; the backward from the forward's saved pair statistics, and
    recomputing them (saving disabled)."""
    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", str(1 << 40) if saved else "0")
    B, Cin, Cout, W = 1, 2, 3, 200
    if merge == "identity":
        Cout = Cin
    x = seeded(31, B, Cin, H, W, kind="randn")
    w = seeded(32, *_weight_shape(merge, Cin, Cout, K, K), kind="randn", scale=0.1)
    pairs = Cout if merge == "identity" else Cout * Cin
    alpha = torch.full((pairs,), a) + seeded(33, pairs, kind="randn", scale=0.1)
    alpha = alpha.reshape((Cout,) if merge == "identity" else (Cout, Cin))
    g = seeded(34, B, Cout, H, W, kind="randn")
    for actual, expected in _smorph_case(merge, x, w, alpha, g):
        assert normwise_error(actual, expected) <= 1e-6


@pytest.mark.parametrize("alphas", ["mixed", "zero"], ids=["alpha-2-3", "alpha-0-3"])
@pytest.mark.parametrize("saved", [True, False], ids=["saved-stats", "recomputed"])
@pytest.mark.parametrize("merge", ["sum", "max", "identity"])
@pytest.mark.parametrize("K", [3, 7])
def test_smorph_static_nan_input(K, merge, saved, alphas, monkeypatch):
    """An in-image NaN in the input propagates through the float32 static smorph kernels as through
    the reference (its window's pair outputs, and the gradients they route, are NaN; NaN never wins
    the window's extremum, nor the MAX merge), on interior and border tiles; every finite value
    within tolerance. The "zero" case gives every other pair alpha = 0, whose exponentials the
    kernels take without evaluating the exponential."""
    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", str(1 << 40) if saved else "0")
    B, Cin, Cout, H, W = 1, 2, 3, 20, 200
    if merge == "identity":
        Cout = Cin
    x = seeded(51, B, Cin, H, W, kind="randn")
    x[0, 0, 9, 100] = float("nan")  # an interior tile
    x[0, 1, 0, 3] = float("nan")  # a border tile, next to the image corner
    w = seeded(52, *_weight_shape(merge, Cin, Cout, K, K), kind="randn", scale=0.1)
    pairs = Cout if merge == "identity" else Cout * Cin
    alpha = torch.where(torch.arange(pairs) % 2 == 0, 2.0 if alphas == "mixed" else 0.0, -3.0)
    alpha = alpha.reshape((Cout,) if merge == "identity" else (Cout, Cin))
    g = seeded(53, B, Cout, H, W, kind="randn")
    results = _smorph_case(merge, x, w, alpha, g)
    # The oracle's output holds NaN, except under MAX, whose merge never picks a NaN channel.
    assert np.isnan(results[0][1]).any() == (merge != "max")
    for actual, expected in results:
        assert normwise_error(actual, expected) <= 1e-6


def test_smorph_saves_statistics_only_for_a_backward(monkeypatch):
    """The forward keeps the pair statistics only when a backward can follow (grad mode on and an
    input that requires grad), within the per-call cap; they live as long as the autograd graph that
    holds them; the results do not depend on them."""
    mca, native, _ = _mca()
    from morphocore_amd import _C

    dev = torch.device("cuda")
    live = lambda: _C.saved_stats_live_bytes(torch.cuda.current_device())  # noqa: E731
    base = live()
    x = seeded(61, 1, 2, 12, 70, kind="randn").to(dev)
    w = seeded(62, 3, 2, 3, 3, kind="randn", scale=0.1).to(dev)
    alpha = torch.full((3, 2), 2.0, device=dev)
    nbytes = native.smorph_stats_bytes(2, torch.float32, (1, 2, 3, 2, 12, 70, 3, 3))
    assert nbytes == 12 * 3 * 2 * 12 * 70
    with torch.no_grad():
        y0 = mca.functional.smorph(x, w, alpha, channel_merge_mode="sum")
    assert live() == base
    y1 = mca.functional.smorph(x, w, alpha, channel_merge_mode="sum")  # nothing requires grad
    assert live() == base
    xr = x.clone().requires_grad_(True)
    y2 = mca.functional.smorph(xr, w, alpha, channel_merge_mode="sum")
    assert live() == base + nbytes
    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", "0")
    y3 = mca.functional.smorph(xr, w, alpha, channel_merge_mode="sum")
    assert live() == base + nbytes
    for y in (y1, y2, y3):
        assert torch.equal(y, y0)
    del y2
    assert live() == base


def test_smorph_stack_saved_statistics_budget(monkeypatch):
    """One budget for every live saved-statistics buffer of the process: in a 3-layer smorph stack
    whose budget holds two layers' statistics, the third layer's backward recomputes them, and the
    outputs and gradients are those of a run that saves every layer's (within the tolerance: the two
    backwards add the same terms in different orders)."""
    mca, native, _ = _mca()
    from morphocore_amd import _C

    dev = torch.device("cuda")
    live = lambda: _C.saved_stats_live_bytes(torch.cuda.current_device())  # noqa: E731
    C, H, W, K = 4, 24, 70, 5
    nbytes = native.smorph_stats_bytes(2, torch.float32, (2, C, C, C, H, W, K, K))
    x = seeded(71, 2, C, H, W, kind="randn").to(dev)
    ws = [seeded(72 + l, C, C, K, K, kind="randn", scale=0.1).to(dev) for l in range(3)]
    alphas = [torch.full((C, C), a, device=dev) for a in (1.5, -2.0, 3.0)]
    g = seeded(79, 2, C, H, W, kind="randn").to(dev)

    def run():
        xr = x.clone().requires_grad_(True)
        wr = [w.clone().requires_grad_(True) for w in ws]
        base = live()
        y = xr
        saved = []
        for wl, al in zip(wr, alphas):
            y = mca.functional.smorph(y, wl, al, channel_merge_mode="sum")
            saved.append(live() - base)
        y.backward(g)
        return y.detach(), [xr.grad] + [wl.grad for wl in wr], saved

    y_all, g_all, saved_all = run()
    assert saved_all == [nbytes, 2 * nbytes, 3 * nbytes]
    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_BUDGET", str(live() + 2 * nbytes + nbytes // 2))
    y_two, g_two, saved_two = run()
    assert saved_two == [nbytes, 2 * nbytes, 2 * nbytes]
    assert torch.equal(y_two, y_all)
    for a, b in zip(g_two, g_all):
        assert normwise_error(a.cpu().numpy(), b.cpu().numpy()) <= 1e-6


def _window_extremum(x, w, dilation_like):
    """ref of every pair and pixel, (B, Cout, Cin, H, W): the extremum of x[y + KH/2 - kh, c + KW/2 - kw]
    + w[kh, kw] over the in-image taps (one rounding per tap, so exact in float32)."""
    B, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    PH, PW = KH // 2, KW // 2  # odd sizes: KH = 2 PH + 1
    fill = -np.inf if dilation_like else np.inf
    xp = np.full((B, Cin, H + 2 * PH, W + 2 * PW), fill, dtype=np.float32)
    xp[:, :, PH:PH + H, PW:PW + W] = x
    best = np.full((B, Cout, Cin, H, W), fill, dtype=np.float32)
    for kh in range(KH):
        for kw in range(KW):
            # Input row y + PH - kh sits at padded row y + 2 PH - kh.
            oy, ox = 2 * PH - kh, 2 * PW - kw
            win = xp[:, None, :, oy:oy + H, ox:ox + W] + w[None, :, :, kh, kw, None, None]
            best = np.maximum(best, win) if dilation_like else np.minimum(best, win)
    return best


@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("K", [3, 7, 11])
def test_smorph_saved_stats_abi(K, merge):
    """mca_smorph_forward_stats_f32 / mca_smorph_backward_stats_f32 through the C ABI: the output is
    bit for bit the plain forward's; the saved ref is the window's extremum; W / S merges to the
    output (MAX / MIN / IDENTITY exactly); the backward from the statistics matches the oracle and the
    recomputing backward."""
    _, native, _ = _mca()
    dev = torch.device("cuda")
    B, Cin, Cout, H, W = 2, 3, 4, 21, 70
    if merge == "identity":
        Cout = Cin
    x = seeded(41, B, Cin, H, W, kind="randn")
    w = seeded(42, *_weight_shape(merge, Cin, Cout, K, K), kind="randn", scale=0.1)
    pairs = Cout if merge == "identity" else Cout * Cin
    # Dilation-like and erosion-like pairs side by side.
    alpha = torch.where(torch.arange(pairs) % 2 == 0, 3.0, -2.0) + seeded(43, pairs, kind="randn", scale=0.1)
    g = seeded(44, B, Cout, H, W, kind="randn")
    m = O.MERGES[merge]
    geom = (B, Cin, Cout, w.shape[1], H, W, K, K)
    nbytes = native.smorph_stats_bytes(m, torch.float32, geom)
    P = 1 if merge == "identity" else Cin
    assert nbytes == 12 * B * Cout * P * H * W
    xd, wd, ad, gd = x.to(dev), w.to(dev), alpha.to(dev), g.to(dev)
    stats = torch.full((nbytes // 4,), float("nan"), device=dev)
    out0 = torch.empty((B, Cout, H, W), device=dev)
    out1 = torch.empty_like(out0)
    native.smorph_forward(m, xd, wd, ad, out0, geom)
    native.smorph_forward(m, xd, wd, ad, out1, geom, stats=stats)
    out = _np(out1)
    assert np.array_equal(_np(out0), out)
    ref, inv, outp = (a.reshape(B, Cout, P, H, W) for a in _np(stats).reshape(3, -1))
    assert np.isfinite(ref).all() and np.isfinite(inv).all() and np.isfinite(outp).all()
    # ref: per pair, the extremum its alpha's sign selects.
    a_np = alpha.numpy().reshape(Cout, P)
    w_np = w.numpy()
    if merge == "identity":
        ext_d = np.stack([_window_extremum(x.numpy()[:, c:c + 1], w_np[c:c + 1], True)[:, 0, 0] for c in range(Cin)], axis=1)[:, :, None]
        ext_e = np.stack([_window_extremum(x.numpy()[:, c:c + 1], w_np[c:c + 1], False)[:, 0, 0] for c in range(Cin)], axis=1)[:, :, None]
    else:
        ext_d, ext_e = _window_extremum(x.numpy(), w_np, True), _window_extremum(x.numpy(), w_np, False)
    want = np.where((a_np >= 0)[None, :, :, None, None], ext_d, ext_e)
    assert np.array_equal(ref, want)
    if merge == "max":
        assert np.array_equal(outp.max(axis=2), out)
    elif merge == "min":
        assert np.array_equal(outp.min(axis=2), out)
    elif merge == "identity":
        assert np.array_equal(outp[:, :, 0], out)
    else:
        total = outp.astype(np.float64).sum(axis=2) / (Cin if merge == "mean" else 1)
        assert normwise_error(out, total) <= 1e-6
    # Backward from the statistics, against the oracle and against the recomputing backward.
    rgx, rgw, rga = O.smorph_backward(m, x.numpy(), w_np, alpha.numpy(), g.numpy())
    grads = []
    for st in (stats, None):
        gx, gw, ga = torch.empty_like(xd), torch.empty_like(wd), torch.empty_like(ad)
        native.smorph_backward(m, xd, wd, ad, out1, gd, gx, gw, ga, geom, stats=st)
        grads.append((_np(gx), _np(gw), _np(ga)))
    for got in grads:
        for actual, expected in zip(got, (rgx, rgw, rga)):
            assert normwise_error(actual, expected) <= 1e-6
    for a1, a0 in zip(*grads):
        assert normwise_error(a1, a0) <= 1e-6


@pytest.mark.parametrize("merge", ["sum", "max"])
def test_smorph_shared_alpha(merge):
    x = seeded(25, 1, 2, 11, 13, kind="randn")
    w = seeded(26, 3, 2, 3, 3, kind="randn", scale=0.1)
    alpha = torch.tensor(2.5)
    g = seeded(27, 1, 3, 11, 13, kind="randn")
    for actual, expected in _smorph_case(merge, x, w, alpha, g):
        assert normwise_error(actual, expected) <= 1e-6


def test_smorph_functional_matches_blend():
    """functional.smorph blends w with its flip by tanh(alpha) before the operator (smorph.py:56-70)."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    x = seeded(28, 2, 3, 16, 16, kind="randn")
    w = seeded(29, 4, 3, 5, 5, kind="randn", scale=0.1)
    alpha = seeded(30, 4, 3, kind="randn")
    out = mca.functional.smorph(x.to(dev), w.to(dev), alpha.to(dev), channel_merge_mode="mean")
    wt = O.smorph_w_tilde(w.numpy(), alpha.numpy(), "mean")
    ref = O.smorph_forward(O.AVERAGE, x.numpy(), wt, alpha.numpy())
    assert normwise_error(_np(out), ref) <= 1e-6


# ------------------------------------------------------------------------------------------------
# The benchmark configurations (configs[0..4]), at sizes the oracle finishes in seconds
# ------------------------------------------------------------------------------------------------

def test_config1_dilation_max_full_size():
    """dilation fwd+bwd fp32, merge 'max', x (4,3,64,64) ~U[0,1), w (16,3,3,3) ~N(0,0.1), seed 0."""
    torch.manual_seed(0)
    x = torch.rand(4, 3, 64, 64)
    w = torch.randn(16, 3, 3, 3) * 0.1
    g = seeded(1, 4, 16, 64, 64, kind="randn")
    out, ref, gx, rgx, gw, rgw = _backward_case(O.DILATION, "max", "replicate", torch.float32, x, w, g)
    assert np.array_equal(out, ref)
    assert normwise_error(gx, rgx) <= 1e-6 and normwise_error(gw, rgw) <= 1e-6
    o2, idx = kernel_forward(O.DILATION, "max", "replicate", 0.0, x, w, save=True)
    _, ridx = O.morpho_forward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x.numpy(), w.numpy(), save_indices=True)
    assert np.array_equal(idx, ridx)


@pytest.mark.parametrize("variant", ["random", "quantised"])
def test_config2_erosion_sum(variant):
    """configs[1] at B=2: erosion fp32, merge 'sum', (2,32,128,128), w (32,32,5,5) ~N(0,0.05); the
    quantised variant has x in {0..15}/16 and w = 0."""
    x = seeded(0, 2, 32, 128, 128, kind="quant" if variant == "quantised" else "rand")
    w = torch.zeros(32, 32, 5, 5) if variant == "quantised" else seeded(1, 32, 32, 5, 5, kind="randn", scale=0.05)
    g = seeded(2, 2, 32, 128, 128, kind="quant") * 16 - 8 if variant == "quantised" else seeded(2, 2, 32, 128, 128, kind="randn")
    out, ref, gx, rgx, gw, rgw = _backward_case(O.EROSION, "sum", "replicate", torch.float32, x, w, g)
    assert np.array_equal(out, ref)
    if variant == "quantised":
        assert np.array_equal(gx, rgx) and np.array_equal(gw, rgw)
    else:
        assert normwise_error(gx, rgx) <= 1e-6 and normwise_error(gw, rgw) <= 1e-6


@pytest.mark.parametrize("a", [-20.0, -1.0, 0.0, 1.0, 20.0])
def test_config3_smorph_mean(a):
    """configs[2] with its channel counts, Cin = Cout = 64, at a small image (1, 64, 24, 70): w (64,64,7,7)
    ~N(0,0.1), alpha = full(a)."""
    x = seeded(0, 1, 64, 24, 70, kind="randn")
    w = seeded(1, 64, 64, 7, 7, kind="randn", scale=0.1)
    alpha = torch.full((64, 64), a)
    wt = torch.from_numpy(O.smorph_w_tilde(w.numpy(), alpha.numpy(), "mean"))
    g = seeded(2, 1, 64, 24, 70, kind="randn")
    for actual, expected in _smorph_case("mean", x, wt, alpha, g):
        assert normwise_error(actual, expected) <= 1e-6


def test_config4_dilation_identity_f64():
    """configs[3] with its 128 channels at (4,128,112,112) float64, identity, w (128,1,3,3) ~N(0,0.1);
    the literal (C,C,3,3) weight is rejected as by the reference."""
    x = seeded(0, 4, 128, 112, 112, dtype=torch.float64, low=-1.0, scale=2.0)
    w = seeded(1, 128, 1, 3, 3, dtype=torch.float64, kind="randn", scale=0.1)
    g = seeded(2, 4, 128, 112, 112, dtype=torch.float64, kind="randn")
    out, ref, gx, rgx, gw, rgw = _backward_case(O.DILATION, "identity", "replicate", torch.float64, x, w, g)
    assert np.array_equal(out, ref)
    assert normwise_error(gx, rgx) <= 1e-12 and normwise_error(gw, rgw) <= 1e-12
    with pytest.raises(RuntimeError, match="Identity mode requires weight.shape\\[1\\] == 1"):
        torch.ops.morphocore.dilation(x.cuda(), torch.zeros(128, 128, 3, 3, dtype=torch.float64, device="cuda"), 5, 3, 0.0, True, 0.0)


def test_config5_stack_reduced():
    """configs[4] at (1,4,40,40), K=11: dilation(max) -> smorph(alpha=5, sum) -> erosion(min), fwd+bwd."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    C, K = 4, 11
    x = seeded(0, 1, C, 40, 40)
    ws = [seeded(1 + l, C, C, K, K, kind="randn", scale=0.05) for l in range(3)]
    alpha = torch.full((C, C), 5.0)
    g = seeded(9, 1, C, 40, 40, kind="randn")
    # GPU, through the public API.
    xd = x.to(dev).requires_grad_(True)
    wd = [w.to(dev).requires_grad_(True) for w in ws]
    ad = alpha.to(dev).requires_grad_(True)
    y1 = mca.functional.dilation(xd, wd[0], "max", "replicate")
    y1.retain_grad()
    y2 = mca.functional.smorph(y1, wd[1], ad, channel_merge_mode="sum")
    y2.retain_grad()
    y3 = mca.functional.erosion(y2, wd[2], "min", "replicate")
    y3.backward(g.to(dev))
    # Oracle, layer by layer, with the GPU's own intermediate activations as inputs so that each
    # layer is checked at its own tolerance.
    r1, i1 = O.morpho_forward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x.numpy(), ws[0].numpy(), save_indices=True)
    assert np.array_equal(_np(y1), r1)
    wt = O.smorph_w_tilde(ws[1].numpy(), alpha.numpy(), "sum")
    r2 = O.smorph_forward(O.ADD, _np(y1), wt, alpha.numpy())
    assert normwise_error(_np(y2), r2) <= 1e-6
    w3f = np.ascontiguousarray(ws[2].flip((-2, -1)).numpy())
    r3, i3 = O.morpho_forward(O.EROSION, O.MIN, O.REPLICATE, 0.0, _np(y2), w3f, save_indices=True)
    assert np.array_equal(_np(y3), r3)
    # Backward, layer by layer from the top, each layer fed the GPU's own output gradient.
    gy2, gw3f = O.morpho_backward(O.EROSION, O.MIN, O.REPLICATE, 0.0, _np(y2), w3f, g.numpy(), indices=i3)
    assert normwise_error(_np(wd[2].grad), gw3f[:, :, ::-1, ::-1]) <= 1e-6
    assert normwise_error(_np(y2.grad), gy2) <= 1e-6
    gy1, gwt, ga_direct = O.smorph_backward(O.ADD, _np(y1), wt, alpha.numpy(), _np(y2.grad))
    assert normwise_error(_np(y1.grad), gy1) <= 1e-6
    # w~ -> (w1, alpha) through torch on the CPU (functional/smorph.py:56-70), plus alpha's direct term.
    w1c, ac = ws[1].clone().requires_grad_(True), alpha.clone().requires_grad_(True)
    t = torch.tanh(ac).unsqueeze(-1).unsqueeze(-1)
    wtt = t * ((1 - t) / 2 * w1c.flip(dims=(-2, -1)) + (1 + t) / 2 * w1c)
    torch.autograd.backward([wtt, ac], [torch.from_numpy(gwt), torch.from_numpy(ga_direct)])
    assert normwise_error(_np(wd[1].grad), w1c.grad.numpy()) <= 1e-6
    assert normwise_error(_np(ad.grad), ac.grad.numpy()) <= 1e-6
    gx, gw0 = O.morpho_backward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x.numpy(), ws[0].numpy(), _np(y1.grad), indices=i1)
    assert normwise_error(_np(xd.grad), gx) <= 1e-6
    assert normwise_error(_np(wd[0].grad), gw0) <= 1e-6


# ------------------------------------------------------------------------------------------------
# Full benchmark sizes: size-independent properties
# ------------------------------------------------------------------------------------------------

def test_config2_full_size_properties():
    """configs[1] at full size (16,32,128,128): batch element 0 matches the oracle exactly; with an
    all-ones output gradient, every (o, i) pair routes each pixel's gradient to exactly one tap, so
    each grad_weight[o, i] sums to -B*H*W (erosion sign), exactly."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    x = seeded(0, 16, 32, 128, 128)
    w = seeded(1, 32, 32, 5, 5, kind="randn", scale=0.05)
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    out = mca.functional.erosion(xd, wd, "sum", "replicate")
    out.backward(torch.ones_like(out))
    ref, _ = O.morpho_forward(O.EROSION, O.ADD, O.REPLICATE, 0.0, x[:1].numpy(), np.ascontiguousarray(w.flip((-2, -1)).numpy()))
    assert np.array_equal(_np(out[:1]), ref)
    row_sums = wd.grad.double().sum(dim=(2, 3))
    assert torch.equal(row_sums, torch.full_like(row_sums, -16 * 128 * 128))
    # Every input pixel's gradient counts the (o, pixel) pairs that picked it: a non-negative integer.
    gx = xd.grad
    assert torch.equal(gx, gx.round()) and bool((gx >= 0).all())
    assert float(gx.double().sum()) <= 16 * 32 * 32 * 128 * 128


@pytest.mark.parametrize("merge,K,a", [("mean", 7, 1.0), ("mean", 7, -20.0), ("sum", 11, 5.0), ("max", 5, 3.0), ("identity", 7, -1.0)])
def test_smorph_large_grid_saved_matches_recomputed(merge, K, a, monkeypatch):
    """At a size with thousands of workgroups (configs[2]-like channels, 160 x 200 images), the
    backward from saved statistics (two rows per wave) and the recomputing backward (one row per
    wave) are independent kernels: their forward outputs are bit for bit equal and their gradients
    agree to the float32 tolerance; batch element 0 of the forward matches the oracle."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    B, C, H, W = 2, 16, 160, 200
    x = seeded(71, B, C, H, W, kind="randn")
    w = seeded(72, *_weight_shape(merge, C, C, K, K), kind="randn", scale=0.1)
    pairs = C if merge == "identity" else C * C
    alpha = (torch.full((pairs,), a) + seeded(73, pairs, kind="randn", scale=0.05)).reshape((C,) if merge == "identity" else (C, C))
    g = seeded(74, B, C, H, W, kind="randn")
    results = []
    for limit in (str(1 << 40), "0"):
        monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", limit)
        xd = x.to(dev).requires_grad_(True)
        wd = w.to(dev).requires_grad_(True)
        ad = alpha.to(dev).requires_grad_(True)
        out = torch.ops.morphocore.smorph(xd, wd, ad, O.MERGES[merge])
        out.backward(g.to(dev))
        results.append((_np(out), _np(xd.grad), _np(wd.grad), _np(ad.grad)))
    saved, recomputed = results
    assert np.array_equal(saved[0], recomputed[0])
    for s_, r_ in zip(saved[1:], recomputed[1:]):
        assert normwise_error(s_, r_) <= 1e-6
    ref = O.smorph_forward(O.MERGES[merge], x[:1].numpy(), w.numpy(), alpha.numpy())
    assert normwise_error(saved[0][:1], ref) <= 1e-6
    # grad_input of batch element 0 depends on that element alone: the oracle's batch-1 backward.
    rgx, _, _ = O.smorph_backward(O.MERGES[merge], x[:1].numpy(), w.numpy(), alpha.numpy(), g[:1].numpy())
    assert normwise_error(saved[1][:1], rgx) <= 1e-6
    assert normwise_error(recomputed[1][:1], rgx) <= 1e-6


# ------------------------------------------------------------------------------------------------
# Saved per-pair taps (sum / mean / identity) and the recompute path
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("merge", ["sum", "identity"])
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
@pytest.mark.parametrize("shape", [(2, 3, 4, 21, 70, 3, 3), (1, 3, 5, 17, 66, 5, 5), (1, 2, 2, 9, 20, 7, 7), (1, 2, 3, 12, 11, 4, 2),
                                   (1, 2, 2, 30, 70, 11, 11)])
def test_saved_pair_taps_are_first_extremal_taps(op, merge, dtype, shape):
    """The taps the forward saves for the per-pair merges are each pair's first extremal tap (the
    strict scan of morpho_op_cpu_kernels.hxx:211-252), on quantised inputs full of ties."""
    _, native, _ = _mca()
    B, Cin, Cout, H, W, KH, KW = shape
    if merge == "identity":
        Cout = Cin
    x = seeded(31, B, Cin, H, W, dtype=dtype, kind="quant")
    w = (seeded(32, *_weight_shape(merge, Cin, Cout, KH, KW), dtype=dtype, kind="quant") * 4).round() / 4
    dev = torch.device("cuda")
    geom = (B, Cin, Cout, w.shape[1], H, W, KH, KW)
    nbytes = native.indices_bytes(O.MERGES[merge], geom)
    taps = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty((B, Cout, H, W), dtype=dtype, device=dev)
    native.morpho_forward(op, O.MERGES[merge], True, 0.0, x.to(dev), w.to(dev), 0, out, taps, geom)
    cpair = 1 if merge == "identity" else Cin
    got = _np(taps).reshape(B, Cout, cpair, H, W)
    xn, wn = x.numpy(), w.numpy()
    for b in range(B):
        for o in range(Cout):
            for c in range(cpair):
                i = o if merge == "identity" else c
                _, arg = O.brute.pair(xn[b, i], wn[o, c], op, O.REPLICATE, 0.0)
                assert np.array_equal(got[b, o, c], arg), (b, o, c)
    ref, _ = O.morpho_forward(op, O.MERGES[merge], O.REPLICATE, 0.0, xn, wn)
    assert np.array_equal(_np(out), ref)


@pytest.mark.parametrize("merge", MERGES)
def test_saved_and_recomputed_winners_give_the_same_gradients(merge):
    """save_indices=True (winners kept by the forward) and False (recomputed by the backward) give
    bit-identical gradients; so does a forward run without autograd."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    B, Cin, Cout, H, W, K = 2, 3, 4, 33, 65, 5
    if merge == "identity":
        Cout = Cin
    x = seeded(33, B, Cin, H, W).to(dev)
    w = seeded(34, *_weight_shape(merge, Cin, Cout, K, K), kind="randn", scale=0.1).to(dev)
    g = seeded(35, B, Cout, H, W, kind="quant").to(dev)
    grads = []
    for save in (True, False):
        xd = x.clone().requires_grad_(True)
        wd = w.clone().requires_grad_(True)
        out = mca.functional.erosion(xd, wd, merge, "replicate", save_indices=save)
        out.backward(g)
        grads.append((out.detach(), xd.grad, wd.grad))
    with torch.no_grad():
        plain = mca.functional.erosion(x, w, merge, "replicate")
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][0], plain)
    # Accumulation order of float atomics may differ between runs: compare within the contract.
    assert normwise_error(_np(grads[0][1]), _np(grads[1][1])) <= 1e-6
    assert normwise_error(_np(grads[0][2]), _np(grads[1][2])) <= 1e-6


@pytest.mark.parametrize("merge", ["sum", "mean", "identity"])
@pytest.mark.parametrize("K", [3, 7])
def test_recomputed_taps_in_batch_chunks(merge, K, monkeypatch):
    """Without saved taps the backward recomputes them a few batch elements at a time
    (MORPHOCORE_AMD_RECOMPUTE_BYTES bounds the buffer): one element per chunk gives the gradients of
    the whole-batch recomputation, and both match the oracle."""
    mca, _, _ = _mca()
    dev = torch.device("cuda")
    B, Cin, Cout, H, W = 5, 3, 4, 21, 70
    if merge == "identity":
        Cout = Cin
    x = seeded(36, B, Cin, H, W)
    w = seeded(37, *_weight_shape(merge, Cin, Cout, K, K), kind="randn", scale=0.1)
    g = seeded(38, B, Cout, H, W, kind="randn")
    grads = []
    for budget in (None, "1"):
        if budget is None:
            monkeypatch.delenv("MORPHOCORE_AMD_RECOMPUTE_BYTES", raising=False)
        else:
            monkeypatch.setenv("MORPHOCORE_AMD_RECOMPUTE_BYTES", budget)
        xd = x.to(dev).requires_grad_(True)
        wd = w.to(dev).requires_grad_(True)
        out = mca.functional.dilation(xd, wd, merge, "replicate", save_indices=False)
        out.backward(g.to(dev))
        grads.append((_np(xd.grad), _np(wd.grad)))
    gx, gw = O.morpho_backward(O.DILATION, O.MERGES[merge], O.REPLICATE, 0.0, x.numpy(), w.numpy(), g.numpy())
    for got in grads:
        assert normwise_error(got[0], gx) <= 1e-6 and normwise_error(got[1], gw) <= 1e-6
    assert np.array_equal(grads[0][1], grads[1][1])
