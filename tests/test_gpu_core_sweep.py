"""Seeded sweep of the operators over random geometries, against the oracle.

Each case draws its batch, channel counts, plane size (ragged tiles, planes narrower or shorter than a
tile or than the element, one channel), element size (square and rectangular, even and odd), merge,
padding, dtype (dilation / erosion also float16 and bfloat16) and saving choice, then runs the operator through torch.ops.morphocore (the product
path) and compares with the oracle: dilation / erosion forwards bit for bit, smorph forwards and every
gradient within 1e-6 (float32) / 1e-12 (float64) norm-wise (a shared alpha's gradient, a sum over the
pairs that can cancel, relative to the sum of its terms' magnitudes, as is any weight, alpha or beta
gradient whose terms cancel so far that it misses the norm-wise measure). The sweep exercises the launch plans
(tilings, workspace layouts, saved-statistics slots, small-grid shapes) on shapes no hand-written
case picks. Two more families: elements beyond the compiled static sizes, up to 51x51 (the generic
kernels, two-byte pair taps past 256 taps, the large-element smorph backwards), and IDENTITY 3x3 / 5x5
planes whose width is a multiple of 8 (the row-band kernels, partial last bands); and dilation / erosion on
planes large enough for the forward's full launch shape (at least 1024 workgroups), which the other
families' planes never reach.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error

pytestmark = pytest.mark.gpu

MERGES = ["max", "min", "sum", "mean", "identity"]
PADDINGS = ["zero", "geodesic", "constant", "replicate"]
SIZES = [(1, 1), (1, 3), (2, 2), (3, 3), (3, 5), (4, 2), (5, 5), (5, 3), (7, 7), (2, 5), (11, 11)]


def _geometry(rng, dtypes=(torch.float32, torch.float64)):
    KH, KW = SIZES[int(rng.integers(0, len(SIZES)))]
    large = KH * KW > 49
    # One case in four takes a larger plane (several strips and tile rows per plane) with few channels.
    wide = rng.integers(0, 4) == 0
    hmax, wmax = (120, 260) if wide else ((40, 90) if large else (90, 150))
    cmax = 4 if wide or large else 10
    return dict(B=int(rng.integers(1, 4)), Cin=int(rng.integers(1, cmax)), Cout=int(rng.integers(1, cmax)),
                H=int(rng.integers(1, hmax)), W=int(rng.integers(1, wmax)), KH=KH, KW=KW,
                dtype=dtypes[int(rng.integers(0, len(dtypes)))], seed=int(rng.integers(0, 1 << 30)))


def _morpho_cases(n, seed):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        c = _geometry(rng, (torch.float32, torch.float64, torch.float16, torch.bfloat16))
        c.update(op=int(rng.integers(0, 2)), merge=MERGES[int(rng.integers(0, 5))], padding=PADDINGS[int(rng.integers(0, 4))],
                 pv=float(rng.normal()), save=bool(rng.integers(0, 2)))
        if c["merge"] == "identity":
            c["Cout"] = c["Cin"]
        yield c


def _smorph_cases(n, seed, merges):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        c = _geometry(rng)
        c.update(merge=merges[int(rng.integers(0, len(merges)))], shared=bool(rng.integers(0, 2)),
                 alpha_scale=float(rng.choice([0.0, 1.0, 5.0, 20.0])), save=bool(rng.integers(0, 2)))
        if c["merge"] == "identity":
            c["Cout"] = c["Cin"]
        yield c


def _ids(c):
    return f"{c['B']}x{c['Cin']}x{c['Cout']}x{c['H']}x{c['W']}k{c['KH']}x{c['KW']}"


def _gen(c):
    g = torch.Generator().manual_seed(c["seed"])
    return lambda *s, scale=1.0: (torch.randn(*s, generator=g, dtype=torch.float64) * scale).to(c["dtype"])  # noqa: E731


HALF = (torch.float16, torch.bfloat16)
# 16-bit gradients are rounded once from float32 sums the oracle forms in another order: within about
# one unit in their last place (as tests/test_gpu_half.py).
GTOL = {torch.float32: TOL[torch.float32], torch.float64: TOL[torch.float64], torch.float16: 1e-3, torch.bfloat16: 8e-3}


def _check(got, want, dtype, what):
    err = normwise_error(got.detach().cpu().numpy(), want)
    assert err <= TOL[dtype], f"{what}: {err}"


# Elements beyond the compiled static sizes, up to 51x51 (the generic kernels; more than 256 taps
# saves two-byte pair taps), on small planes and channel counts.
LARGE = [(13, 13), (15, 15), (9, 17), (17, 9), (21, 21), (25, 25), (31, 31), (35, 35), (41, 41), (51, 51), (12, 12), (1, 31)]


def _large_geometry(rng, dtypes):
    KH, KW = LARGE[int(rng.integers(0, len(LARGE)))]
    big = KH * KW > 700
    hmax, wmax, cmax = (40, 48, 3) if big else (70, 90, 5)
    return dict(B=int(rng.integers(1, 3)), Cin=int(rng.integers(1, cmax + 1)), Cout=int(rng.integers(1, cmax + 1)),
                H=int(rng.integers(1, hmax)), W=int(rng.integers(1, wmax)), KH=KH, KW=KW,
                dtype=dtypes[int(rng.integers(0, len(dtypes)))], seed=int(rng.integers(0, 1 << 30)))


def _morpho_large_cases(n, seed):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        c = _large_geometry(rng, (torch.float32, torch.float64, torch.float16, torch.bfloat16))
        c.update(op=int(rng.integers(0, 2)), merge=MERGES[int(rng.integers(0, 5))], padding=PADDINGS[int(rng.integers(0, 4))],
                 pv=float(rng.normal()), save=bool(rng.integers(0, 2)))
        if c["merge"] == "identity":
            c["Cout"] = c["Cin"]
        yield c


def _smorph_large_cases(n, seed, merges):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        c = _large_geometry(rng, (torch.float32, torch.float64))
        c.update(merge=merges[int(rng.integers(0, len(merges)))], shared=bool(rng.integers(0, 2)),
                 alpha_scale=float(rng.choice([0.0, 1.0, 5.0, 20.0])), save=bool(rng.integers(0, 2)))
        if c["merge"] == "identity":
            c["Cout"] = c["Cin"]
        yield c


def _band_cases(n, seed):
    """IDENTITY 3x3 / 5x5 on planes whose width is a multiple of 8: the row-band kernels' shapes (any
    height, so partial last bands; every padding and dtype)."""
    rng = np.random.default_rng(seed)
    for _ in range(n):
        K = 3 if rng.integers(0, 2) == 0 else 5
        C = int(rng.integers(1, 11))
        yield dict(B=int(rng.integers(1, 4)), Cin=C, Cout=C, H=int(rng.integers(1, 130)), W=8 * int(rng.integers(1, 33)), KH=K, KW=K,
                   dtype=(torch.float32, torch.float64, torch.float16, torch.bfloat16)[int(rng.integers(0, 4))],
                   seed=int(rng.integers(0, 1 << 30)), op=int(rng.integers(0, 2)), merge="identity",
                   padding=PADDINGS[int(rng.integers(0, 4))], pv=float(rng.normal()), save=bool(rng.integers(0, 2)))


def _full_launch_cases(n, seed):
    """Dilation / erosion on planes large enough that the forward takes its full launch shape (at least
    1024 workgroups of 16 x 64 output tiles: 4 rows per wave, several output channels per workgroup),
    which the smaller cases above never reach."""
    rng = np.random.default_rng(seed)
    while n > 0:
        K = [3, 5, 7, 11][int(rng.integers(0, 4))]
        merge = MERGES[int(rng.integers(0, 5))]
        Cin = int(rng.integers(1, 4 if K == 11 else 6))
        Cout = Cin if merge == "identity" else int(rng.integers(1, 9))
        B, H, W = int(rng.integers(2, 5)), int(rng.integers(200, 330)), int(rng.integers(500, 760))
        groups = Cout if merge == "identity" or Cout < 4 else (Cout + 3) // 4
        if B * -(-H // 16) * -(-W // 64) * groups < 1024:
            continue
        n -= 1
        yield dict(B=B, Cin=Cin, Cout=Cout, H=H, W=W, KH=K, KW=K, seed=int(rng.integers(0, 1 << 30)),
                   dtype=(torch.float32, torch.float64, torch.float16, torch.bfloat16)[int(rng.integers(0, 4))],
                   op=int(rng.integers(0, 2)), merge=merge, padding=PADDINGS[int(rng.integers(0, 4))], pv=float(rng.normal()),
                   save=bool(rng.integers(0, 2)))


@pytest.mark.parametrize("c", list(_morpho_cases(200, 7101)), ids=_ids)
def test_morpho_sweep(c):
    _morpho_run(c)


@pytest.mark.parametrize("c", list(_morpho_large_cases(60, 7404)), ids=_ids)
def test_morpho_large_element_sweep(c):
    _morpho_run(c)


@pytest.mark.parametrize("c", list(_band_cases(60, 7505)), ids=_ids)
def test_morpho_band_sweep(c):
    _morpho_run(c)


@pytest.mark.parametrize("c", list(_full_launch_cases(24, 7808)), ids=_ids)
def test_morpho_full_launch_sweep(c):
    _morpho_run(c)


def _morpho_run(c):
    import morphocore_amd  # noqa: F401  (registers torch.ops.morphocore)

    dev = torch.device("cuda")
    mk = _gen(c)
    cw = 1 if c["merge"] == "identity" else c["Cin"]
    x = mk(c["B"], c["Cin"], c["H"], c["W"])
    w = mk(c["Cout"], cw, c["KH"], c["KW"], scale=0.3)
    gout = mk(c["B"], c["Cout"], c["H"], c["W"])
    merge, padding = O.MERGES[c["merge"]], O.PADDINGS[c["padding"]]
    fn = torch.ops.morphocore.dilation if c["op"] == O.DILATION else torch.ops.morphocore.erosion
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    out = fn(xd, wd, merge, padding, c["pv"], c["save"], 0.0)
    out.backward(gout.to(dev))
    # 16-bit tensors: the float32 oracle on the same (exactly converted) values and the float32 padding
    # value, each result rounded once.
    half = c["dtype"] in HALF
    xs, ws, gs = ((t.float() if half else t).numpy() for t in (x, w, gout))
    pv = c["pv"]
    ref, _ = O.morpho_forward(c["op"], merge, padding, pv, xs, ws)
    rounded = (lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(c["dtype"]).float().numpy()) if half else (lambda a: a)  # noqa: E731
    assert np.array_equal(out.detach().float().cpu().numpy() if half else out.detach().cpu().numpy(), rounded(ref)), "forward differs"
    gx, gw = O.morpho_backward(c["op"], merge, padding, pv, xs, ws, gs)
    for name, got, want in (("grad_input", xd.grad, gx), ("grad_weight", wd.grad, gw)):
        err = normwise_error(got.detach().float().cpu().numpy() if half else got.detach().cpu().numpy(), rounded(want))
        assert err <= GTOL[c["dtype"]], f"{name}: {err}"


def _smorph_run(c, monkeypatch, scm):
    import morphocore_amd  # noqa: F401

    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", "-1" if c["save"] else "0")
    dev = torch.device("cuda")
    mk = _gen(c)
    cw = 1 if c["merge"] == "identity" else c["Cin"]
    x = mk(c["B"], c["Cin"], c["H"], c["W"])
    w = mk(c["Cout"], cw, c["KH"], c["KW"], scale=0.3)
    pairs = c["Cout"] if c["merge"] == "identity" else c["Cout"] * c["Cin"]
    alpha = (mk(1) if c["shared"] else mk(pairs)) * c["alpha_scale"]
    alpha = alpha.reshape(()) if c["shared"] else alpha.reshape((c["Cout"],) if c["merge"] == "identity" else (c["Cout"], c["Cin"]))
    gout = mk(c["B"], c["Cout"], c["H"], c["W"])
    xd, wd, ad = (t.to(dev).requires_grad_(True) for t in (x, w, alpha))
    beta = None
    if scm:
        beta = mk(c["Cout"], scale=3.0)
        bd = beta.to(dev).requires_grad_(True)
        out = torch.ops.morphocore.smorph_scm(xd, wd, ad, bd)
        out.backward(gout.to(dev))
        ref = O.smorph_scm_forward(x.numpy(), w.numpy(), alpha.numpy(), beta.numpy())
        backward = lambda *a: O.smorph_scm_backward(*a)  # noqa: E731
        args = (x, w, alpha, beta, gout)
        got = (xd.grad, wd.grad, ad.grad, bd.grad)
    else:
        merge = O.MERGES[c["merge"]]
        out = torch.ops.morphocore.smorph(xd, wd, ad, merge)
        out.backward(gout.to(dev))
        ref = O.smorph_forward(merge, x.numpy(), w.numpy(), alpha.numpy())
        backward = lambda *a: O.smorph_backward(merge, *a)  # noqa: E731
        args = (x, w, alpha, gout)
        got = (xd.grad, wd.grad, ad.grad)
    want = backward(*(t.numpy() for t in args))
    _check(out, ref, c["dtype"], "forward")
    magnitudes = None
    for name, a, b in zip(("grad_input", "grad_weight", "grad_alpha", "grad_beta"), got, want):
        if name == "grad_input":
            _check(a, b, c["dtype"], name)
            continue
        got_np = a.detach().cpu().numpy().astype(np.float64)
        shared = name == "grad_alpha" and c["shared"]
        if not shared and normwise_error(got_np, b) <= TOL[c["dtype"]]:
            continue
        # A weight, alpha (or SMOOTH beta) gradient sums a term over every pixel (and a shared alpha over
        # every pair too); the terms can cancel far below their size (one weight of a 1x1 element summing
        # a random-sign gradient over 60,000 pixels; alpha terms of both signs), and then no float32
        # evaluation meets 1e-6 of the result: the reference extension's own float32 result lies further
        # than that from the float64 oracle (up to 9.5e-5 for alpha on an 8,100-case sweep). Such sums are
        # compared relative to the sum of their terms' magnitudes (the oracle's, smorph_term_magnitudes),
        # which bounds the error any summation order can make.
        if magnitudes is None:
            if scm:
                magnitudes = O.smorph_scm_term_magnitudes(x.numpy(), w.numpy(), alpha.numpy(), beta.numpy(), gout.numpy())
            else:
                magnitudes = O.smorph_term_magnitudes(O.MERGES[c["merge"]], x.numpy(), w.numpy(), alpha.numpy(), gout.numpy())
        scale = float(np.max(np.abs(magnitudes[("grad_weight", "grad_alpha", "grad_beta").index(name)])))
        err = float(np.max(np.abs(got_np - b))) / max(scale, 1e-30)
        assert err <= TOL[c["dtype"]], f"{name}: {err} of the sum of its terms' magnitudes"


@pytest.mark.parametrize("c", list(_smorph_cases(120, 7202, MERGES)), ids=_ids)
def test_smorph_sweep(c, monkeypatch):
    _smorph_run(c, monkeypatch, scm=False)


@pytest.mark.parametrize("c", list(_smorph_cases(80, 7303, ["sum"])), ids=_ids)
def test_smorph_scm_sweep(c, monkeypatch):
    _smorph_run(c, monkeypatch, scm=True)


@pytest.mark.parametrize("c", list(_smorph_large_cases(40, 7606, MERGES)), ids=_ids)
def test_smorph_large_element_sweep(c, monkeypatch):
    _smorph_run(c, monkeypatch, scm=False)


@pytest.mark.parametrize("c", list(_smorph_large_cases(12, 7707, ["sum"])), ids=_ids)
def test_smorph_scm_large_element_sweep(c, monkeypatch):
    _smorph_run(c, monkeypatch, scm=True)


@pytest.mark.parametrize("save", [False, True])
def test_smorph_max_pair_just_outside_the_winner_tolerance(save, monkeypatch):
    """A MAX merge where a second channel's pair output lies 1.0133e-6 below the winner's (batch 1,
    output channel 1, pixel (16, 142)): outside the 1e-6 tolerance once the pair output is rounded, as
    the reference rounds it, but inside it if the winner count fused W * (1 / S) into the subtraction,
    which then split that pixel's gradient between two channels (grad_input off by 8e-3 there)."""
    c = dict(B=3, Cin=7, Cout=6, H=85, W=143, KH=4, KW=2, dtype=torch.float32, seed=803402658, merge="max", shared=True,
             alpha_scale=5.0, save=save)
    _smorph_run(c, monkeypatch, scm=False)
