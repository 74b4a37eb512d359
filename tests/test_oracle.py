"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

* against the reference's own CPU extension: vectors in tests/golden/ref_vectors.npz written by
  tests/golden/make_golden.py from oracle/_ref (built from the reference sources);
* against numpy brute force built like the reference's test references (tests/functional/utils.py:6-49,
  test_padding.py:9-45 in the reference);
* against the mathematics: float64 central finite differences for every gradient (including smorph's
  alpha), closed-form gradient routing on exact inputs, the alpha -> +-inf and alpha = 0 limits of
  smorph, and the reference's known-answer padding tests (test_padding.py:95-143);
* the oracle's exponential against libm within the accuracy its method promises.
"""
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import normwise_error

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")
MERGES = ["max", "min", "sum", "mean", "identity"]
PADDINGS = ["zero", "geodesic", "constant", "replicate"]
TOLS = {"f32": 1e-6, "f64": 1e-12}


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def _golden_morpho_cases(golden):
    for key in golden.files:
        parts = key.split("/")
        if len(parts) == 7 and parts[1] == "morpho" and parts[6] == "out":
            yield parts[0], parts[2], parts[3], parts[4], parts[5]


def test_golden_morpho_forward_and_gradients(golden):
    n = 0
    for dname, op, merge, padding, variant in _golden_morpho_cases(golden):
        key = f"{dname}/morpho/{op}/{merge}/{padding}/{variant}"
        x = golden[f"{dname}/x" if variant == "rand" else f"{dname}/xq"]
        w = golden[f"{dname}/wi" if merge == "identity" else f"{dname}/w"]
        if variant == "quant":
            w = np.zeros_like(w)
        g = golden[f"{dname}/gi" if merge == "identity" else f"{dname}/g"]
        opi = O.DILATION if op == "dilation" else O.EROSION
        out, idx = O.morpho_forward(opi, O.MERGES[merge], O.PADDINGS[padding], 0.25, x, w, save_indices=merge in ("max", "min"))
        assert np.array_equal(out, golden[key + "/out"]), key
        assert np.array_equal(np.signbit(out), np.signbit(golden[key + "/out"])), key
        gx, gw = O.morpho_backward(opi, O.MERGES[merge], O.PADDINGS[padding], 0.25, x, w, g, indices=idx)
        assert normwise_error(gx, golden[key + "/gx"]) <= TOLS[dname], key
        assert normwise_error(gw, golden[key + "/gw"]) <= TOLS[dname], key
        n += 1
    assert n >= 60


def test_golden_smorph(golden):
    n = 0
    for dname in ("f32", "f64"):
        x = golden[f"{dname}/x"]
        for merge in MERGES:
            wt = golden[f"{dname}/smorph/{merge}/w"]
            g = golden[f"{dname}/gi" if merge == "identity" else f"{dname}/g"]
            for aname in ("neg", "zero", "mixed", "shared"):
                key = f"{dname}/smorph/{merge}/{aname}"
                alpha = golden[key + "/alpha"]
                out = O.smorph_forward(O.MERGES[merge], x, wt, alpha)
                assert normwise_error(out, golden[key + "/out"]) <= TOLS[dname], key
                gx, gw, ga = O.smorph_backward(O.MERGES[merge], x, wt, alpha, g)
                assert normwise_error(gx, golden[key + "/gx"]) <= TOLS[dname], key
                assert normwise_error(gw, golden[key + "/gw"]) <= TOLS[dname], key
                assert normwise_error(ga, golden[key + "/ga"]) <= TOLS[dname], key
                n += 1
    assert n == 40


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("padding", PADDINGS)
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_forward_matches_brute_force(op, merge, padding, dtype):
    rng = np.random.default_rng(0)
    for (B, Cin, Cout, H, W, KH, KW) in [(2, 3, 4, 6, 7, 3, 3), (1, 2, 3, 5, 4, 4, 2), (1, 2, 2, 3, 3, 5, 5)]:
        if merge == "identity":
            Cout = Cin
        x = rng.standard_normal((B, Cin, H, W)).astype(dtype)
        w = (rng.standard_normal((Cout, 1 if merge == "identity" else Cin, KH, KW)) * 0.3).astype(dtype)
        out, idx = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], -0.75, x, w, save_indices=merge in ("max", "min"))
        ref, ref_idx = O.brute.forward(op, O.MERGES[merge], O.PADDINGS[padding], -0.75, x, w)
        assert np.array_equal(out, ref)
        if merge in ("max", "min"):
            assert np.array_equal(idx, ref_idx)


def test_forward_ties_first_tap_first_channel():
    """Quantised input, zero weight: every window ties; the first tap and first channel win."""
    rng = np.random.default_rng(1)
    x = (rng.integers(0, 4, (1, 3, 6, 6)) / 4).astype(np.float32)
    w = np.zeros((2, 3, 3, 3), np.float32)
    for merge in ("max", "min"):
        out, idx = O.morpho_forward(O.DILATION, O.MERGES[merge], O.REPLICATE, 0.0, x, w, save_indices=True)
        ref, ref_idx = O.brute.forward(O.DILATION, O.MERGES[merge], O.REPLICATE, 0.0, x, w)
        assert np.array_equal(out, ref) and np.array_equal(idx, ref_idx)
    # All-minus-infinity windows keep tap 0 of channel 0, and the MAX merge clamps to lowest().
    w_inf = np.full((1, 2, 3, 3), -np.inf, np.float32)
    out, idx = O.morpho_forward(O.DILATION, O.MAX, O.GEODESIC, 0.0, x[:, :2], w_inf, save_indices=True)
    assert np.all(out == np.finfo(np.float32).min) and np.all(idx == 0)


def test_smorph_limits():
    """alpha -> +inf / -inf gives dilation / erosion over in-image taps; alpha = 0 gives the plain
    mean of the in-image values (reference tests/functional/utils.py:71-78)."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 2, 7, 8))
    w = rng.standard_normal((3, 2, 3, 3)) * 0.1
    big = np.full((3, 2), 1000.0)
    dil, _ = O.morpho_forward(O.DILATION, O.ADD, O.GEODESIC, 0.0, x, w)
    np.testing.assert_allclose(O.smorph_forward(O.ADD, x, w, big), dil, rtol=0, atol=1e-2)
    ero, _ = O.morpho_forward(O.EROSION, O.ADD, O.GEODESIC, 0.0, x, -w)
    np.testing.assert_allclose(O.smorph_forward(O.ADD, x, w, -big), ero, rtol=0, atol=1e-2)
    mean = O.smorph_forward(O.IDENTITY, x, w[:2, :1], np.zeros(2))
    for c in range(2):
        np.testing.assert_allclose(mean[0, c], O.brute.smorph_pair(x[0, c], w[c, 0], 0.0), rtol=1e-12)


def test_smorph_matches_brute_force():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 6, 5))
    for merge in MERGES:
        ident = merge == "identity"
        Cout = 3 if ident else 4
        w = rng.standard_normal((Cout, 1 if ident else 3, 3, 5)) * 0.2
        alpha = rng.standard_normal(Cout if ident else (Cout, 3)) * 3
        out = O.smorph_forward(O.MERGES[merge], x, w, alpha)
        a = alpha.reshape(-1)
        for b in range(2):
            for o in range(Cout):
                if ident:
                    ref = O.brute.smorph_pair(x[b, o], w[o, 0], a[o])
                else:
                    pairs = [O.brute.smorph_pair(x[b, i], w[o, i], a[o * 3 + i]) for i in range(3)]
                    if merge == "max":
                        ref = np.maximum.reduce(pairs)
                    elif merge == "min":
                        ref = np.minimum.reduce(pairs)
                    else:
                        ref = sum(pairs) / (3 if merge == "mean" else 1)
                np.testing.assert_allclose(out[b, o], ref, rtol=1e-13, atol=1e-13)


def test_exp_accuracy():
    """The restated vector exponential (morpho_cpu_simd.hpp:127-169) is within 1 ulp (float) and
    2 ulp (double) of the correctly rounded exp on a dense grid."""
    lib = O.lib()
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001), np.linspace(-1, 1, 2001)])
    worst32 = worst64 = 0.0
    for v in xs:
        v32 = float(np.float32(v))
        exact = math.exp(v32)
        got = lib.oracle_expf(v32)
        worst32 = max(worst32, abs(got - exact) / float(np.spacing(np.float32(exact))))
        got64 = lib.oracle_exp(v)
        worst64 = max(worst64, abs(got64 - math.exp(v)) / float(np.spacing(math.exp(v))))
    assert worst32 <= 1.0 and worst64 <= 2.0, (worst32, worst64)


def _finite_difference(f, arr, eps):
    grad = np.zeros_like(arr)
    flat = arr.reshape(-1)
    gflat = grad.reshape(-1)
    for j in range(flat.size):
        keep = flat[j]
        flat[j] = keep + eps
        up = f()
        flat[j] = keep - eps
        down = f()
        flat[j] = keep
        gflat[j] = (up - down) / (2 * eps)
    return grad


@pytest.mark.parametrize("padding", ["geodesic", "zero", "constant"])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_morpho_gradients_match_finite_differences(op, merge, padding):
    """Gradients of a weighted sum of outputs, on inputs whose taps never tie (x*10 + arange, as the
    reference's gradcheck separates ties, test_morpho_operation.py:333-337).

    Fill paddings only: under 'replicate' the reference drops the gradient of a tap that read the
    clamped edge pixel (morpho_op_cpu_backward.hxx:39-88), which is not the derivative of the
    forward; that rule is pinned by the golden vectors of the reference build instead."""
    rng = np.random.default_rng(4)
    B, Cin, Cout, H, W, K = 1, 2, 3, 5, 6, 3
    if merge == "identity":
        Cout = Cin
    x = rng.standard_normal((B, Cin, H, W)) * 10 + np.arange(B * Cin * H * W).reshape(B, Cin, H, W) * 0.37
    w = rng.standard_normal((Cout, 1 if merge == "identity" else Cin, K, K)) * 10 + np.arange(Cout * (1 if merge == "identity" else Cin) * K * K).reshape(Cout, -1, K, K) * 0.11
    g = rng.standard_normal((B, Cout, H, W))
    m, p = O.MERGES[merge], O.PADDINGS[padding]

    def loss():
        out, _ = O.morpho_forward(op, m, p, 0.0, x, w)
        return float(np.sum(out * g))

    out, idx = O.morpho_forward(op, m, p, 0.0, x, w, save_indices=merge in ("max", "min"))
    gx, gw = O.morpho_backward(op, m, p, 0.0, x, w, g, indices=idx)
    np.testing.assert_allclose(gx, _finite_difference(loss, x, 1e-6), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(gw, _finite_difference(loss, w, 1e-6), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("merge", MERGES)
def test_smorph_gradients_match_finite_differences(merge):
    rng = np.random.default_rng(5)
    B, Cin, H, W, K = 1, 2, 5, 4, 3
    Cout = Cin if merge == "identity" else 3
    x = rng.standard_normal((B, Cin, H, W))
    w = rng.standard_normal((Cout, 1 if merge == "identity" else Cin, K, K)) * 0.3
    alpha = rng.standard_normal(Cout if merge == "identity" else (Cout, Cin)) * 2
    g = rng.standard_normal((B, Cout, H, W))
    m = O.MERGES[merge]
    if merge in ("max", "min"):
        # Separate the channels so that no pair lies within the winner tolerance of another.
        x = x + np.arange(Cin).reshape(1, Cin, 1, 1) * 5.0

    def loss():
        return float(np.sum(O.smorph_forward(m, x, w, alpha) * g))

    gx, gw, ga = O.smorph_backward(m, x, w, alpha, g)
    np.testing.assert_allclose(gx, _finite_difference(loss, x, 1e-6), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(gw, _finite_difference(loss, w, 1e-6), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(ga, _finite_difference(loss, alpha, 1e-6), rtol=1e-5, atol=1e-7)


def test_gradient_routing_closed_form():
    """Per-pair merges route each pixel's gradient to exactly one tap: with an all-ones gradient,
    grad_weight[o, i] sums to sign * B * H * W and grad_input sums to the count of in-image picks."""
    rng = np.random.default_rng(6)
    x = rng.random((2, 3, 9, 10)).astype(np.float32)
    w = (rng.standard_normal((4, 3, 5, 5)) * 0.05).astype(np.float32)
    g = np.ones((2, 4, 9, 10), np.float32)
    for op, sign in ((O.DILATION, 1.0), (O.EROSION, -1.0)):
        gx, gw = O.morpho_backward(op, O.ADD, O.GEODESIC, 0.0, x, w, g)
        assert np.array_equal(gw.sum(axis=(2, 3)), np.full((4, 3), sign * 2 * 9 * 10, np.float32))
        # Geodesic borders never win, so every pick is in-image.
        assert gx.sum() == 2 * 4 * 3 * 9 * 10


class TestReferencePaddingKnownAnswers:
    """The reference's known-answer padding tests (test_padding.py:95-143), on the oracle."""

    @pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
    def test_zero_equals_constant_zero(self, op):
        rng = np.random.default_rng(7)
        x = rng.standard_normal((2, 3, 16, 16)).astype(np.float32)
        w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
        for merge in (O.ADD, O.MAX):
            a, _ = O.morpho_forward(op, merge, O.ZERO, 0.0, x, w)
            b, _ = O.morpho_forward(op, merge, O.CONSTANT, 0.0, x, w)
            assert np.array_equal(a, b)

    @pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
    def test_geodesic_never_wins(self, op):
        rng = np.random.default_rng(8)
        x = rng.standard_normal((1, 1, 12, 12)).astype(np.float32)
        w = np.zeros((1, 1, 5, 5), np.float32)
        a, _ = O.morpho_forward(op, O.ADD, O.GEODESIC, 0.0, x, w)
        b, _ = O.morpho_forward(op, O.ADD, O.CONSTANT, -1e9 if op == O.DILATION else 1e9, x, w)
        assert np.array_equal(a, b)

    @pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
    def test_constant_border_dominates(self, op):
        rng = np.random.default_rng(9)
        x = rng.random((1, 1, 8, 8)).astype(np.float32)
        extreme = 50.0 if op == O.DILATION else -50.0
        out, _ = O.morpho_forward(op, O.ADD, O.CONSTANT, extreme, x, np.zeros((1, 1, 3, 3), np.float32))
        out = out[0, 0]
        border = np.ones_like(out, dtype=bool)
        border[1:-1, 1:-1] = False
        assert np.all(out[border] == extreme) and np.all(out[~border] != extreme)

    @pytest.mark.parametrize("padding", PADDINGS)
    def test_interior_is_padding_independent(self, padding):
        rng = np.random.default_rng(10)
        x = rng.standard_normal((1, 1, 20, 20)).astype(np.float32)
        w = rng.standard_normal((1, 1, 5, 5)).astype(np.float32)
        ref, _ = O.morpho_forward(O.DILATION, O.ADD, O.GEODESIC, 0.0, x, w)
        out, _ = O.morpho_forward(O.DILATION, O.ADD, O.PADDINGS[padding], 4.0, x, w)
        assert np.array_equal(out[0, 0, 2:-2, 2:-2], ref[0, 0, 2:-2, 2:-2])


def test_planted_mistakes_are_caught():
    """Mistakes planted in a copy of the oracle's contract (on the CPU) fail the brute force: a
    flipped tap orientation and a non-strict (last-tap) tie rule."""
    rng = np.random.default_rng(11)
    x = (rng.integers(0, 4, (1, 2, 6, 7)) / 4).astype(np.float32)
    w = np.zeros((2, 2, 3, 3), np.float32)
    w[:, :, 0, 1] = 0.5
    out, idx = O.morpho_forward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x, w, save_indices=True)
    flipped, fidx = O.morpho_forward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x, np.ascontiguousarray(w[:, :, ::-1, ::-1]), save_indices=True)
    assert not np.array_equal(out, flipped) or not np.array_equal(idx, fidx)
    # The last-tap rule on ties would select a later tap than the brute force's first one.
    _, ref_idx = O.brute.forward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x, np.zeros_like(w))
    _, tie_idx = O.morpho_forward(O.DILATION, O.MAX, O.REPLICATE, 0.0, x, np.zeros_like(w), save_indices=True)
    assert np.array_equal(tie_idx, ref_idx) and np.any((ref_idx & 0xFFFF) != 8)


@pytest.mark.parametrize("merge", MERGES)
def test_per_sample_weights_equal_per_sample_calls(merge):
    """The oracle's per-sample structuring element (weight noise, morpho_op_wrap.hxx:55-64) equals one
    call per batch element with that element's weight; grad_weight is their sum (the reference's own
    noise test, test_weight_noise.py:42-60)."""
    rng = np.random.default_rng(12)
    B, Cin, Cout, H, W, K = 3, 2, 3, 7, 8, 3
    if merge == "identity":
        Cout = Cin
    Cw = 1 if merge == "identity" else Cin
    x = rng.standard_normal((B, Cin, H, W))
    w = rng.standard_normal((Cout, Cw, K, K)) * 0.2
    sample = w[None] + rng.uniform(-0.05, 0.05, (B, Cout, Cw, K, K))
    g = rng.standard_normal((B, Cout, H, W))
    m = O.MERGES[merge]
    out, idx = O.morpho_forward(O.DILATION, m, O.GEODESIC, 0.0, x, w, save_indices=merge in ("max", "min"), sample_weight=sample)
    gx, gw = O.morpho_backward(O.DILATION, m, O.GEODESIC, 0.0, x, w, g, indices=idx, sample_weight=sample)
    gw_sum = np.zeros_like(w)
    for b in range(B):
        ob, ib = O.morpho_forward(O.DILATION, m, O.GEODESIC, 0.0, x[b:b + 1], sample[b], save_indices=merge in ("max", "min"))
        assert np.array_equal(out[b:b + 1], ob)
        gxb, gwb = O.morpho_backward(O.DILATION, m, O.GEODESIC, 0.0, x[b:b + 1], sample[b], g[b:b + 1], indices=ib)
        np.testing.assert_allclose(gx[b:b + 1], gxb, rtol=1e-12, atol=1e-12)
        gw_sum += gwb
    np.testing.assert_allclose(gw, gw_sum, rtol=1e-12, atol=1e-12)


def test_golden_smorph_scm(golden):
    """The SMOOTH channel merge (smorph_scm) against the reference's own CPU build: forward bit for
    bit, gradients of x, w~, alpha and beta within the tolerance."""
    n = 0
    for dname in ("f32", "f64"):
        x = golden[f"{dname}/x"]
        g = golden[f"{dname}/g"]
        wt = golden[f"{dname}/scm/w"]
        for aname in ("mixed", "shared"):
            for bname in ("pos", "neg", "zero", "mixed"):
                key = f"{dname}/scm/{aname}/{bname}"
                alpha, beta = golden[key + "/alpha"], golden[key + "/beta"]
                out = O.smorph_scm_forward(x, wt, alpha, beta)
                assert np.array_equal(out, golden[key + "/out"]), key
                gx, gw, ga, gb = O.smorph_scm_backward(x, wt, alpha, beta, g)
                for got, name in ((gx, "gx"), (gw, "gw"), (ga, "ga"), (gb, "gb")):
                    assert got.shape == golden[f"{key}/{name}"].shape, (key, name)
                    assert normwise_error(got, golden[f"{key}/{name}"]) <= TOLS[dname], (key, name)
                n += 1
    assert n == 16


def test_smorph_scm_limits():
    """What the mathematics fixes for the SMOOTH merge of the pair outputs c_i (each pair's smorph
    output, taken from the oracle's ADD merge with a single input channel):
    beta = 0 gives their mean, beta -> +inf their maximum and -inf their minimum (closed forms), and
    one input channel gives c_0 itself, bit for bit (q = exp(0) = 1)."""
    rng = np.random.default_rng(21)
    B, Cin, Cout, H, W, K = 2, 3, 2, 6, 7, 3
    x = rng.standard_normal((B, Cin, H, W))
    w = rng.standard_normal((Cout, Cin, K, K)) * 0.2
    alpha = rng.standard_normal((Cout, Cin)) * 2
    # c[b, o, i] from single-channel smorph calls
    c = np.stack([np.stack([O.smorph_forward(O.ADD, x[:, i:i + 1], w[o:o + 1, i:i + 1], alpha[o, i])[:, 0] for i in range(Cin)], 1)
                  for o in range(Cout)], 1)
    assert c.shape == (B, Cout, Cin, H, W)
    mean = O.smorph_scm_forward(x, w, alpha, np.zeros(Cout))
    np.testing.assert_allclose(mean, c.mean(axis=2), rtol=1e-13, atol=1e-13)
    hi = O.smorph_scm_forward(x, w, alpha, np.full(Cout, 1e6))
    np.testing.assert_allclose(hi, c.max(axis=2), rtol=0, atol=1e-4)
    lo = O.smorph_scm_forward(x, w, alpha, np.full(Cout, -1e6))
    np.testing.assert_allclose(lo, c.min(axis=2), rtol=0, atol=1e-4)
    for dtype in (np.float32, np.float64):
        x1, w1 = x[:, :1].astype(dtype), w[:, :1].astype(dtype)
        one = O.smorph_scm_forward(x1, w1, alpha[:, :1].astype(dtype), np.array([3.0, -2.0], dtype))
        assert np.array_equal(one, O.smorph_forward(O.ADD, x1, w1, alpha[:, :1].astype(dtype)))


def test_smorph_scm_gradients_match_finite_differences():
    """float64 central finite differences of a weighted sum of smorph_scm outputs, for x, w~, alpha
    and beta (a dropped or mis-signed term of the channel merge's derivative fails here)."""
    rng = np.random.default_rng(22)
    B, Cin, Cout, H, W, K = 1, 3, 2, 4, 5, 3
    x = rng.standard_normal((B, Cin, H, W))
    w = rng.standard_normal((Cout, Cin, K, K)) * 0.3
    alpha = rng.standard_normal((Cout, Cin)) * 2
    beta = np.array([1.7, -2.4])
    g = rng.standard_normal((B, Cout, H, W))

    def loss():
        return float(np.sum(O.smorph_scm_forward(x, w, alpha, beta) * g))

    gx, gw, ga, gb = O.smorph_scm_backward(x, w, alpha, beta, g)
    for got, arr in ((gx, x), (gw, w), (ga, alpha), (gb, beta)):
        np.testing.assert_allclose(got, _finite_difference(loss, arr, 1e-6), rtol=1e-5, atol=1e-7)


# ----------------------------------------------------------------------------------------------
# The smorph structuring-element blend w~ (functional/smorph.py:56-70), which the oracle computes
# with torch exactly as the reference's Python and every smorph test through functional.smorph
# uses as its expected value: pinned by closed forms derived apart from the formula.
# ----------------------------------------------------------------------------------------------

# An asymmetric 2x3 element with exact (small integer) entries.
_W23 = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
# alpha with tanh(alpha) = 1/2 exactly (in float64 and, rounded, in float32): the blend is then
# 1/2 (1/4 flip(w) + 3/4 w) = flip(w) / 8 + 3 w / 8, worked out by hand for _W23 ...
_ALPHA_HALF = {np.float64: 0.5493061443340549, np.float32: 0.54930615}
_W23_HALF = np.array([[1.125, 1.375, 1.625], [1.875, 2.125, 2.375]])
# ... and with tanh(alpha) = -1/2: -1/2 (3/4 flip(w) + 1/4 w) = -flip(_W23_HALF).
_W23_MINUS_HALF = np.array([[-2.375, -2.125, -1.875], [-1.625, -1.375, -1.125]])


def _w_tilde_failures(fn, dtype):
    """Checks of a w~ function fn(w, alpha, merge_name) -> array; returns the names of those that fail."""
    failed = []
    rng = np.random.default_rng(5)
    w = rng.standard_normal((3, 2, 3, 4)).astype(dtype)
    fw = w[:, :, ::-1, ::-1]
    # alpha = 0: tanh 0 = 0 zeroes the blend.
    if not np.array_equal(fn(w, np.zeros((3, 2), dtype), "sum"), np.zeros_like(w)):
        failed.append("alpha 0")
    # alpha = +-20: tanh rounds to +-1 in both dtypes, so w~ = w and w~ = -flip(w) exactly.
    if not np.array_equal(fn(w, np.full((3, 2), 20.0, dtype), "sum"), w):
        failed.append("alpha +20")
    if not np.array_equal(fn(w, np.full((3, 2), -20.0, dtype), "sum"), -fw):
        failed.append("alpha -20")
    # tanh alpha = +-1/2 on the asymmetric element, against the hand-computed values.
    w23 = _W23.astype(dtype).reshape(1, 1, 2, 3)
    a = _ALPHA_HALF[dtype]
    if not np.array_equal(fn(w23, np.full((1, 1), a, dtype), "sum")[0, 0], _W23_HALF.astype(dtype)):
        failed.append("tanh 1/2")
    if not np.array_equal(fn(w23, np.full((1, 1), -a, dtype), "sum")[0, 0], _W23_MINUS_HALF.astype(dtype)):
        failed.append("tanh -1/2")
    # Shapes: a per-pair (Cout, Cin) alpha, a 0-d shared one, and the identity merge's (C,) and (C, 1),
    # each entry from {0, 20, -20} so that every block has its own closed form.
    choice = rng.integers(0, 3, (3, 2))
    vals = np.array([0.0, 20.0, -20.0], dtype)
    closed = lambda k, blk, fblk: (np.zeros_like(blk), blk, -fblk)[k]  # noqa: E731
    got = fn(w, vals[choice], "sum")
    if not all(np.array_equal(got[o, i], closed(choice[o, i], w[o, i], fw[o, i])) for o in range(3) for i in range(2)):
        failed.append("per-pair alpha")
    if not np.array_equal(fn(w, np.array(-20.0, dtype), "max"), -fw):
        failed.append("shared 0-d alpha")
    wi = w[:, :1]
    fwi = wi[:, :, ::-1, ::-1]
    for shape in ((3,), (3, 1)):
        got = fn(wi, vals[choice[:, 0]].reshape(shape), "identity")
        if not all(np.array_equal(got[c, 0], closed(choice[c, 0], wi[c, 0], fwi[c, 0])) for c in range(3)):
            failed.append(f"identity alpha {shape}")
    # Derivatives, by central differences in float64, against the closed forms
    # d w~_j / d w_k = t (1 + t) / 2 [k = j] + t (1 - t) / 2 [k = flip(j)] and
    # d w~ / d alpha = (1 - t^2) ((1 - 2 t) / 2 flip(w) + (1 + 2 t) / 2 w).
    if dtype == np.float64:
        w1 = w[:1, :1].copy()
        alpha = 0.37
        t = math.tanh(alpha)
        eps = 1e-6
        fd = (fn(w1, np.full((1, 1), alpha + eps), "sum") - fn(w1, np.full((1, 1), alpha - eps), "sum")) / (2 * eps)
        want = (1 - t * t) * ((1 - 2 * t) / 2 * w1[:, :, ::-1, ::-1] + (1 + 2 * t) / 2 * w1)
        if np.max(np.abs(fd - want)) > 1e-8:
            failed.append("d/d alpha")
        KH, KW = w1.shape[2:]
        for kh, kw in ((0, 0), (1, 2), (2, 1)):
            d = np.zeros_like(w1)
            d[0, 0, kh, kw] = eps
            fd = (fn(w1 + d, np.full((1, 1), alpha), "sum") - fn(w1 - d, np.full((1, 1), alpha), "sum")) / (2 * eps)
            want = np.zeros_like(w1)
            want[0, 0, kh, kw] += t * (1 + t) / 2
            want[0, 0, KH - 1 - kh, KW - 1 - kw] += t * (1 - t) / 2
            if np.max(np.abs(fd - want)) > 1e-8:
                failed.append(f"d/d w[{kh},{kw}]")
    return failed


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_smorph_w_tilde_closed_forms(dtype):
    """oracle.smorph_w_tilde against closed forms: alpha = 0, +-20, tanh alpha = +-1/2 by hand on an
    asymmetric element, the per-pair / shared / identity alpha shapes, and its derivatives in w and
    alpha by central differences."""
    assert _w_tilde_failures(O.smorph_w_tilde, dtype) == []


def test_smorph_w_tilde_planted_mistakes_are_caught():
    """Plausible mistakes in the blend each fail at least one of the closed-form checks: the two
    weights swapped, the flip missing or along one axis only, the leading tanh missing, the identity
    alpha broadcast along the input channels."""
    import torch

    def variant(mistake):
        def fn(w, alpha, merge_name):
            wt, at = torch.as_tensor(np.ascontiguousarray(w)), torch.as_tensor(np.asarray(alpha))
            if mistake == "identity broadcast" and merge_name == "identity":
                ta = torch.tanh(at).reshape(1, -1, 1, 1)
            elif merge_name == "identity" or at.dim() == 1:
                ta = torch.tanh(at).view(-1, 1, 1, 1)
            else:
                ta = torch.tanh(at).unsqueeze(-1).unsqueeze(-1)
            t1, t2 = (1 + ta) / 2, (1 - ta) / 2
            if mistake == "swap":
                t1, t2 = t2, t1
            flipped = {"no flip": wt, "flip rows": wt.flip(dims=(-2,))}.get(mistake, wt.flip(dims=(-2, -1)))
            blend = t2 * flipped + t1 * wt
            return (blend if mistake == "no tanh" else ta * blend).numpy()
        return fn

    for mistake in ("swap", "no flip", "flip rows", "no tanh", "identity broadcast"):
        assert _w_tilde_failures(variant(mistake), np.float64), mistake


@pytest.mark.parametrize("merge,alpha_shape", [("sum", (3, 2)), ("max", ()), ("identity", (3,)), ("identity", (3, 1)), ("mean", (3,))])
def test_functional_smorph_passes_the_oracle_w_tilde(merge, alpha_shape, monkeypatch):
    """The product's functional.smorph hands its operator the same w~ as oracle.smorph_w_tilde, bit for
    bit (the operator itself is replaced by a recorder: no kernel runs on the CPU)."""
    import importlib

    import torch

    smod = importlib.import_module("morphocore_amd.functional.smorph")
    seen = {}

    class Rec:
        def smorph(self, x, w, alpha, merge_code):
            seen["w"] = w
            return x

    monkeypatch.setattr(smod, "ops", Rec())
    g = torch.Generator().manual_seed(3)
    cw = 1 if merge == "identity" else 2
    w = torch.randn(3, cw, 3, 5, generator=g, dtype=torch.float64)
    alpha = torch.randn(alpha_shape, generator=g, dtype=torch.float64) * 2
    smod.smorph(torch.zeros(1, cw if merge != "identity" else 3, 4, 4, dtype=torch.float64), w, alpha, channel_merge_mode=merge)
    assert np.array_equal(seen["w"].numpy(), O.smorph_w_tilde(w.numpy(), alpha.numpy(), merge))


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                                                    "libmorphocore_ref.so")), reason="the reference's CPU extension is not built")
@pytest.mark.parametrize("merge", ["mean", "max"])
def test_reference_runner_agrees_with_the_oracle(merge):
    """oracle/ref_run.py (the reference's own CPU extension in a child process, which the GPU tests at
    the configs' channel counts check against) returns what the C oracle computes for the same smorph."""
    from tests.helpers import reference_run

    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 3, 11, 13)).astype(np.float32)
    wt = (rng.standard_normal((4, 3, 5, 5)) * 0.1).astype(np.float32)
    alpha = rng.uniform(-4, 4, (4, 3)).astype(np.float32)
    g = rng.standard_normal((2, 4, 11, 13)).astype(np.float32)
    m = O.MERGES[merge]
    got = reference_run("smorph", x=x, wt=wt, alpha=alpha, grad=g, merge=np.array(m))
    assert np.array_equal(got["out"], O.smorph_forward(m, x, wt, alpha))
    for k, want in zip(("grad_input", "grad_weight", "grad_alpha"), O.smorph_backward(m, x, wt, alpha, g)):
        assert normwise_error(got[k], want) <= 1e-6, k


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_smorph_term_magnitudes(dtype):
    """The oracle's sums of the weight, alpha and beta terms' magnitudes (the scale of the GPU tests'
    measure for sums that cancel): equal to the gradient where every term has one sign (a 1x2 element with alpha > 0
    and a positive output gradient: each pixel's terms pg (v - ref)(v - out) are 0 and positive), at least
    the gradient's magnitude otherwise, unchanged by the gradient's sign, linear in its scale, summed over
    the pairs for a shared alpha, and with the normal backward unchanged afterwards."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 3, 6, 9)).astype(dtype)
    w = (rng.standard_normal((2, 3, 1, 2)) * 0.3).astype(dtype)
    alpha = rng.uniform(0.5, 3.0, (2, 3)).astype(dtype)
    gpos = np.abs(rng.standard_normal((2, 2, 6, 9))).astype(dtype)
    tol = 1e-6 if dtype == np.float32 else 1e-12
    assert normwise_error(O.smorph_term_magnitudes(O.ADD, x, w, alpha, gpos)[1], O.smorph_backward(O.ADD, x, w, alpha, gpos)[2]) <= tol
    g = rng.standard_normal((2, 2, 6, 9)).astype(dtype)
    before = O.smorph_backward(O.AVERAGE, x, w, alpha, g)
    for merge in (O.ADD, O.AVERAGE, O.MAX, O.MIN):
        grads = O.smorph_backward(merge, x, w, alpha, g)[1:]
        mags = O.smorph_term_magnitudes(merge, x, w, alpha, g)
        for grad, mag, mag_neg, mag2 in zip(grads, mags, O.smorph_term_magnitudes(merge, x, w, alpha, -g),
                                            O.smorph_term_magnitudes(merge, x, w, alpha, 2 * g)):
            assert np.all(mag >= np.abs(grad) * (1 - tol)), merge
            assert np.array_equal(mag_neg, mag), merge
            assert normwise_error(mag2, 2 * mag) <= tol, merge
    shared = np.asarray(alpha[0, 0])
    per_pair = O.smorph_term_magnitudes(O.ADD, x, w, np.full((2, 3), shared, dtype), g)[1]
    assert abs(float(O.smorph_term_magnitudes(O.ADD, x, w, shared, g)[1]) - float(per_pair.sum(dtype=np.float64))) <= tol * float(per_pair.sum())
    after = O.smorph_backward(O.AVERAGE, x, w, alpha, g)
    assert all(np.array_equal(p, q) for p, q in zip(before, after))
    beta = rng.standard_normal(2).astype(dtype)
    ga, gb = O.smorph_scm_backward(x, w, alpha, beta, g)[2:]
    mw, ma, mb = O.smorph_scm_term_magnitudes(x, w, alpha, beta, g)
    gw = O.smorph_scm_backward(x, w, alpha, beta, g)[1]
    assert np.all(mw >= np.abs(gw) * (1 - tol)) and np.all(ma >= np.abs(ga) * (1 - tol)) and np.all(mb >= np.abs(gb) * (1 - tol))
    assert np.array_equal(O.smorph_scm_term_magnitudes(x, w, alpha, beta, -g)[2], mb)
