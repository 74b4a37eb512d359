"""More GPU coverage against the oracle: the device exponential bit for bit, the nn layers (forward,
backward, training / evaluation switching of weight noise and dropout, reference
tests/functional/test_weight_noise.py:93-127), determinism of repeated runs, and a smorph shape whose
two backward plans lay out different numbers of partial slots."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def test_smorph_exp_bitwise_float32():
    """Every float32 in [-200, -0] (both signs of zero, subnormals, the underflow threshold), NaN and
    -inf: the kernels' exponential equals the oracle's restatement of the reference's bit for bit."""
    from morphocore_amd import _native

    dev = torch.device("cuda")
    lo = np.array([-0.0], np.float32).view(np.uint32)[0]
    hi = np.array([-200.0], np.float32).view(np.uint32)[0]
    chunk = 1 << 26
    checked = 0
    for start in range(int(lo), int(hi) + 1, chunk):
        bits = np.arange(start, min(start + chunk, int(hi) + 1), dtype=np.uint32)
        x = bits.view(np.float32)
        y = torch.empty(x.size, dtype=torch.float32, device=dev)
        _native.probe_smorph_exp(torch.from_numpy(x).to(dev), y)
        got = y.cpu().numpy().view(np.uint32)
        want = O.exp_array(x).view(np.uint32)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{bad.size} mismatches, first at x = {x[bad[0]]!r}"
        checked += x.size
    assert checked == int(hi) - int(lo) + 1
    special = np.array([0.0, np.nan, -np.inf, -87.33654, -87.3365, -103.97], np.float32)
    y = torch.empty(special.size, dtype=torch.float32, device=dev)
    _native.probe_smorph_exp(torch.from_numpy(special).to(dev), y)
    got, want = y.cpu().numpy(), O.exp_array(special)
    assert np.array_equal(got.view(np.uint32)[1:2] & 0x7FC00000, np.array([0x7FC00000], np.uint32))  # NaN stays NaN
    assert np.array_equal(np.delete(got, 1).view(np.uint32), np.delete(want, 1).view(np.uint32))


def test_smorph_exp_bitwise_float64():
    """float64: 2^24 arguments spread over [-760, 0] plus every power-of-two neighbourhood near 0 and
    the underflow threshold, bit for bit against the oracle."""
    from morphocore_amd import _native

    rng = np.random.default_rng(5)
    x = np.concatenate([-rng.random(1 << 24) * 760.0, -np.logspace(-300, 2.8, 4096), np.nextafter(-708.39641, 0.0) + np.arange(-64, 64) * 1e-13,
                        np.array([-0.0, 0.0, -np.inf])])
    dev = torch.device("cuda")
    y = torch.empty(x.size, dtype=torch.float64, device=dev)
    _native.probe_smorph_exp(torch.from_numpy(x).to(dev), y)
    assert np.array_equal(y.cpu().numpy().view(np.uint64), O.exp_array(x).view(np.uint64))


@pytest.mark.parametrize("layer", ["Dilation", "Erosion", "SMorph"])
def test_nn_layers_forward_backward_against_oracle(layer):
    """The layers' forward and backward on the GPU (weights set away from their zero
    initialisation) against the oracle, through the functional layer's transforms (erosion's flip,
    smorph's w~)."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    torch.manual_seed(0)
    cls = getattr(mca.nn, layer)
    kwargs = {"channel_merge_mode": "max" if layer != "SMorph" else "mean"}
    if layer == "SMorph":
        kwargs["init_alpha"] = 1.5
    m = cls(3, 4, (5, 3), **kwargs).to(dev)
    with torch.no_grad():
        m.weight.copy_(seeded(101, *m.weight.shape, kind="randn", scale=0.2))
    x = seeded(102, 2, 3, 17, 66, kind="randn")
    g = seeded(103, 2, 4, 17, 66, kind="randn")
    xd = x.to(dev).requires_grad_(True)
    out = m(xd)
    out.backward(g.to(dev))
    w = m.weight.detach().cpu()
    if layer == "SMorph":
        alpha = m.alpha.detach().cpu()
        wt = O.smorph_w_tilde(w.numpy(), alpha.numpy(), "mean")
        ref = O.smorph_forward(O.AVERAGE, x.numpy(), wt, alpha.numpy())
        gx, _, _ = O.smorph_backward(O.AVERAGE, x.numpy(), wt, alpha.numpy(), g.numpy())
        assert normwise_error(_np(out), ref) <= 1e-6
        assert m.alpha.grad is not None and torch.isfinite(m.alpha.grad).all()
    else:
        op = O.DILATION if layer == "Dilation" else O.EROSION
        wk = w.numpy() if layer == "Dilation" else np.ascontiguousarray(w.flip((-2, -1)).numpy())
        ref, idx = O.morpho_forward(op, O.MAX, O.REPLICATE, 0.0, x.numpy(), wk, save_indices=True)
        gx, gwk = O.morpho_backward(op, O.MAX, O.REPLICATE, 0.0, x.numpy(), wk, g.numpy(), indices=idx)
        assert np.array_equal(_np(out), ref)
        gw = gwk if layer == "Dilation" else gwk[:, :, ::-1, ::-1]
        assert normwise_error(_np(m.weight.grad), gw) <= 1e-6
    assert normwise_error(_np(xd.grad), gx) <= 1e-6


@pytest.mark.parametrize("layer", ["Dilation", "Erosion"])
def test_nn_layers_follow_training_mode(layer):
    """Weight noise and dropout act in training only (reference test_weight_noise.py:113-127): in
    evaluation two calls agree and equal the noise-free layer; in training two seeds differ, the same
    seed repeats exactly, and the backward runs."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    torch.manual_seed(0)
    m = getattr(mca.nn, layer)(3, 3, 3, noise_scale=0.5, weight_dropout=0.3).to(dev)
    with torch.no_grad():
        m.weight.copy_(seeded(104, *m.weight.shape, kind="randn", scale=0.3))
    x = seeded(105, 2, 3, 12, 70, kind="randn").to(dev)
    clean = getattr(mca.nn, layer)(3, 3, 3).to(dev)
    with torch.no_grad():
        clean.weight.copy_(m.weight)
    m.eval()
    assert torch.equal(m(x), m(x)) and torch.equal(m(x), clean(x))
    m.train()
    torch.manual_seed(1)
    first = m(x)
    torch.manual_seed(2)
    second = m(x)
    torch.manual_seed(1)
    again = m(x)
    assert not torch.equal(first, second)
    assert torch.equal(first, again)
    first.sum().backward()
    assert torch.isfinite(m.weight.grad).all()


@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_seeded_dropout_matches_reference_draw_order(op):
    """Weight dropout with a seed drops the taps the reference's loop drops (functional/dilation.py:78-87:
    rand_like(w) > p, then for each (o, i) pair without a survivor one randint, in (o, i) order), and
    the dropped taps act as -inf (dilation) / +inf after erosion's flip."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    w = seeded(106, 4, 3, 3, 3, kind="randn", scale=0.3).to(dev)
    x = seeded(107, 1, 3, 10, 66, kind="randn").to(dev)
    fn = getattr(mca.functional, op)
    torch.manual_seed(11)
    out = fn(x, w, "sum", "geodesic", weight_dropout=0.9, training=True)
    # The reference's draw, restated on the same generator.
    torch.manual_seed(11)
    keep = torch.rand_like(w) > 0.9
    for i in range(w.shape[0]):
        for j in range(w.shape[1]):
            if not keep[i, j].any():
                flat = torch.randint(0, keep[i, j].numel(), (1,)).item()
                keep[i, j].view(-1)[flat] = True
    wd = torch.where(keep, w, torch.tensor(-float("inf"), device=dev))
    expected = fn(x, wd, "sum", "geodesic")
    assert torch.equal(out, expected)


@pytest.mark.parametrize("case", ["erosion-sum", "dilation-max", "smorph-saved", "smorph-recomputed", "scm"])
def test_repeated_runs_give_identical_weight_and_alpha_gradients(case, monkeypatch):
    """Two identical forward + backward runs give bit-identical grad_weight and grad_alpha (per-slot
    partials summed in a fixed order; the LDS bins add float values into double accumulators).
    grad_input of the smorph backwards is flushed from each workgroup's tile with float atomics at
    the tile halos, so it may differ in the last bits between runs; it is compared within the
    tolerance."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    monkeypatch.setenv("MORPHOCORE_AMD_SAVED_STATS_LIMIT", "0" if case == "smorph-recomputed" else str(1 << 40))
    runs = []
    for _ in range(2):
        torch.manual_seed(0)
        if case in ("erosion-sum", "dilation-max"):
            x = seeded(108, 4, 32, 64, 64).to(dev).requires_grad_(True)
            w = seeded(109, 32, 32, 5, 5, kind="randn", scale=0.05).to(dev).requires_grad_(True)
            fn = mca.functional.erosion if case == "erosion-sum" else mca.functional.dilation
            out = fn(x, w, case.split("-")[1], "replicate")
            params = [w]
        else:
            x = seeded(110, 2, 16, 64, 70, kind="randn").to(dev).requires_grad_(True)
            w = seeded(111, 16, 16, 7, 7, kind="randn", scale=0.1).to(dev).requires_grad_(True)
            a = torch.full((16, 16), 1.5, device=dev, requires_grad=True)
            if case == "scm":
                b = torch.linspace(-2.0, 2.0, 16, device=dev).requires_grad_(True)
                out = mca.functional.smorph(x, w, a, beta=b)
                params = [w, a, b]
            else:
                out = mca.functional.smorph(x, w, a, channel_merge_mode="mean")
                params = [w, a]
        out.backward(seeded(112, *out.shape, kind="randn").to(dev))
        runs.append([_np(x.grad)] + [_np(p.grad) for p in params])
    first, second = runs
    assert normwise_error(second[0], first[0]) <= 1e-6
    for a_, b_ in zip(first[1:], second[1:]):
        assert np.array_equal(a_, b_)


def test_smorph_saved_statistics_at_a_shape_with_more_saved_slots():
    """4 x 64 x 100 x 100 with a 3x3 element: the backward from saved statistics lays out 26 slots
    per batch element where the recomputing one lays out 25; both match the oracle."""
    import morphocore_amd as mca

    dev = torch.device("cuda")
    x = seeded(113, 4, 64, 100, 100, kind="randn")
    w = seeded(114, 64, 64, 3, 3, kind="randn", scale=0.1)
    alpha = torch.full((64, 64), 2.0)
    g = seeded(115, 4, 64, 100, 100, kind="randn")
    xd, wd, ad = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True), alpha.to(dev).requires_grad_(True)
    out = torch.ops.morphocore.smorph(xd, wd, ad, O.ADD)
    from morphocore_amd import _C
    assert _C.saved_stats_live_bytes(torch.cuda.current_device()) >= 12 * 4 * 64 * 64 * 100 * 100
    out.backward(g.to(dev))
    ref = O.smorph_forward(O.ADD, x.numpy(), w.numpy(), alpha.numpy())
    gx, gw, ga = O.smorph_backward(O.ADD, x.numpy(), w.numpy(), alpha.numpy(), g.numpy())
    assert normwise_error(_np(out), ref) <= 1e-6
    for got, want in ((xd.grad, gx), (wd.grad, gw), (ad.grad, ga)):
        assert normwise_error(_np(got), want) <= 1e-6
