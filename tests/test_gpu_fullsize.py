"""Parity at BASELINE.json's full sizes (configs[2], configs[3] and configs[4]'s layers), where the
CPU oracle cannot run the whole problem, through properties that do not depend on the size:

* region checks: an output depends only on the inputs of its window, so the oracle run on a crop of
  the input reproduces the outputs of a region whose windows lie inside the crop (a crop that reaches
  the image's edge keeps the edge's padding semantics). The same holds for grad_input: a region's
  input gradient receives only from outputs within the element's radius of it, whose windows lie
  within twice the radius. Regions at the top-left corner, the bottom-right corner and inside the
  image, of the first and last batch elements;
* conservation with an all-ones output gradient: a smorph pair routes each output pixel's gradient
  over its taps with weights p_k (1 + alpha (v_k - out)), which sum to 1 since out = sum p_k v_k;
  so every grad_weight[o, i] sums to B*H*W (times the merge's scale) and grad_input to
  B*Cout*Cin*H*W (the same scale), within float32 rounding. A max / min / identity merge routes
  each output pixel's gradient to exactly one tap: grad_weight sums exactly to the pixel count and
  grad_input is a non-negative integer count, checked on regions (with replicate padding a winning
  tap outside the image routes to no input pixel, as in the reference, so its total is at most the
  pixel count).

Each case prints its name before the GPU work. Sizes and distributions are BASELINE.json's configs.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import normwise_error, seeded

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


@pytest.fixture(autouse=True)
def _ops():
    import morphocore_amd  # noqa: F401  (registers torch.ops.morphocore)


def _regions(B, H, W, size):
    """(b, r0, c0) of output regions of `size` x `size`: corners and the middle of the first and last
    batch elements."""
    return [(0, 0, 0), (0, (H - size) // 2, (W - size) // 2), (B - 1, H - size, W - size), (B - 1, 0, W - size)]


def _crop(n, lo, hi, radius):
    return max(0, lo - radius), min(n, hi + radius)


def _check_forward_regions(out_gpu, x, fn_oracle, P, size, tol):
    """Compares out_gpu over regions with the oracle run on crops of x (radius P around the region)."""
    B, _, H, W = x.shape
    for b, r0, c0 in _regions(B, H, W, size):
        h0, h1 = _crop(H, r0, r0 + size, P)
        w0, w1 = _crop(W, c0, c0 + size, P)
        ref = fn_oracle(np.ascontiguousarray(_np(x[b:b + 1, :, h0:h1, w0:w1])))
        want = ref[0, :, r0 - h0:r0 - h0 + size, c0 - w0:c0 - w0 + size]
        got = _np(out_gpu[b, :, r0:r0 + size, c0:c0 + size])
        if tol == 0:
            assert np.array_equal(got, want), f"forward region {(b, r0, c0)}"
        else:
            err = normwise_error(got, want)
            assert err <= tol, f"forward region {(b, r0, c0)}: {err}"


def _check_grad_input_regions(gx_gpu, x, g, fn_oracle_bwd, P, size, tol):
    """grad_input over regions against the oracle's backward on crops of radius 2P (and the output
    gradient on the same crop)."""
    B, _, H, W = x.shape
    for b, r0, c0 in _regions(B, H, W, size):
        h0, h1 = _crop(H, r0, r0 + size, 2 * P)
        w0, w1 = _crop(W, c0, c0 + size, 2 * P)
        xc = np.ascontiguousarray(_np(x[b:b + 1, :, h0:h1, w0:w1]))
        gc = np.ascontiguousarray(_np(g[b:b + 1, :, h0:h1, w0:w1]))
        want = fn_oracle_bwd(xc, gc)[0, :, r0 - h0:r0 - h0 + size, c0 - w0:c0 - w0 + size]
        got = _np(gx_gpu[b, :, r0:r0 + size, c0:c0 + size])
        if tol == 0:
            assert np.array_equal(got, want), f"grad_input region {(b, r0, c0)}"
            continue
        err = normwise_error(got, want)
        assert err <= tol, f"grad_input region {(b, r0, c0)}: {err}"


def _smorph_full(merge, B, C, H, W, K, a, x_kind, w_scale, seed):
    """One smorph layer at full size through torch.ops.morphocore.smorph (w~ given directly): forward
    and grad_input regions against the oracle with a random output gradient, then the conservation
    sums with an all-ones one."""
    dev = torch.device("cuda")
    P = K // 2
    m = O.MERGES[merge]
    scale = 1.0 / C if merge == "mean" else 1.0
    x = seeded(seed, B, C, H, W, kind=x_kind).to(dev)
    wt = seeded(seed + 1, C, C, K, K, kind="randn", scale=w_scale).to(dev)
    alpha = torch.full((C, C), a, device=dev)
    g = seeded(seed + 2, B, C, H, W, kind="randn").to(dev)
    xr = x.clone().requires_grad_(True)
    out = torch.ops.morphocore.smorph(xr, wt, alpha, m)
    out.backward(g)
    an, wn = _np(alpha), _np(wt)
    _check_forward_regions(out, x, lambda xc: O.smorph_forward(m, xc, wn, an), P, 8, 1e-6)
    _check_grad_input_regions(xr.grad, x, g, lambda xc, gc: O.smorph_backward(m, xc, wn, an, gc)[0], P, 8, 1e-6)
    del out, xr
    # Conservation with an all-ones output gradient.
    xr = x.clone().requires_grad_(True)
    wr = wt.clone().requires_grad_(True)
    out = torch.ops.morphocore.smorph(xr, wr, alpha, m)
    out.backward(torch.ones_like(out))
    per_pair = wr.grad.double().sum(dim=(2, 3))
    n = B * H * W * scale
    err = float((per_pair - n).abs().max()) / n
    assert err <= 1e-6, f"grad_weight[o, i] sums: {err}"
    total = float(xr.grad.double().sum())
    assert abs(total - n * C * C) / (n * C * C) <= 1e-6, f"grad_input sum: {total}"


@pytest.mark.parametrize("a", [-20.0, -1.0, 0.0, 1.0, 20.0])
def test_config3_full_size_smorph(a):
    """configs[2] at its full size: (8, 64, 256, 256), w~ (64, 64, 7, 7) ~N(0, 0.1), mean merge."""
    print(f"configs[2] full size, alpha {a}", flush=True)
    _smorph_full("mean", 8, 64, 256, 256, 7, a, "randn", 0.1, 40)


def test_config5_full_size_layers():
    """configs[4]'s three layers at full size (8, 64, 512, 512), 11x11: dilation (max, replicate) and
    erosion (min, replicate) forwards and their all-ones backward's grad_input exactly on regions,
    their grad_weight sums exactly; the smorph layer (alpha 5, sum) as configs[2] above. x ~U[0, 1),
    elements ~N(0, 0.05)."""
    dev = torch.device("cuda")
    B, C, H, W, K = 8, 64, 512, 512, 11
    P = K // 2
    x = seeded(0, B, C, H, W).to(dev)
    for op, merge in ((O.DILATION, "max"), (O.EROSION, "min")):
        print(f"configs[4] full size, {'dilation' if op == O.DILATION else 'erosion'} {merge}", flush=True)
        w = seeded(1 + op, C, C, K, K, kind="randn", scale=0.05).to(dev)
        fn = torch.ops.morphocore.dilation if op == O.DILATION else torch.ops.morphocore.erosion
        xr = x.clone().requires_grad_(True)
        wr = w.clone().requires_grad_(True)
        out = fn(xr, wr, O.MERGES[merge], O.PADDINGS["replicate"], 0.0, True, 0.0)
        wn = _np(w)
        _check_forward_regions(out, x, lambda xc: O.morpho_forward(op, O.MERGES[merge], O.PADDINGS["replicate"], 0.0, xc, wn)[0],
                               P, 8, 0)
        ones = torch.ones_like(out)
        out.backward(ones)
        # Each output pixel's gradient goes to exactly one (input channel, tap): grad_weight[o] sums to
        # +-B*H*W; grad_input counts the winners that read each input pixel.
        sign = 1.0 if op == O.DILATION else -1.0
        per_o = wr.grad.double().sum(dim=(1, 2, 3))
        assert torch.equal(per_o, torch.full_like(per_o, sign * B * H * W))
        gx = xr.grad.double()
        assert torch.equal(gx, gx.round()) and bool((gx >= 0).all())
        assert float(gx.sum()) <= B * C * H * W
        _check_grad_input_regions(
            xr.grad, x, ones,
            lambda xc, gc: O.morpho_backward(op, O.MERGES[merge], O.PADDINGS["replicate"], 0.0, xc, wn, gc)[0], P, 8, 0.0)
        del out, xr, wr, gx, ones
        torch.cuda.empty_cache()
    del x
    torch.cuda.empty_cache()
    print("configs[4] full size, smorph sum alpha 5", flush=True)
    _smorph_full("sum", B, C, H, W, K, 5.0, "rand", 0.05, 50)


def test_config4_full_size_identity_f64():
    """configs[3] at its full size (32, 128, 112, 112) float64, dilation identity 3x3 (replicate):
    regions of the forward and of the all-ones backward's grad_input exactly; grad_weight[c] sums to
    B*H*W exactly."""
    print("configs[3] full size", flush=True)
    dev = torch.device("cuda")
    B, C, H, W = 32, 128, 112, 112
    x = seeded(0, B, C, H, W, dtype=torch.float64, low=-1.0, scale=2.0).to(dev)
    w = seeded(1, C, 1, 3, 3, dtype=torch.float64, kind="randn", scale=0.1).to(dev)
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    out = torch.ops.morphocore.dilation(xr, wr, O.MERGES["identity"], O.PADDINGS["replicate"], 0.0, True, 0.0)
    wn = _np(w)
    _check_forward_regions(out, x, lambda xc: O.morpho_forward(O.DILATION, O.MERGES["identity"], O.PADDINGS["replicate"], 0.0, xc, wn)[0],
                           1, 16, 0)
    ones = torch.ones_like(out)
    out.backward(ones)
    per_c = wr.grad.sum(dim=(1, 2, 3))
    assert torch.equal(per_c, torch.full_like(per_c, float(B * H * W)))
    gx = xr.grad
    assert torch.equal(gx, gx.round()) and bool((gx >= 0).all())
    assert float(gx.sum()) <= B * C * H * W
    _check_grad_input_regions(
        gx, x, ones,
        lambda xc, gc: O.morpho_backward(O.DILATION, O.MERGES["identity"], O.PADDINGS["replicate"], 0.0, xc, wn, gc)[0], 1, 16, 0.0)


def test_scm_full_size():
    """smorph_scm at configs[2]'s full size (bench.py --config 9): (8, 64, 256, 256), w~ (64, 64, 7, 7)
    ~N(0, 0.1), alpha 1, beta per output channel: forward and grad_input regions against the oracle
    on crops; with an all-ones output gradient the soft merge's weights q_i (1 + beta (c_i - out)) sum
    to 1 over the input channels, and each pair's routing weights to 1 over its taps, so grad_weight[o]
    sums to B*H*W and grad_input to B*Cout*H*W."""
    print("smorph_scm full size", flush=True)
    dev = torch.device("cuda")
    B, C, H, W, K = 8, 64, 256, 256, 7
    P = K // 2
    x = seeded(60, B, C, H, W, kind="randn").to(dev)
    wt = seeded(61, C, C, K, K, kind="randn", scale=0.1).to(dev)
    alpha = torch.full((C, C), 1.0, device=dev)
    beta = (torch.linspace(-3.0, 3.0, C)).to(dev)
    g = seeded(62, B, C, H, W, kind="randn").to(dev)
    xr = x.clone().requires_grad_(True)
    out = torch.ops.morphocore.smorph_scm(xr, wt, alpha, beta)
    out.backward(g)
    an, wn, bn = _np(alpha), _np(wt), _np(beta)
    _check_forward_regions(out, x, lambda xc: O.smorph_scm_forward(xc, wn, an, bn), P, 8, 1e-6)
    _check_grad_input_regions(xr.grad, x, g, lambda xc, gc: O.smorph_scm_backward(xc, wn, an, bn, gc)[0], P, 8, 1e-6)
    del out, xr
    xr = x.clone().requires_grad_(True)
    wr = wt.clone().requires_grad_(True)
    out = torch.ops.morphocore.smorph_scm(xr, wr, alpha, beta)
    out.backward(torch.ones_like(out))
    per_o = wr.grad.double().sum(dim=(1, 2, 3))
    n = B * H * W
    err = float((per_o - n).abs().max()) / n
    assert err <= 1e-6, f"grad_weight[o] sums: {err}"
    total = float(xr.grad.double().sum())
    assert abs(total - n * C) / (n * C) <= 1e-6, f"grad_input sum: {total}"
