"""torch.autograd.gradcheck of the operators on the GPU in float64, as the reference's own tests run it
(tests/functional/test_morpho_operation.py:246-389): the analytic gradients come from the HIP backward
kernels, the numerical ones from central differences of the HIP forward kernels.

* dilation and erosion, every merge, with geodesic padding as the reference's tests run them
  (tests/functional/utils.py:52-53; with replicate padding the reference's backward drops the
  gradient of a winning tap that reads a clamped pixel outside the image, which the golden vectors pin,
  so central differences of the forward disagree with it there by design), over shapes with one or
  several channels, odd and even elements and planes smaller than the element; the inputs and
  elements are spread as x * 10 + arange (the reference's test_grad_random, :333-337), so that no two
  taps of a window come within the finite-difference step of a tie, where the max-plus operators are
  not differentiable;
* smorph for alpha from -1000 to 1000, per-pair, shared (0-d) and per-channel (identity) alpha, every
  merge, with the gradients of x, w and alpha (:360-389);
* the compositions opening, closing (both through the fused operator) and sigma_layer.
Each case prints its name before the GPU work."""
import pytest
import torch

import morphocore_amd as mca

pytestmark = pytest.mark.gpu

F = mca.functional
MERGES = ["max", "min", "sum", "mean", "identity"]
# (B, Cin, Cout, H, W, KH, KW)
SHAPES = [(1, 1, 1, 5, 5, 3, 3), (2, 3, 4, 7, 9, 3, 3), (1, 2, 2, 6, 11, 5, 5), (2, 2, 3, 8, 8, 3, 3), (1, 3, 1, 4, 13, 5, 3),
          (1, 2, 3, 9, 6, 2, 4), (1, 2, 2, 3, 2, 5, 5)]


def _spread(shape, gen, scale=10.0):
    """randn * scale + arange over the tensor: distinct, well separated values (no near ties)."""
    n = 1
    for s in shape:
        n *= s
    v = torch.randn(shape, generator=gen, dtype=torch.float64) * scale + torch.arange(n, dtype=torch.float64).reshape(shape)
    return v.cuda().requires_grad_()


def _case(shape, merge, seed):
    B, Cin, Cout, H, W, KH, KW = shape
    if merge == "identity":
        Cout = Cin
    gen = torch.Generator().manual_seed(seed)
    x = _spread((B, Cin, H, W), gen)
    w = _spread((Cout, 1 if merge == "identity" else Cin, KH, KW), gen, scale=5.0)
    return x, w


@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_gradcheck_dilation_erosion(op, merge):
    fn = getattr(F, op)
    for si, shape in enumerate(SHAPES):
        print(f"gradcheck {op} {merge} {shape}", flush=True)
        x, w = _case(shape, merge, 100 + si)
        for save in (True, False):
            assert torch.autograd.gradcheck(lambda a, b: fn(a, b, merge, "geodesic", save_indices=save), (x, w), eps=1e-6,
                                            atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("alpha", [-1000.0, -10.0, -1.0, -0.25, 0.0, 0.25, 1.0, 10.0, 1000.0])
@pytest.mark.parametrize("merge", MERGES)
def test_gradcheck_smorph(merge, alpha):
    for si, shape in enumerate([(1, 2, 3, 6, 7, 3, 3), (2, 1, 2, 5, 4, 3, 5), (1, 3, 2, 4, 9, 5, 5)]):
        B, Cin, Cout, H, W, KH, KW = shape
        if merge == "identity":
            Cout = Cin
        print(f"gradcheck smorph {merge} alpha={alpha} {shape}", flush=True)
        gen = torch.Generator().manual_seed(200 + si)
        # Smaller spreads than the max-plus cases keep the softmax weights away from 0 and 1 at
        # |alpha| <= 10 (where the smooth operator's derivatives are large and the differences
        # need them resolved); at |alpha| = 1000 it is the hard extremum of well separated taps.
        x = (torch.randn((B, Cin, H, W), generator=gen, dtype=torch.float64)).cuda().requires_grad_()
        w = (torch.randn((Cout, 1 if merge == "identity" else Cin, KH, KW), generator=gen, dtype=torch.float64) * 0.5).cuda().requires_grad_()
        if abs(alpha) >= 1000:
            x = _spread((B, Cin, H, W), gen, scale=1.0)
        shapes = [(Cout, Cin) if merge != "identity" else (Cout,), ()]
        for ashape in shapes:
            a = (torch.full(ashape, alpha, dtype=torch.float64) + (torch.rand(ashape, generator=gen, dtype=torch.float64) * 0.1 if alpha else 0)).cuda()
            a.requires_grad_()
            assert torch.autograd.gradcheck(lambda xx, ww, aa: F.smorph(xx, ww, aa, channel_merge_mode=merge), (x, w, a), eps=1e-6,
                                            atol=1e-6, rtol=1e-4)


def test_gradcheck_compositions():
    gen = torch.Generator().manual_seed(300)
    for K in (3, 5):
        print(f"gradcheck opening / closing / sigma_layer {K}x{K}", flush=True)
        x = _spread((2, 3, 9, 10), gen)
        w1 = _spread((3, 1, K, K), gen, scale=5.0)
        w2 = _spread((3, 1, K, K), gen, scale=5.0)
        for fn in (F.opening, F.closing):
            assert torch.autograd.gradcheck(lambda a, b, c: fn(a, b, c, "identity", "geodesic"), (x, w1, w2), eps=1e-6, atol=1e-6, rtol=1e-5)
        alpha = torch.randn((3, 1), generator=gen, dtype=torch.float64).cuda().requires_grad_()
        assert torch.autograd.gradcheck(lambda a, b, c: F.sigma_layer(a, b, c, "identity", "geodesic"), (x, w1, alpha), eps=1e-6, atol=1e-6,
                                        rtol=1e-4)
