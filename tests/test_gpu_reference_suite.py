"""The reference's own test suite (morphocore tests/functional/*.py), restated against this package on the
GPU.

Each test names the reference test it follows (file:line) and keeps that test's inputs, tolerances and
assertions. Where the reference compares its CPU and CUDA paths (test_cuda_cpu.py, test_padding.py:202-
240), the HIP path is compared with the oracle, the CPU restatement of the reference's extension; where
it compares with a numpy construction of the operators (tests/functional/utils.py:6-47,
test_padding.py:9-47), with the oracle's numpy brute force built the same way (``oracle.brute``). The
reference runs every test on 'cpu' and 'cuda'; this package has only the HIP device. Its four operations
(utils.py:52-78): 'dilation' and 'erosion' (sum merge and geodesic padding unless a test says otherwise)
and 'Sdilation' / 'Serosion', smorph with alpha = +1000 / -1000, which tends to them.

Two of the reference's tests are widened: its random-input gradcheck (test_morpho_operation.py:279-358)
checks the gradient of the input only (its weight does not require grad) and is run here for the weight
too; its identity-independence test (:213-241) skips CUDA and leaves its check commented out, which is
run here.
"""
import numpy as np
import pytest
import torch

import morphocore_amd.functional as F
import morphocore_amd.nn as N
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
OPERATIONS = ["Sdilation", "Serosion", "dilation", "erosion"]


def _run(operation, x, w, merge="sum", save_indices=True, padding="geodesic"):
    """The reference tests' dispatch_operation (tests/functional/utils.py:52-78)."""
    if operation in ("dilation", "erosion"):
        fn = F.dilation if operation == "dilation" else F.erosion
        return fn(x, w, channel_merge_mode=merge, save_indices=save_indices, padding_mode=padding)
    two_d = x.dim() == 2
    cin, cout = (1, 1) if two_d else (x.shape[1], w.shape[0])
    shape = (cout,) if merge == "identity" else (cout, cin)
    a = 1000.0 if operation == "Sdilation" else -1000.0
    return F.smorph(x, w, torch.full(shape, a, dtype=x.dtype, device=x.device), channel_merge_mode=merge)


def _brute(image, selem, operation, padding="geodesic", value=0.0):
    """One channel through the reference tests' numpy construction (utils.py:6-47, test_padding.py:9-47):
    dilation adds the element, erosion subtracts the flipped element; the hard and smooth operations
    share it."""
    op = O.DILATION if operation in ("dilation", "Sdilation") else O.EROSION
    se = selem if op == O.DILATION else np.ascontiguousarray(selem[::-1, ::-1])
    pad = O.PADDINGS[padding]
    fill = O.fill_value(op, pad, value, np.float64)
    best, _ = O.brute.pair(np.asarray(image, dtype=np.float64), np.asarray(se, dtype=np.float64), op, pad, fill)
    return best


def _close(operation, got, want):
    """The reference's tolerances for these comparisons (test_morpho_operation.py:22-25)."""
    tol = dict(rtol=1e-3, atol=1e-3) if operation.startswith("S") else dict(rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(got.detach().cpu().numpy(), want, **tol)


def _np(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape)


def _f32(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(DEV)


# ------------------------------------------------------------------------------------------------
# test_morpho_operation.py: TestMorphologicalOperations (:9-241)
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("operation", OPERATIONS)
def test_morphology_4d(operation):
    """test_morpho_operation.py:11-25: a 64x64 image and a 3x3 element as [1, 1, H, W] tensors."""
    image, kernel = _np(1, 64, 64), _np(2, 3, 3)
    got = _run(operation, _f32(image)[None, None], _f32(kernel)[None, None])[0, 0]
    _close(operation, got, _brute(image, kernel, operation))


@pytest.mark.parametrize("operation", OPERATIONS)
def test_morphology_2d(operation):
    """test_morpho_operation.py:27-41: the same with 2-D tensors (the operators keep the input's rank)."""
    image, kernel = _np(3, 64, 64), _np(4, 3, 3)
    got = _run(operation, _f32(image), _f32(kernel))
    assert got.shape == (64, 64)
    _close(operation, got, _brute(image, kernel, operation))


@pytest.mark.parametrize("operation", OPERATIONS)
def test_morphology_weird_size(operation):
    """test_morpho_operation.py:43-57: a 13x4 image, narrower than its 5x5 element."""
    image, kernel = _np(5, 13, 4), _np(6, 5, 5)
    _close(operation, _run(operation, _f32(image), _f32(kernel)), _brute(image, kernel, operation))


@pytest.mark.parametrize("operation", OPERATIONS)
def test_batch_morphology(operation):
    """test_morpho_operation.py:59-81: two images, one element."""
    images, kernel = _np(7, 2, 64, 64), _np(8, 3, 3)
    got = _run(operation, _f32(images)[:, None], _f32(kernel)[None, None])[:, 0]
    _close(operation, got, np.stack([_brute(im, kernel, operation) for im in images]))


@pytest.mark.parametrize("operation", OPERATIONS)
def test_one_channel_to_many(operation):
    """test_morpho_operation.py:83-121: one input channel, three elements, three output channels."""
    image, kernels = _np(9, 32, 32), _np(10, 3, 3, 3)
    got = _run(operation, _f32(image)[None, None], _f32(kernels)[:, None])[0]
    _close(operation, got, np.stack([_brute(image, k, operation) for k in kernels]))


@pytest.mark.parametrize("operation", OPERATIONS)
def test_many_channel_to_one(operation):
    """test_morpho_operation.py:123-168: three input channels summed into one output (sum merge)."""
    images, kernels = _np(11, 3, 32, 32), _np(12, 3, 3, 3)
    got = _run(operation, _f32(images)[None], _f32(kernels)[None])[0, 0]
    _close(operation, got, sum(_brute(images[c], kernels[c], operation) for c in range(3)))


@pytest.mark.parametrize("operation", OPERATIONS)
def test_many_channel_to_many(operation):
    """test_morpho_operation.py:170-211: every output channel sums the contributions of all inputs."""
    images, kernels = _np(13, 3, 32, 32), _np(14, 3, 3, 3, 3).astype(np.float32)
    got = _run(operation, _f32(images)[None], _f32(kernels))[0]
    want = np.stack([sum(_brute(images[i], kernels[o, i], operation) for i in range(3)) for o in range(3)])
    _close(operation, got, want)


@pytest.mark.parametrize("operation", OPERATIONS)
def test_identity_independence(operation):
    """test_morpho_operation.py:213-241: with the identity merge every output channel sees only its own
    input channel (the reference skips this on CUDA and leaves the check commented out; it is run here)."""
    g = torch.Generator().manual_seed(15)
    x = torch.randn(1, 2, 8, 8, generator=g).to(DEV)
    w = torch.randn(2, 1, 3, 3, generator=g).to(DEV)
    whole = _run(operation, x, w, merge="identity")
    for c in range(2):
        alone = _run(operation, x[:, c:c + 1].contiguous(), w[c:c + 1].contiguous(), merge="identity")
        np.testing.assert_allclose(whole[0, c].cpu().numpy(), alone[0, 0].cpu().numpy(), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------------------------------------
# test_morpho_operation.py: TestMorphologyBackward (:244-389)
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("operation", OPERATIONS)
def test_grad_deterministic(operation):
    """test_morpho_operation.py:246-277: gradcheck (float32, as there) on a 3x3 ramp image."""
    x = torch.arange(1.0, 10.0).reshape(1, 1, 3, 3).to(DEV).requires_grad_(True)
    w = (torch.arange(1.0, 10.0) / 10).reshape(1, 1, 3, 3).to(DEV)
    tol = 1e-2 if operation.startswith("S") else 1e-3
    assert torch.autograd.gradcheck(lambda a, b: _run(operation, a, b), (x, w), eps=1e-4, atol=tol, rtol=tol * 10, nondet_tol=1e-5,
                                    fast_mode=False)


GRAD_SHAPES = [
    ((1, 1, 5, 5), (1, 1, 3, 3)), ((1, 1, 7, 7), (1, 1, 5, 5)), ((1, 1, 6, 8), (1, 1, 3, 5)), ((1, 1, 8, 6), (1, 1, 5, 3)),
    ((1, 1, 7, 9), (1, 1, 3, 7)), ((1, 1, 4, 8), (1, 1, 3, 3)), ((1, 1, 8, 4), (1, 1, 3, 3)), ((1, 1, 6, 10), (1, 1, 3, 3)),
    ((2, 1, 4, 4), (1, 1, 3, 3)), ((3, 1, 5, 5), (1, 1, 3, 3)), ((2, 1, 6, 8), (1, 1, 3, 5)), ((1, 2, 6, 6), (1, 2, 3, 3)),
    ((1, 3, 5, 7), (1, 3, 3, 3)), ((1, 4, 6, 6), (1, 4, 5, 5)), ((1, 1, 6, 6), (3, 1, 3, 3)), ((1, 1, 8, 8), (4, 1, 3, 3)),
    ((1, 1, 5, 9), (2, 1, 3, 5)), ((1, 2, 6, 6), (3, 2, 3, 3)), ((1, 3, 7, 7), (2, 3, 5, 5)), ((1, 2, 8, 8), (4, 2, 5, 5)),
    ((2, 2, 5, 5), (1, 2, 3, 3)), ((3, 1, 4, 6), (2, 1, 3, 3)), ((2, 3, 6, 8), (2, 3, 3, 5)), ((1, 1, 10, 8), (1, 1, 5, 7)),
    ((1, 1, 3, 3), (1, 1, 3, 3)), ((1, 1, 4, 3), (1, 1, 3, 3)), ((1, 1, 3, 5), (1, 1, 3, 3)), ((1, 1, 12, 4), (1, 1, 3, 3)),
    ((1, 1, 4, 12), (1, 1, 3, 3)), ((1, 1, 8, 8), (1, 1, 7, 3)), ((1, 1, 8, 8), (1, 1, 3, 7)),
]


@pytest.mark.parametrize("merge", ["sum", "mean", "min", "max"])
@pytest.mark.parametrize("operation", OPERATIONS)
def test_grad_random(operation, merge):
    """test_morpho_operation.py:279-358: gradcheck in float64 over the reference's 31 shapes, inputs and
    elements spread as randn * 10 + arange (no near ties); the smooth operations with the sum and mean
    merges only, as there. The element's gradient is checked too."""
    if operation.startswith("S") and merge in ("min", "max"):
        pytest.skip(f"channel_merge_mode '{merge}' not applicable for {operation} (as in the reference)")
    torch.manual_seed(42)
    for x_shape, w_shape in GRAD_SHAPES:
        print(f"gradcheck {operation} {merge} {x_shape} {w_shape}", flush=True)
        x = torch.randn(*x_shape, dtype=torch.float64) * 10 + torch.arange(int(np.prod(x_shape)), dtype=torch.float64).reshape(x_shape)
        w = torch.randn(*w_shape, dtype=torch.float64) * 10 + torch.arange(int(np.prod(w_shape)), dtype=torch.float64).reshape(w_shape)
        x, w = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
        assert torch.autograd.gradcheck(lambda a, b: _run(operation, a, b, merge), (x, w), eps=1e-4, atol=1e-2, rtol=1e-1, nondet_tol=1e-5,
                                        fast_mode=False)


@pytest.mark.parametrize("alpha", [-1000, -10.0, -1.0, -0.5, -0.1, 0.0, 0.1, 0.5, 1.0, 10.0, 1000.0])
def test_grad_smorph(alpha):
    """test_morpho_operation.py:360-389: gradcheck of smorph in x, w and a 0-d alpha (sum merge, a 4x3
    element)."""
    g = torch.Generator().manual_seed(16)
    x = torch.randn(1, 3, 8, 6, dtype=torch.float64, generator=g).to(DEV).requires_grad_(True)
    w = torch.randn(1, 3, 4, 3, dtype=torch.float64, generator=g).to(DEV).requires_grad_(True)
    a = torch.tensor(alpha, dtype=torch.float64).to(DEV).requires_grad_(True)
    tol = 1e-2 if abs(alpha) < 1e-3 else 1e-3
    assert torch.autograd.gradcheck(lambda xx, ww, aa: F.smorph(xx, ww, aa), (x, w, a), eps=1e-4, atol=tol, rtol=tol * 10, nondet_tol=1e-5,
                                    fast_mode=False)


# ------------------------------------------------------------------------------------------------
# test_indices_opti_cuda.py: saving the winners changes nothing
# ------------------------------------------------------------------------------------------------

CASES_IDX = [("dilation", "max"), ("dilation", "min"), ("erosion", "max"), ("erosion", "min")]


def test_forward_save_indices_consistency():
    """test_indices_opti_cuda.py:6-49."""
    torch.manual_seed(42)
    for operation, merge in CASES_IDX:
        img = torch.randn(2, 4, 16, 16, device=DEV)
        weight = torch.randn(4, 4, 5, 5, device=DEV)
        fn = F.dilation if operation == "dilation" else F.erosion
        a = fn(img, weight, channel_merge_mode=merge, save_indices=False)
        b = fn(img, weight, channel_merge_mode=merge, save_indices=True)
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-6), (operation, merge)


def test_backward_save_indices_consistency():
    """test_indices_opti_cuda.py:52-121."""
    torch.manual_seed(42)
    for operation, merge in CASES_IDX:
        img = torch.randn(2, 4, 16, 16, device=DEV)
        weight = torch.randn(4, 4, 5, 5, device=DEV)
        fn = F.dilation if operation == "dilation" else F.erosion
        grads = []
        for save in (False, True):
            x = img.clone().requires_grad_(True)
            w = weight.clone().requires_grad_(True)
            fn(x, w, channel_merge_mode=merge, save_indices=save).sum().backward()
            grads.append((x.grad, w.grad))
        assert torch.allclose(grads[0][0], grads[1][0], rtol=1e-4, atol=1e-5), (operation, merge)
        assert torch.allclose(grads[0][1], grads[1][1], rtol=1e-4, atol=1e-5), (operation, merge)


# ------------------------------------------------------------------------------------------------
# test_cuda_cpu.py: the device path against the CPU extension's results (here: the oracle)
# ------------------------------------------------------------------------------------------------

def _oracle_forward(operation, x, w, merge):
    """The reference CPU extension's result for _run(operation, x, w, merge) (float32 numpy)."""
    if operation in ("dilation", "erosion"):
        op = O.DILATION if operation == "dilation" else O.EROSION
        wk = w if op == O.DILATION else np.ascontiguousarray(w[..., ::-1, ::-1])
        return O.morpho_forward(op, O.MERGES[merge], O.GEODESIC, 0.0, x, wk)[0]
    a = 1000.0 if operation == "Sdilation" else -1000.0
    alpha = np.full((w.shape[0],) if merge == "identity" else (w.shape[0], x.shape[1]), a, dtype=x.dtype)
    return O.smorph_forward(O.MERGES[merge], x, O.smorph_w_tilde(w, alpha, merge), alpha)


def _oracle_grads(operation, x, w, merge):
    """Gradients of out.sum() in x and w by the oracle (the smooth operations' w~ chained by torch on the
    CPU, as the functional layer does)."""
    g = np.ones((x.shape[0], w.shape[0]) + x.shape[2:], dtype=x.dtype)
    if operation in ("dilation", "erosion"):
        op = O.DILATION if operation == "dilation" else O.EROSION
        wk = w if op == O.DILATION else np.ascontiguousarray(w[..., ::-1, ::-1])
        gx, gw = O.morpho_backward(op, O.MERGES[merge], O.GEODESIC, 0.0, x, wk, g)
        return gx, (gw if op == O.DILATION else gw[..., ::-1, ::-1])
    a = 1000.0 if operation == "Sdilation" else -1000.0
    alpha = np.full((w.shape[0],) if merge == "identity" else (w.shape[0], x.shape[1]), a, dtype=x.dtype)
    wt = torch.from_numpy(w).requires_grad_(True)
    at = torch.from_numpy(alpha)
    tanh_a = torch.tanh(at).view(-1, 1, 1, 1) if merge == "identity" else torch.tanh(at)[..., None, None]
    w_tilde = tanh_a * ((1 - tanh_a) / 2 * wt.flip((-2, -1)) + (1 + tanh_a) / 2 * wt)
    gx, gwt, _ = O.smorph_backward(O.MERGES[merge], x, w_tilde.detach().numpy(), alpha, g)
    (gw,) = torch.autograd.grad(w_tilde, wt, torch.from_numpy(np.ascontiguousarray(gwt)))
    return gx, gw.numpy()


@pytest.mark.parametrize("merge", ["sum", "mean", "min", "max", "identity"])
@pytest.mark.parametrize("operation", OPERATIONS)
@pytest.mark.parametrize("x_shape,w_shape", [((1, 1, 4, 4), (1, 1, 3, 3)), ((2, 3, 8, 8), (2, 3, 3, 3)), ((1, 1, 5, 7), (1, 1, 3, 3))])
def test_forward_cpu_vs_cuda(x_shape, w_shape, operation, merge):
    """test_cuda_cpu.py:9-57 (rtol 1e-5, atol 1e-6)."""
    if merge == "identity" and x_shape[1] != w_shape[0]:
        pytest.skip("IDENTITY mode requires in_channels == out_channels (as in the reference)")
    if merge == "identity":
        w_shape = (w_shape[0], 1) + w_shape[2:]
    torch.manual_seed(42)
    x = torch.randn(*x_shape)
    w = torch.randn(*w_shape)
    got = _run(operation, x.to(DEV), w.to(DEV), merge).cpu()
    want = torch.from_numpy(_oracle_forward(operation, x.numpy(), w.numpy(), merge))
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("merge", ["sum", "mean", "min", "max", "identity"])
@pytest.mark.parametrize("operation", OPERATIONS)
@pytest.mark.parametrize("x_shape,w_shape", [((1, 1, 4, 4), (1, 1, 3, 3)), ((1, 1, 32, 32), (1, 1, 3, 3))])
def test_backward_cpu_vs_cuda(x_shape, w_shape, operation, merge):
    """test_cuda_cpu.py:59-149: out.sum()'s gradients (rtol 1e-4, atol 1e-6)."""
    torch.manual_seed(42)
    x = torch.randn(*x_shape)
    w = torch.randn(*w_shape)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    out = _run(operation, xd, wd, merge)
    out.sum().backward()
    torch.testing.assert_close(out.detach().cpu(), torch.from_numpy(_oracle_forward(operation, x.numpy(), w.numpy(), merge)), rtol=1e-4,
                               atol=1e-6)
    gx, gw = _oracle_grads(operation, x.numpy(), w.numpy(), merge)
    torch.testing.assert_close(xd.grad.cpu(), torch.from_numpy(np.ascontiguousarray(gx)), rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(wd.grad.cpu(), torch.from_numpy(np.ascontiguousarray(gw)), rtol=1e-4, atol=1e-6)


# ------------------------------------------------------------------------------------------------
# test_padding.py
# ------------------------------------------------------------------------------------------------

def _apply(operation, image, selem, padding, value=0.0, merge="max"):
    """test_padding.py:50-53."""
    fn = F.dilation if operation == "dilation" else F.erosion
    return fn(image, selem, channel_merge_mode=merge, padding_mode=padding, padding_value=value)


PAD_CASES = [("zero", 0.0), ("geodesic", 0.0), ("constant", 0.0), ("constant", -3.5), ("constant", 7.25), ("replicate", 0.0)]


@pytest.mark.parametrize("kernel_size", [3, 5])
@pytest.mark.parametrize("padding,value", PAD_CASES)
@pytest.mark.parametrize("operation", ["dilation", "erosion"])
def test_padding_matches_reference(operation, padding, value, kernel_size):
    """test_padding.py:54-78 (float32, 17x23, rtol = atol = 1e-5)."""
    rng = np.random.default_rng(0)
    image, kernel = rng.standard_normal((17, 23)), rng.standard_normal((kernel_size, kernel_size))
    got = _apply(operation, _f32(image)[None, None], _f32(kernel)[None, None], padding, value)
    np.testing.assert_allclose(got.squeeze().cpu().numpy(), _brute(image, kernel, operation, padding, value), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("kernel_size", [3, 5])
@pytest.mark.parametrize("padding,value", PAD_CASES)
@pytest.mark.parametrize("operation", ["dilation", "erosion"])
def test_padding_matches_reference_double(operation, padding, value, kernel_size):
    """test_padding.py:80-92 (float64, 11x9, rtol = atol = 1e-10)."""
    rng = np.random.default_rng(1)
    image, kernel = rng.standard_normal((11, 9)), rng.standard_normal((kernel_size, kernel_size))
    got = _apply(operation, torch.from_numpy(image)[None, None].to(DEV), torch.from_numpy(kernel)[None, None].to(DEV), padding, value)
    np.testing.assert_allclose(got.squeeze().cpu().numpy(), _brute(image, kernel, operation, padding, value), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("operation", ["dilation", "erosion"])
def test_zero_equals_constant_zero(operation):
    """test_padding.py:98-106."""
    torch.manual_seed(17)
    image, kernel = torch.randn(2, 3, 16, 16, device=DEV), torch.randn(4, 3, 3, 3, device=DEV)
    torch.testing.assert_close(_apply(operation, image, kernel, "zero"), _apply(operation, image, kernel, "constant", 0.0))


@pytest.mark.parametrize("operation", ["dilation", "erosion"])
def test_geodesic_never_wins(operation):
    """test_padding.py:108-118: geodesic equals a constant border far past any value."""
    torch.manual_seed(18)
    image, kernel = torch.randn(1, 1, 12, 12, device=DEV), torch.zeros(1, 1, 5, 5, device=DEV)
    unreachable = -1e9 if operation == "dilation" else 1e9
    torch.testing.assert_close(_apply(operation, image, kernel, "geodesic"), _apply(operation, image, kernel, "constant", unreachable))


@pytest.mark.parametrize("operation", ["dilation", "erosion"])
def test_constant_border_dominates(operation):
    """test_padding.py:120-132: a constant past the data takes every output touching the border."""
    torch.manual_seed(19)
    image, kernel = torch.rand(1, 1, 8, 8, device=DEV), torch.zeros(1, 1, 3, 3, device=DEV)
    extreme = 50.0 if operation == "dilation" else -50.0
    result = _apply(operation, image, kernel, "constant", extreme).squeeze()
    border = torch.ones_like(result, dtype=torch.bool)
    border[1:-1, 1:-1] = False
    assert torch.all(result[border] == extreme)
    assert torch.all(result[~border] != extreme)


@pytest.mark.parametrize("padding", ["zero", "geodesic", "constant", "replicate"])
def test_interior_is_padding_independent(padding):
    """test_padding.py:134-143."""
    torch.manual_seed(20)
    image, kernel = torch.randn(1, 1, 20, 20, device=DEV), torch.randn(1, 1, 5, 5, device=DEV)
    reference = _apply("dilation", image, kernel, "geodesic").squeeze()
    result = _apply("dilation", image, kernel, padding, 4.0).squeeze()
    torch.testing.assert_close(result[2:-2, 2:-2], reference[2:-2, 2:-2])


@pytest.mark.parametrize("merge", ["sum", "max", "min", "mean", "identity"])
@pytest.mark.parametrize("padding", ["zero", "geodesic", "constant", "replicate"])
def test_every_merge_mode_accepts_every_padding(padding, merge):
    """test_padding.py:148-160."""
    torch.manual_seed(21)
    image = torch.randn(2, 3, 12, 12, device=DEV)
    kernel = torch.randn(3, 1 if merge == "identity" else 3, 3, 3, device=DEV)
    result = _apply("dilation", image, kernel, padding, 1.5, merge=merge)
    assert result.shape == (2, 3, 12, 12)
    assert torch.isfinite(result).all()


@pytest.mark.parametrize("operation", ["dilation", "erosion"])
@pytest.mark.parametrize("padding", ["zero", "geodesic", "constant", "replicate"])
def test_backward_runs_and_reaches_the_weight(padding, operation):
    """test_padding.py:162-172."""
    torch.manual_seed(22)
    image = torch.randn(1, 2, 10, 10, device=DEV, requires_grad=True)
    kernel = torch.randn(2, 2, 3, 3, device=DEV, requires_grad=True)
    _apply(operation, image, kernel, padding, 0.5).sum().backward()
    assert image.grad is not None and torch.isfinite(image.grad).all()
    assert kernel.grad is not None and torch.isfinite(kernel.grad).all()
    assert kernel.grad.abs().sum() > 0


@pytest.mark.parametrize("padding", ["zero", "geodesic", "constant", "replicate"])
def test_kernel_larger_than_image(padding):
    """test_padding.py:174-183: a 9x9 element on a 3x3 image."""
    torch.manual_seed(23)
    result = _apply("dilation", torch.randn(1, 1, 3, 3, device=DEV), torch.zeros(1, 1, 9, 9, device=DEV), padding, 2.0)
    assert result.shape == (1, 1, 3, 3)
    assert torch.isfinite(result).all()


def test_unknown_padding_mode_is_rejected():
    """test_padding.py:185-190."""
    with pytest.raises(ValueError, match="Unknown padding mode"):
        F.dilation(torch.randn(1, 1, 8, 8, device=DEV), torch.zeros(1, 1, 3, 3, device=DEV), padding_mode="reflect")


def test_padding_value_defaults_to_zero():
    """test_padding.py:192-199."""
    torch.manual_seed(24)
    image, kernel = torch.randn(1, 1, 8, 8, device=DEV), torch.zeros(1, 1, 3, 3, device=DEV)
    torch.testing.assert_close(F.dilation(image, kernel, padding_mode="constant"), F.dilation(image, kernel, padding_mode="zero"))


@pytest.mark.parametrize("merge", ["sum", "max", "min", "mean"])
@pytest.mark.parametrize("operation", ["dilation", "erosion"])
@pytest.mark.parametrize("padding", ["zero", "geodesic", "constant", "replicate"])
def test_padding_forward_parity(padding, operation, merge):
    """test_padding.py:204-220: against the CPU extension's result (the oracle), rtol = atol = 1e-4."""
    torch.manual_seed(7)
    image, kernel = torch.randn(2, 3, 24, 24), torch.randn(4, 3, 5, 5)
    got = _apply(operation, image.to(DEV), kernel.to(DEV), padding, -2.5, merge=merge).cpu()
    op = O.DILATION if operation == "dilation" else O.EROSION
    wk = kernel.numpy() if op == O.DILATION else np.ascontiguousarray(kernel.numpy()[..., ::-1, ::-1])
    want, _ = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], -2.5, image.numpy(), wk)
    torch.testing.assert_close(got, torch.from_numpy(want), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("operation", ["dilation", "erosion"])
@pytest.mark.parametrize("padding", ["zero", "geodesic", "constant", "replicate"])
def test_padding_backward_parity(padding, operation):
    """test_padding.py:222-240: out.sum()'s gradients against the oracle, rtol = atol = 1e-4."""
    torch.manual_seed(11)
    image, kernel = torch.randn(1, 2, 16, 16), torch.randn(2, 2, 3, 3)
    x, w = image.to(DEV).requires_grad_(True), kernel.to(DEV).requires_grad_(True)
    _apply(operation, x, w, padding, -2.5).sum().backward()
    op = O.DILATION if operation == "dilation" else O.EROSION
    wk = kernel.numpy() if op == O.DILATION else np.ascontiguousarray(kernel.numpy()[..., ::-1, ::-1])
    g = np.ones((1, 2, 16, 16), dtype=np.float32)
    gx, gw = O.morpho_backward(op, O.MAX, O.PADDINGS[padding], -2.5, image.numpy(), wk, g)
    gw = gw if op == O.DILATION else gw[..., ::-1, ::-1]
    torch.testing.assert_close(x.grad.cpu(), torch.from_numpy(gx), rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(w.grad.cpu(), torch.from_numpy(np.ascontiguousarray(gw)), rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------------------------------------
# test_opening_closing_sharing.py
# ------------------------------------------------------------------------------------------------

LAYERS = [(N.Opening, "anti"), (N.Closing, "ext")]


def _trained_like(layer):
    """test_opening_closing_sharing.py:11-16: the element moved off its zero initialisation."""
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(torch.randn_like(p) * 0.5)
    return layer


def _violation_pct(y, x, sense):
    """test_opening_closing_sharing.py:19-22."""
    bad = y > x + 1e-5 if sense == "anti" else y < x - 1e-5
    return bad.float().mean().item() * 100


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_shared_by_default(cls, sense):
    """test_opening_closing_sharing.py:28-33."""
    layer = cls(3, 3, 5).to(DEV)
    assert layer.erosion.weight is layer.dilation.weight
    assert len(list(layer.parameters())) == 1
    assert tuple(layer.erosion.weight.shape) == (3, 1, 5, 5)


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_opt_out_gives_two_parameters(cls, sense):
    """test_opening_closing_sharing.py:35-38."""
    layer = cls(3, 3, 5, share_weights=False).to(DEV)
    assert layer.erosion.weight is not layer.dilation.weight
    assert len(list(layer.parameters())) == 2


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_shared_is_idempotent_and_ordered(cls, sense):
    """test_opening_closing_sharing.py:40-47: anti-extensive (opening) / extensive (closing) and
    idempotent with one element and geodesic padding."""
    torch.manual_seed(25)
    layer = _trained_like(cls(3, 3, 5, padding_mode="geodesic").to(DEV))
    x = torch.randn(2, 3, 20, 20, device=DEV)
    y = layer(x)
    assert _violation_pct(y, x, sense) == 0.0
    assert (layer(y) - y).abs().max().item() < 1e-5


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_independent_weights_lose_the_property(cls, sense):
    """test_opening_closing_sharing.py:49-55."""
    torch.manual_seed(26)
    layer = _trained_like(cls(3, 3, 5, padding_mode="geodesic", share_weights=False).to(DEV))
    x = torch.randn(2, 3, 20, 20, device=DEV)
    y = layer(x)
    assert (layer(y) - y).abs().max().item() > 1e-3


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_interior_holds_for_every_padding_mode(cls, sense):
    """test_opening_closing_sharing.py:57-65."""
    torch.manual_seed(27)
    x = torch.randn(2, 3, 24, 24, device=DEV)
    for padding in ("zero", "geodesic", "constant", "replicate"):
        layer = _trained_like(cls(3, 3, 5, padding_mode=padding).to(DEV))
        y = layer(x)
        inner = (slice(None), slice(None), slice(4, -4), slice(4, -4))
        assert _violation_pct(y[inner], x[inner], sense) == 0.0, padding


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_gradient_reaches_the_shared_weight(cls, sense):
    """test_opening_closing_sharing.py:67-72."""
    torch.manual_seed(28)
    layer = _trained_like(cls(3, 3, 5).to(DEV))
    layer(torch.randn(2, 3, 16, 16, device=DEV)).sum().backward()
    grad = layer.erosion.weight.grad
    assert grad is not None and torch.isfinite(grad).all() and grad.abs().sum() > 0


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_sharing_rejects_channel_mismatch_and_merging(cls, sense):
    """test_opening_closing_sharing.py:74-80."""
    with pytest.raises(ValueError, match="in_channels == out_channels"):
        cls(3, 8, 5)
    with pytest.raises(ValueError, match="channel_merge_mode='identity'"):
        cls(3, 3, 5, channel_merge_mode="sum")


@pytest.mark.parametrize("cls,sense", LAYERS)
def test_opt_out_still_allows_channel_mismatch(cls, sense):
    """test_opening_closing_sharing.py:82-84."""
    layer = cls(3, 8, 5, share_weights=False).to(DEV)
    assert layer(torch.randn(2, 3, 16, 16, device=DEV)).shape == (2, 8, 16, 16)


# ------------------------------------------------------------------------------------------------
# test_weight_dropout.py
# ------------------------------------------------------------------------------------------------

def _dropout_weights():
    """test_weight_dropout.py:16-21."""
    torch.manual_seed(1234)
    return torch.randn(3, 3, 3, 3, device=DEV), torch.randn(3, 1, 3, 3, device=DEV), torch.randn(3, 3, device=DEV)


def _functional_call(name, x, weights, dropout, training):
    """test_weight_dropout.py:24-31."""
    w, w_second, alpha = weights
    common = dict(weight_dropout=dropout, training=training)
    if name == "opening":
        return F.opening(x, w, w_second, **common)
    if name == "closing":
        return F.closing(x, w, w_second, **common)
    return F.sigma_layer(x, w, alpha, **common)


@pytest.mark.parametrize("name", ["opening", "closing", "sigma_layer"])
def test_dropout_inactive_outside_training(name):
    """test_weight_dropout.py:37-47."""
    torch.manual_seed(0)
    x = torch.randn(1, 3, 16, 16, device=DEV)
    weights = _dropout_weights()
    torch.manual_seed(1)
    first = _functional_call(name, x, weights, 0.5, training=False)
    torch.manual_seed(2)
    second = _functional_call(name, x, weights, 0.5, training=False)
    torch.testing.assert_close(first, second)


@pytest.mark.parametrize("name", ["opening", "closing", "sigma_layer"])
def test_dropout_active_during_training(name):
    """test_weight_dropout.py:49-60."""
    torch.manual_seed(0)
    x = torch.randn(1, 3, 16, 16, device=DEV)
    weights = _dropout_weights()
    torch.manual_seed(1)
    dropped = _functional_call(name, x, weights, 0.5, training=True)
    torch.manual_seed(1)
    plain = _functional_call(name, x, weights, 0.0, training=True)
    assert not torch.equal(dropped, plain)


@pytest.mark.parametrize("name", ["opening", "closing", "sigma_layer"])
def test_dropout_zero_probability_is_a_no_op(name):
    """test_weight_dropout.py:62-73."""
    torch.manual_seed(0)
    x = torch.randn(1, 3, 16, 16, device=DEV)
    weights = _dropout_weights()
    torch.manual_seed(1)
    training = _functional_call(name, x, weights, 0.0, training=True)
    torch.manual_seed(1)
    inference = _functional_call(name, x, weights, 0.0, training=False)
    torch.testing.assert_close(training, inference)


@pytest.mark.parametrize("cls", [N.Opening, N.Closing, N.SigmaLayer])
def test_dropout_module_follows_train_and_eval(cls):
    """test_weight_dropout.py:79-87."""
    torch.manual_seed(29)
    layer = _trained_like(cls(3, 3, 3, weight_dropout=0.5).to(DEV))
    x = torch.randn(2, 3, 16, 16, device=DEV)
    layer.eval()
    torch.testing.assert_close(layer(x), layer(x))
    layer.train()
    assert not torch.equal(layer(x), layer(x))


@pytest.mark.parametrize("cls", [N.Opening, N.Closing, N.SigmaLayer])
def test_dropout_defaults_to_disabled(cls):
    """test_weight_dropout.py:89-94."""
    torch.manual_seed(30)
    layer = _trained_like(cls(3, 3, 3).to(DEV)).train()
    x = torch.randn(2, 3, 16, 16, device=DEV)
    assert getattr(layer, "weight_dropout", 0.0) == 0.0
    torch.testing.assert_close(layer(x), layer(x))


@pytest.mark.parametrize("cls", [N.Opening, N.Closing, N.SigmaLayer])
def test_gradients_survive_dropout(cls):
    """test_weight_dropout.py:96-104 (zero padding: see the geodesic interaction below)."""
    torch.manual_seed(31)
    layer = _trained_like(cls(3, 3, 3, weight_dropout=0.3, padding_mode="zero").to(DEV)).train()
    layer(torch.randn(2, 3, 16, 16, device=DEV)).sum().backward()
    for name, p in layer.named_parameters():
        assert p.grad is not None, name
        assert torch.isfinite(p.grad).all(), name


def test_dropout_dilation_border_goes_infinite():
    """test_weight_dropout.py:115-122: one surviving tap and geodesic padding leave a border pixel with no
    finite candidate."""
    torch.manual_seed(32)
    x = torch.randn(1, 1, 8, 8, device=DEV)
    w = torch.full((1, 1, 3, 3), -float("inf"), device=DEV)
    w[0, 0, 0, 0] = 0.0
    assert torch.isinf(F.dilation(x, w, padding_mode="geodesic")).any()
    assert not torch.isinf(F.dilation(x, w, padding_mode="zero")).any()
    assert not torch.isinf(F.dilation(x, w, padding_mode="replicate")).any()


def test_dropout_sigma_layer_gradient_goes_infinite():
    """test_weight_dropout.py:124-139: the same element in sigma_layer gives a non-finite alpha gradient
    with geodesic padding (the reference's known defect, kept) and a finite one with zero padding."""
    torch.manual_seed(33)
    w = torch.full((1, 1, 3, 3), -float("inf"), device=DEV)
    w[0, 0, 0, 0] = 0.0
    x = torch.randn(1, 1, 8, 8, device=DEV)
    alpha = torch.zeros(1, 1, device=DEV, requires_grad=True)
    F.sigma_layer(x, w, alpha, padding_mode="geodesic").sum().backward()
    assert not torch.isfinite(alpha.grad).all()
    safe = torch.zeros(1, 1, device=DEV, requires_grad=True)
    F.sigma_layer(x, w, safe, padding_mode="zero").sum().backward()
    assert torch.isfinite(safe.grad).all()


# ------------------------------------------------------------------------------------------------
# test_weight_noise.py
# ------------------------------------------------------------------------------------------------

NOISE_MERGES = ["sum", "max", "min", "mean", "identity"]


def _noise_inputs(merge, dtype=torch.float32):
    """test_weight_noise.py:11-15."""
    torch.manual_seed(0)
    x = torch.randn(3, 4, 9, 11, dtype=dtype).to(DEV)
    w = torch.randn(4, 1 if merge == "identity" else 4, 3, 5, dtype=dtype).to(DEV)
    return x, w


def _draw_noise(w, batch, scale):
    """test_weight_noise.py:18-21: one weight-shaped draw in [-s, s] per batch element."""
    return (torch.rand((batch,) + tuple(w.shape), dtype=w.dtype, device=w.device) * 2.0 - 1.0) * scale


def _per_sample(op, x, w, noise, merge, save):
    """test_weight_noise.py:24-34: every batch element alone with its own noisy weight (the erosion's
    noise is added to the flipped weight)."""
    outs = []
    for b in range(x.shape[0]):
        if op == "dilation":
            outs.append(F.dilation(x[b:b + 1], w + noise[b], merge, save_indices=save))
        else:
            outs.append(F.erosion(x[b:b + 1], (w.flip((-2, -1)) + noise[b]).flip((-2, -1)), merge, save_indices=save))
    return torch.cat(outs)


@pytest.mark.parametrize("save", [True, False])
@pytest.mark.parametrize("merge", NOISE_MERGES)
@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_noise_matches_per_sample_reference(op, merge, save):
    """test_weight_noise.py:42-60."""
    x, w = _noise_inputs(merge)
    x.requires_grad_(True)
    w.requires_grad_(True)
    fn = F.dilation if op == "dilation" else F.erosion
    torch.manual_seed(7)
    out = fn(x, w, merge, save_indices=save, training=True, noise_scale=0.3)
    grad = torch.randn_like(out)
    gx, gw = torch.autograd.grad(out, (x, w), grad)
    torch.manual_seed(7)
    noise = _draw_noise(w.detach(), x.shape[0], 0.3)
    expected = _per_sample(op, x, w, noise, merge, save)
    egx, egw = torch.autograd.grad(expected, (x, w), grad)
    torch.testing.assert_close(out, expected)
    torch.testing.assert_close(gx, egx)
    torch.testing.assert_close(gw, egw)


@pytest.mark.parametrize("save", [True, False])
@pytest.mark.parametrize("merge", NOISE_MERGES)
@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_noise_gradcheck(op, merge, save):
    """test_weight_noise.py:62-74: the same noise on every evaluation (reseeded), geodesic padding."""
    x, w = _noise_inputs(merge, torch.float64)
    x = x[:2, :, :5, :6].clone().requires_grad_(True)
    w = w[..., :3].clone().requires_grad_(True)
    fn = F.dilation if op == "dilation" else F.erosion

    def noisy(a, b):
        torch.manual_seed(3)
        return fn(a, b, merge, "geodesic", save, training=True, noise_scale=0.5)

    assert torch.autograd.gradcheck(noisy, (x, w))


@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_noise_varies_per_sample(op):
    """test_weight_noise.py:77-89."""
    x, w = _noise_inputs("sum")
    x = x[:1].expand(4, -1, -1, -1).contiguous()
    fn = F.dilation if op == "dilation" else F.erosion
    out = fn(x, w, training=True, noise_scale=0.5)
    assert not torch.equal(out[0], out[1])
    assert (out - fn(x[:1], w)).abs().max() <= 4 * 0.5 + 1e-5


@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_noise_inactive_outside_training(op):
    """test_weight_noise.py:92-97."""
    x, w = _noise_inputs("sum")
    fn = F.dilation if op == "dilation" else F.erosion
    torch.testing.assert_close(fn(x, w, training=False, noise_scale=0.5), fn(x, w))


def test_noise_rejects_negative_scale():
    """test_weight_noise.py:100-103."""
    x, w = _noise_inputs("sum")
    with pytest.raises(RuntimeError, match="noise_scale"):
        F.dilation(x, w, training=True, noise_scale=-0.1)


@pytest.mark.parametrize("layer", [
    lambda: N.Dilation(3, 3, 3, noise_scale=0.5),
    lambda: N.Erosion(3, 3, 3, noise_scale=0.5),
    lambda: N.Opening(3, 3, 3, noise_scale=0.5),
    lambda: N.Closing(3, 3, 3, noise_scale=0.5),
    lambda: N.SigmaLayer(3, 3, 3, noise_scale=0.5),
], ids=["Dilation", "Erosion", "Opening", "Closing", "SigmaLayer"])
def test_noise_layers_follow_training_mode(layer):
    """test_weight_noise.py:106-125."""
    torch.manual_seed(0)
    module = layer().to(DEV)
    x = torch.randn(2, 3, 12, 12).to(DEV)
    module.eval()
    torch.testing.assert_close(module(x), module(x))
    module.train()
    torch.manual_seed(1)
    first = module(x)
    torch.manual_seed(2)
    second = module(x)
    assert not torch.equal(first, second)
    first.sum().backward()
