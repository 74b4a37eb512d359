"""Empty and channel-less inputs through every operator, forward and backward, on the GPU.

An empty batch, image height or width leaves an empty output: every gradient is then zero (the
element's, alpha's and beta's) or empty. No output channel leaves an empty output and a zero input
gradient. No input channel (merges other than 'identity', whose channel counts are equal) leaves every
output at the merge's start value, as the reference's merge over no channel (morpho_merge_policy.hpp:
10-86): lowest() for 'max', max() for 'min', 0 for 'sum' and 0 / 0 for 'mean' (the oracle's values),
with empty input and element gradients; smorph_scm refuses it. None of these launches a kernel that
reads the missing data, and none of the size queries divides by an empty dimension."""
import numpy as np
import pytest
import torch

import morphocore_amd as mca
from oracle import oracle as O

pytestmark = pytest.mark.gpu

F = mca.functional
DEV = "cuda"
MERGES = ["max", "min", "sum", "mean", "identity"]
# (B, Cin, Cout, H, W): an empty batch, height, width; no input channel; no output channel.
SHAPES = {"batch": (0, 2, 3, 6, 9), "height": (2, 2, 3, 0, 9), "width": (2, 2, 3, 6, 0), "no_input_channel": (2, 0, 3, 6, 9),
          "no_output_channel": (2, 2, 0, 6, 9)}


def _shape(kind, merge):
    B, Cin, Cout, H, W = SHAPES[kind]
    if merge == "identity":
        Cout = Cin = 0 if kind in ("no_input_channel", "no_output_channel") else Cin
    return B, Cin, Cout, H, W


def _check_grads(kind, x, w, out, others=()):
    out.sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape and not x.grad.any()
    assert w.grad is not None and w.grad.shape == w.shape and not w.grad.any()
    for t in others:
        assert t.grad is not None and t.grad.shape == t.shape and not t.grad.any()


def _expected_channelless(merge, op, B, Cout, H, W, dtype):
    nt = np.float64 if dtype == torch.float64 else np.float32  # 16-bit: the float32 values, rounded once
    x = np.zeros((B, 0, H, W), dtype=nt)
    w = np.zeros((Cout, 0, 3, 3), dtype=nt)
    ref, _ = O.morpho_forward(op, O.MERGES[merge], O.GEODESIC, 0.0, x, w)
    return torch.from_numpy(ref).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("kind", list(SHAPES))
@pytest.mark.parametrize("op", ["dilation", "erosion"])
def test_dilation_erosion_empty(op, kind, merge, dtype):
    B, Cin, Cout, H, W = _shape(kind, merge)
    print(f"empty {op} {kind} {merge} {dtype} {(B, Cin, Cout, H, W)}", flush=True)
    x = torch.randn(B, Cin, H, W, dtype=dtype, device=DEV).requires_grad_(True)
    w = torch.randn(Cout, 1 if merge == "identity" else Cin, 3, 3, dtype=dtype, device=DEV).requires_grad_(True)
    fn = F.dilation if op == "dilation" else F.erosion
    for save in (True, False):
        x.grad = w.grad = None
        out = fn(x, w, merge, "geodesic", save_indices=save)
        assert out.shape == (B, Cout, H, W) and out.dtype == dtype
        if out.numel() > 0:
            want = _expected_channelless(merge, O.DILATION if op == "dilation" else O.EROSION, B, Cout, H, W, dtype)
            assert torch.equal(out.detach().cpu().isnan(), want.isnan())
            assert torch.equal(out.detach().cpu().nan_to_num(), want.nan_to_num())
        _check_grads(kind, x, w, out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("kind", list(SHAPES))
def test_smorph_empty(kind, merge, dtype):
    B, Cin, Cout, H, W = _shape(kind, merge)
    print(f"empty smorph {kind} {merge} {dtype} {(B, Cin, Cout, H, W)}", flush=True)
    x = torch.randn(B, Cin, H, W, dtype=dtype, device=DEV).requires_grad_(True)
    w = torch.randn(Cout, 1 if merge == "identity" else Cin, 3, 3, dtype=dtype, device=DEV).requires_grad_(True)
    a = torch.full((Cout,) if merge == "identity" else (Cout, Cin), 2.0, dtype=dtype, device=DEV).requires_grad_(True)
    out = F.smorph(x, w, a, channel_merge_mode=merge)
    assert out.shape == (B, Cout, H, W)
    if out.numel() > 0:
        nt = np.float64 if dtype == torch.float64 else np.float32
        ref = O.smorph_forward(O.MERGES[merge], np.zeros((B, 0, H, W), nt), np.zeros((Cout, 0, 3, 3), nt), np.zeros((Cout, 0), nt))
        want = torch.from_numpy(ref).to(dtype)
        assert torch.equal(out.detach().cpu().isnan(), want.isnan())
        assert torch.equal(out.detach().cpu().nan_to_num(), want.nan_to_num())
    _check_grads(kind, x, w, out, (a,))


@pytest.mark.parametrize("kind", ["batch", "height", "width", "no_output_channel"])
def test_smorph_scm_empty(kind):
    B, Cin, Cout, H, W = SHAPES[kind]
    print(f"empty smorph_scm {kind}", flush=True)
    x = torch.randn(B, Cin, H, W, device=DEV).requires_grad_(True)
    w = torch.randn(Cout, Cin, 3, 3, device=DEV).requires_grad_(True)
    a = torch.full((Cout, Cin), 2.0, device=DEV).requires_grad_(True)
    beta = torch.full((Cout,), 1.5, device=DEV).requires_grad_(True)
    out = F.smorph(x, w, a, beta)
    assert out.shape == (B, Cout, H, W)
    _check_grads(kind, x, w, out, (a, beta))


def test_smorph_scm_refuses_no_input_channel():
    x = torch.randn(2, 0, 6, 9, device=DEV)
    with pytest.raises(RuntimeError, match="at least one input channel"):
        F.smorph(x, torch.randn(3, 0, 3, 3, device=DEV), torch.ones(3, 0, device=DEV), torch.ones(3, device=DEV))


@pytest.mark.parametrize("kind", ["batch", "height", "width", "no_input_channel"])
@pytest.mark.parametrize("name", ["opening", "closing", "sigma_layer"])
def test_compositions_empty(name, kind):
    B, C, _, H, W = SHAPES[kind]
    print(f"empty {name} {kind}", flush=True)
    x = torch.randn(B, C, H, W, device=DEV).requires_grad_(True)
    w1 = torch.randn(C, 1, 3, 3, device=DEV).requires_grad_(True)
    if name == "sigma_layer":
        alpha = torch.zeros(C, 1, device=DEV, requires_grad=True)
        out = F.sigma_layer(x, w1, alpha, "identity", "geodesic")
        others = (alpha,)
    else:
        w2 = torch.randn(C, 1, 3, 3, device=DEV).requires_grad_(True)
        out = getattr(F, name)(x, w1, w2, "identity", "geodesic")
        others = (w2,)
    assert out.shape == (B, C, H, W)
    out.sum().backward()
    assert x.grad.shape == x.shape and not x.grad.any()
    for t in (w1,) + others:
        assert t.grad is not None and t.grad.shape == t.shape
        # sigma_layer's alpha gradient over an empty output is 0; the elements' too.
        assert not t.grad.any()
