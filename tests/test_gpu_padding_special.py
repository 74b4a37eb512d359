"""Constant padding with special border values (NaN, +-inf, -0.0, +-FLT_MAX), every merge, against the
oracle: forward values bit for bit (NaN positions equal), max / min winners exactly, gradients within the
contract. A NaN border never wins a tap (the strict scan of morpho_op_cpu_kernels.hxx:202-296), an
infinite one wins every tap that reads it (and routes no gradient to the input, as any out-of-image
tap, morpho_op_cpu_backward.hxx:39-156); small planes make most taps read the border."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded
from tests.test_gpu_parity import kernel_forward

pytestmark = pytest.mark.gpu

VALUES = [float("nan"), float("inf"), float("-inf"), -0.0, 3.4e38, -3.4e38]


@pytest.mark.parametrize("value", VALUES, ids=[str(v) for v in VALUES])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("merge", ["max", "min", "sum", "mean", "identity"])
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_constant_padding_special_values(op, merge, dtype, value):
    import morphocore_amd  # noqa: F401

    B, Cin, Cout, H, W, K = 2, 3, 4, 5, 7, 5
    if merge == "identity":
        Cout = Cin
    print(f"padding {value} op {op} {merge} {dtype}", flush=True)
    x = seeded(951, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(952, Cout, 1 if merge == "identity" else Cin, K, K, dtype=dtype, kind="randn", scale=0.3)
    g = seeded(953, B, Cout, H, W, dtype=dtype, kind="randn")
    ref, ridx = O.morpho_forward(op, O.MERGES[merge], O.CONSTANT, value, x.numpy(), w.numpy(), save_indices=merge in ("max", "min"))
    out, idx = kernel_forward(op, merge, "constant", value, x, w, save=merge in ("max", "min"))
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    nan = np.isnan(ref)
    assert np.array_equal(out[~nan].view(np.int64 if dtype == torch.float64 else np.int32),
                          ref[~nan].view(np.int64 if dtype == torch.float64 else np.int32)), "forward differs"
    if ridx is not None:
        assert np.array_equal(idx, ridx), "winners differ"
    # Gradients through the operator (the op-level element: erosion callers pass it flipped).
    dev = torch.device("cuda")
    xd, wd = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    fn = torch.ops.morphocore.dilation if op == O.DILATION else torch.ops.morphocore.erosion
    o = fn(xd, wd, O.MERGES[merge], O.CONSTANT, value, True, 0.0)
    o.backward(g.to(dev))
    gx, gw = O.morpho_backward(op, O.MERGES[merge], O.CONSTANT, value, x.numpy(), w.numpy(), g.numpy())
    assert normwise_error(xd.grad.cpu().numpy(), gx) <= TOL[dtype]
    assert normwise_error(wd.grad.cpu().numpy(), gw) <= TOL[dtype]
