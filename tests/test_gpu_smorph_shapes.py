"""Smorph parity on the GPU for the elements the static float32 kernels do not cover: rectangular,
even and one-row elements (pad = K // 2 on each axis, so asymmetric windows), float64 at 7x7 and
11x11, and NaN inputs through the generic kernels (float64, 9x9 and 3x5 float32). Every merge,
alpha of both signs and zero; the oracle is the checker (reference smorph_cpu_kernels.hxx:30-147 for
the window bounds)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded
from tests.test_gpu_parity import MERGES, _smorph_case, _weight_shape

pytestmark = pytest.mark.gpu


def _alpha(merge, Cin, Cout, a, dtype, seed):
    pairs = Cout if merge == "identity" else Cout * Cin
    alpha = torch.full((pairs,), a, dtype=dtype) + seeded(seed, pairs, dtype=dtype, kind="randn", scale=0.1 if a != 0 else 0.0)
    return alpha.reshape((Cout,) if merge == "identity" else (Cout, Cin))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("a", [-20.0, 0.0, 20.0])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("KH,KW", [(3, 5), (5, 3), (4, 2), (1, 5)])
def test_smorph_rectangular_and_even_elements(KH, KW, merge, a, dtype):
    B, Cin, Cout, H, W = 2, 3, 4, 18, 70
    if merge == "identity":
        Cout = Cin
    print(f"smorph {KH}x{KW} {merge} alpha={a} {dtype}", flush=True)
    x = seeded(81, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(82, *_weight_shape(merge, Cin, Cout, KH, KW), dtype=dtype, kind="randn", scale=0.1)
    g = seeded(83, B, Cout, H, W, dtype=dtype, kind="randn")
    for actual, expected in _smorph_case(merge, x, w, _alpha(merge, Cin, Cout, a, dtype, 84), g):
        assert normwise_error(actual, expected) <= TOL[dtype]


@pytest.mark.parametrize("a", [-20.0, 1.0, 20.0])
@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("K", [7, 11])
def test_smorph_float64_large_elements(K, merge, a):
    B, Cin, Cout, H, W = 1, 2, 3, 21, 75
    if merge == "identity":
        Cout = Cin
    print(f"smorph f64 {K}x{K} {merge} alpha={a}", flush=True)
    x = seeded(85, B, Cin, H, W, dtype=torch.float64, kind="randn")
    w = seeded(86, *_weight_shape(merge, Cin, Cout, K, K), dtype=torch.float64, kind="randn", scale=0.1)
    g = seeded(87, B, Cout, H, W, dtype=torch.float64, kind="randn")
    for actual, expected in _smorph_case(merge, x, w, _alpha(merge, Cin, Cout, a, torch.float64, 88), g):
        assert normwise_error(actual, expected) <= TOL[torch.float64]


@pytest.mark.parametrize("merge", ["sum", "max", "identity"])
@pytest.mark.parametrize("dtype,KH,KW", [(torch.float64, 3, 3), (torch.float64, 7, 7), (torch.float32, 9, 9), (torch.float32, 3, 5)])
def test_smorph_generic_nan_input(dtype, KH, KW, merge):
    """An in-image NaN propagates through the generic kernels as through the reference: its pairs'
    outputs and routed gradients are NaN (a NaN never wins the window's extremum, nor the MAX merge);
    out-of-image taps are excluded by position, not by value. Same NaN positions as the oracle, every
    finite value within the tolerance."""
    B, Cin, Cout, H, W = 1, 2, 3, 20, 100
    if merge == "identity":
        Cout = Cin
    x = seeded(89, B, Cin, H, W, dtype=dtype, kind="randn")
    x[0, 0, 9, 50] = float("nan")
    x[0, 1, 0, 2] = float("nan")
    w = seeded(90, *_weight_shape(merge, Cin, Cout, KH, KW), dtype=dtype, kind="randn", scale=0.1)
    pairs = Cout if merge == "identity" else Cout * Cin
    alpha = torch.where(torch.arange(pairs) % 2 == 0, 2.0, -3.0).to(dtype)
    alpha = alpha.reshape((Cout,) if merge == "identity" else (Cout, Cin))
    g = seeded(91, B, Cout, H, W, dtype=dtype, kind="randn")
    results = _smorph_case(merge, x, w, alpha, g)
    assert np.isnan(results[0][1]).any() == (merge != "max")
    for actual, expected in results:
        assert normwise_error(actual, expected) <= TOL[dtype]


@pytest.mark.parametrize("merge", MERGES)
@pytest.mark.parametrize("K", [3, 5, 7, 11])
def test_smorph_static_forward_bit_exact(K, merge):
    """The float32 static forward equals the oracle bit for bit, on interior and border tiles, for
    pairs whose window passes the bound that drops the exponential's underflow select (small |alpha|,
    alpha = 0) and pairs that keep it (|alpha| = 20 on N(0, 1) data, a NaN-free input with -87 below
    the bound), and an input with +inf (never on the select-free path)."""
    B, Cin, Cout, H, W = 1, 3, 2, 22, 200
    if merge == "identity":
        Cout = Cin
    x = seeded(141, B, Cin, H, W, kind="randn")
    w = seeded(142, *_weight_shape(merge, Cin, Cout, K, K), kind="randn", scale=0.1)
    pairs = Cout if merge == "identity" else Cout * Cin
    for alphas in ([0.0, 0.7, -2.0, 3.0, 20.0, -20.0], [20.0, -20.0, 0.5, 0.0, -0.5, 9.0]):
        alpha = torch.tensor([alphas[p % len(alphas)] for p in range(pairs)]).reshape((Cout,) if merge == "identity" else (Cout, Cin))
        for xin in (x, torch.where(torch.arange(W) == 130, torch.tensor(float("inf")), x)):
            import morphocore_amd  # noqa: F401

            with torch.no_grad():
                out = torch.ops.morphocore.smorph(xin.cuda(), w.cuda(), alpha.cuda(), O.MERGES[merge]).cpu().numpy()
            ref = O.smorph_forward(O.MERGES[merge], xin.numpy(), w.numpy(), alpha.numpy())
            assert np.array_equal(out, ref, equal_nan=True), (alphas, float(np.nanmax(np.abs(out - ref))))


@pytest.mark.parametrize("merge", ["mean", "max", "identity"])
@pytest.mark.parametrize("dtype,K,shape", [(torch.float32, 31, (2, 3, 4, 40, 70)), (torch.float64, 31, (2, 3, 4, 40, 70)),
                                           (torch.float64, 41, (1, 2, 3, 30, 70)), (torch.float32, 101, (1, 2, 2, 24, 30))],
                         ids=["f32-31", "f64-31", "f64-41", "f32-101"])
def test_smorph_large_elements(dtype, K, shape, merge):
    """Elements whose default tile, its grad_input copy and bins exceed the LDS budget train as in the
    reference's CPU path, which takes any size (smorph_cpu_kernels.hxx:30-147,387-638): the backward
    takes one row per wave, then the device's whole LDS, then grad_input summed in global memory
    (31x31, 41x41 and 101x101 land on these in turn), with a non-zero workspace; forward and every
    gradient against the oracle."""
    from morphocore_amd import _native

    B, Cin, Cout, H, W = shape
    if merge == "identity":
        Cout = Cin
    print(f"smorph {K}x{K} {merge} {dtype} (device LDS per workgroup: "
          f"{torch.cuda.get_device_properties(0).shared_memory_per_block} bytes)", flush=True)
    x = seeded(150, B, Cin, H, W, dtype=dtype, kind="randn")
    w = seeded(151, *_weight_shape(merge, Cin, Cout, K, K), dtype=dtype, kind="randn", scale=0.1)
    g = seeded(152, B, Cout, H, W, dtype=dtype, kind="randn")
    size = getattr(_native.lib(), f"mca_smorph_backward_workspace_size_{'f32' if dtype == torch.float32 else 'f64'}")
    assert size(O.MERGES[merge], B, Cin, Cout, w.shape[1], H, W, K, K) > 0
    for actual, expected in _smorph_case(merge, x, w, _alpha(merge, Cin, Cout, 3.0, dtype, 153), g):
        assert normwise_error(actual, expected) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_smorph_scm_large_element(dtype):
    """The SMOOTH merge (smorph_scm) with a 31x31 element: forward and every gradient against the oracle."""
    from tests.test_gpu_scm import _check

    B, C, H, W, K = 1, 3, 36, 70, 31
    print(f"smorph_scm {K}x{K} {dtype}", flush=True)
    x = seeded(154, B, C, H, W, dtype=dtype, kind="randn")
    w = seeded(155, C, C, K, K, dtype=dtype, kind="randn", scale=0.1)
    alpha = _alpha("sum", C, C, 2.0, dtype, 156)
    beta = torch.tensor([1.5, -2.0, 0.0], dtype=dtype)
    g = seeded(157, B, C, H, W, dtype=dtype, kind="randn")
    _check(x, w, alpha, beta, g)
