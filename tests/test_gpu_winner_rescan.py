"""The max / min forward's winner rescan sorted by channel (float32 and 16-bit static kernels of 5x5 and
larger, launches of at least 1024 workgroups, up to 256 input channels), against the oracle bit for bit:
values (sign of zero included) and packed (channel << 16 | tap) winners.

The smaller parity cases take the small-grid launch shape, which rescans each pixel from global memory;
these shapes take the full one: 4 rows per wave, 4 (or, under 4 output channels, 1) output channels
per workgroup, ragged last tiles in both directions and a partial last channel group. Inputs stress the
tie rules (morpho_merge_policy.hpp:10-86, morpho_op_cpu_kernels.hxx:202-296): quantised values with
ties between taps and between channels, signed zeros, NaN and infinities; and 256 (the largest count
the sort takes) and 257 input channels (the per-pixel rescan), compared on a corner of the image."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

PADDINGS = ["zero", "geodesic", "constant", "replicate"]


def _forward(op, merge, padding, pv, x, w):
    """One call of the C ABI forward with saved winners (any dtype); values returned as float32 (exact for
    the 16-bit types) and winners."""
    from morphocore_amd import _native

    dev = torch.device("cuda")
    xd, wd = x.to(dev).contiguous(), w.to(dev).contiguous()
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w.shape
    out = torch.empty((B, Cout, H, W), dtype=x.dtype, device=dev)
    idx = torch.empty((B, Cout, H, W), dtype=torch.int32, device=dev)
    fill = O.fill_value(op, O.PADDINGS[padding], pv, np.float64 if x.dtype == torch.float64 else np.float32)
    _native.morpho_forward(op, O.MERGES[merge], padding == "replicate", fill, xd, wd, 0, out, idx, (B, Cin, Cout, Cw, H, W, KH, KW))
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), idx.cpu().numpy()


def _inputs(kind, B, Cin, Cout, H, W, K, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "quant":
        x = torch.randint(0, 8, (B, Cin, H, W), generator=g).float() / 8
        w = torch.randint(-1, 2, (Cout, Cin, K, K), generator=g).float() / 8
    elif kind == "zeros":
        x = torch.where(torch.rand(B, Cin, H, W, generator=g) < 0.5, -0.0, 0.0)
        w = torch.where(torch.rand(Cout, Cin, K, K, generator=g) < 0.5, -0.0, 0.0)
    else:  # "special": N(0, 1) with NaN, +inf and -inf scattered in
        x = torch.randn(B, Cin, H, W, generator=g)
        u = torch.rand(B, Cin, H, W, generator=g)
        x = torch.where(u < 0.002, float("nan"), torch.where(u > 0.999, float("inf"), torch.where((u > 0.5) & (u < 0.501), float("-inf"), x)))
        w = torch.randn(Cout, Cin, K, K, generator=g) * 0.3
    return x, w


def _check(op, merge, padding, pv, x, w, dtype, region=None):
    """Product forward (full image) against the oracle (on the image, or on `region` = (rows, cols): a
    top-left corner whose outputs read no input beyond it): values bit for bit in float32 (NaN against
    NaN), winners exactly."""
    xs, ws = x.to(dtype), w.to(dtype)
    out, idx = _forward(op, merge, padding, pv, xs, ws)
    xo, wo = xs.float().numpy(), ws.float().numpy()  # 16-bit values are exact in float32
    if region is not None:
        xo = np.ascontiguousarray(xo[:, :, :region[0], :region[1]])
    ref, ridx = O.morpho_forward(op, O.MERGES[merge], O.PADDINGS[padding], pv, xo, wo, save_indices=True)
    ref = torch.from_numpy(ref).to(dtype).float().numpy()  # one rounding to the stored type
    if region is not None:
        K = w.shape[-1]
        r, c = region[0] - K // 2, region[1] - K // 2
        out, idx, ref, ridx = out[:, :, :r, :c], idx[:, :, :r, :c], ref[:, :, :r, :c], ridx[:, :, :r, :c]
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(out)), "NaN positions differ"
    assert np.array_equal(np.ascontiguousarray(out).view(np.int32)[~nan], np.ascontiguousarray(ref).view(np.int32)[~nan]), "values differ"
    assert np.array_equal(idx, ridx), f"winners differ at {np.argwhere(idx != ridx)[:5].tolist()}"


@pytest.mark.parametrize("kind", ["quant", "zeros", "special"])
@pytest.mark.parametrize("K", [5, 7, 11])
@pytest.mark.parametrize("merge", ["max", "min"])
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_rescan_full_launch(op, merge, K, kind):
    """4 x 3 -> 6 channels on 250 x 600 planes: 1280 workgroups of 4 output channels, the second group
    half empty, ragged last row and column tiles."""
    padding = PADDINGS[(K + op + (merge == "min")) % 4]
    print(f"rescan op {op} {merge} {K}x{K} {kind} {padding}", flush=True)
    x, w = _inputs(kind, 4, 3, 6, 250, 600, K, 1000 + K)
    _check(op, merge, padding, -0.25, x, w, torch.float32)


@pytest.mark.parametrize("K", [5, 11])
@pytest.mark.parametrize("merge", ["max", "min"])
def test_rescan_one_channel_groups(merge, K):
    """3 output channels (one per workgroup, 4 rows per wave: 4 items per thread)."""
    print(f"rescan 3 output channels {merge} {K}x{K}", flush=True)
    x, w = _inputs("quant", 4, 3, 3, 250, 600, K, 2000 + K)
    _check(O.DILATION, merge, "replicate", 0.0, x, w, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("merge", ["max", "min"])
def test_rescan_16bit(dtype, merge):
    print(f"rescan {dtype} {merge}", flush=True)
    x, w = _inputs("quant", 4, 3, 6, 250, 600, 7, 3000)
    _check(O.EROSION, merge, "zero", 0.0, x, w, dtype)


@pytest.mark.parametrize("Cin", [256, 257])
@pytest.mark.parametrize("merge", ["max", "min"])
def test_rescan_channel_limit(Cin, merge):
    """256 input channels sort their winners (ties between many channels), 257 rescan per pixel; the
    oracle runs on the top-left 40 x 100 corner."""
    print(f"rescan Cin {Cin} {merge}", flush=True)
    x, w = _inputs("quant", 1, Cin, 4, 512, 2048, 5, 4000 + Cin)
    _check(O.DILATION, merge, "geodesic", 0.0, x, w, torch.float32, region=(40, 100))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", ["dilation min +inf", "erosion max -inf", "dilation max -inf", "erosion min +inf"])
def test_rescan_infinite_border(case, dtype):
    """An infinite constant border at the full launch shape. Beyond the merge's clamp (a 'min' of
    dilations reading +inf, a 'max' of erosions reading -inf), every channel's extremum is that infinity,
    the merge stays at max() / lowest() and channel 0 wins with its first tap reading the border. At the
    op's start value (the inputs all -inf / +inf with NaN among them), no tap improves on it and the
    winner is channel 0, tap 0, whatever the NaN taps."""
    name, merge, pv = case.split()
    op = O.DILATION if name == "dilation" else O.EROSION
    print(f"rescan infinite border {case} {dtype}", flush=True)
    x, w = _inputs("special", 4, 3, 6, 250, 600, 5, 5000)
    if (name, merge) in (("dilation", "max"), ("erosion", "min")):
        g = torch.Generator().manual_seed(5001)
        x = torch.where(torch.rand(x.shape, generator=g) < 0.3, float("nan"), float(pv))
    _check(op, merge, "constant", float(pv), x, w, dtype)
