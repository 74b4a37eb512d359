"""The streaming row-band kernels of the IDENTITY merge (3x3 and 5x5 elements, planes whose width is a
multiple of 8: configs[3]'s layer), against the oracle and the numpy brute force of the strict first-tap
scan (reference morpho_op_cpu_kernels.hxx:254-263), and against the tiled kernels they replace (which
still run for buffers that are not 16-byte aligned, taken here from a one-element offset):

* forward values (and the sign of zero results) and the saved first extremal taps bit for bit, every
  padding, dilation and erosion, float32 / float64, bands cut short by the image's last rows, images
  shorter than the element, NaN / +-inf / signed-zero inputs;
* grad_input bit for bit against the tiled gather (the same sums in the same tap order) and within
  the contract against the oracle; grad_weight within the contract (its per-band partial slots add in
  another order); the 16-bit gradients (float32 routing) likewise.
Each case prints its name before the GPU work."""
import numpy as np
import pytest
import torch

from morphocore_amd import _native
from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu

IDENT = 5
PADDINGS = ["zero", "geodesic", "constant", "replicate"]
PV = -0.375
# B, C, H, W: a ragged last band, one 16-row band, a plane shorter than the element, one row.
SHAPES = [(2, 3, 37, 8), (1, 2, 16, 112), (1, 1, 3, 264), (2, 2, 1, 16)]


def _np(t):
    return t.detach().cpu().numpy()


def _first_taps(op, padding, x, w):
    """The strict first-tap scan (kh, then kw) of every pixel in numpy: the first tap reaching the
    extremum, tap 0 when none improves on the start value."""
    B, C, H, W = x.shape
    KH, KW = w.shape[-2:]
    ph, pw = KH // 2, KW // 2
    fill = O.fill_value(op, O.PADDINGS[padding], PV, x.dtype)
    ys, xs = np.arange(H)[:, None], np.arange(W)[None, :]
    best = np.full(x.shape, -np.inf if op == O.DILATION else np.inf, dtype=x.dtype)
    arg = np.zeros(x.shape, dtype=np.int64)
    for kh in range(KH):
        for kw in range(KW):
            yy, xx = ys + ph - kh, xs + pw - kw
            inb = (yy >= 0) & (yy < H) & (xx >= 0) & (xx < W)
            v = x[:, :, np.clip(yy, 0, H - 1), np.clip(xx, 0, W - 1)]
            if padding != "replicate":
                v = np.where(inb, v, x.dtype.type(fill))
            wv = w[None, :, 0, kh, kw, None, None]
            v = v + wv if op == O.DILATION else v - wv
            better = v > best if op == O.DILATION else v < best
            best = np.where(better, v, best)
            arg = np.where(better, kh * KW + kw, arg)
    return best, arg


def _dev(t, offset):
    """t on the GPU; offset 1: at a one-element offset in a larger buffer (not 16-byte aligned)."""
    if not offset:
        return t.cuda().contiguous()
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device="cuda")
    v = buf[1:].view(t.shape)
    v.copy_(t.cuda())
    return v


def _forward(op, padding, x, w, offset):
    B, C, H, W = x.shape
    K = w.shape[-1]
    xd, wd = _dev(x, offset), w.cuda()
    out = _dev(torch.empty_like(x), offset)
    taps = torch.empty((B, C, H, W), dtype=torch.uint8, device="cuda")
    fill = O.fill_value(op, O.PADDINGS[padding], PV, x.numpy().dtype)
    _native.morpho_forward(op, IDENT, padding == "replicate", fill, xd, wd, 0, out, taps, (B, C, C, 1, H, W, K, K))
    torch.cuda.synchronize()
    return _np(out), _np(taps)


def _backward(op, x, w, taps, g, offset, tensors=False):
    """The backward from the saved taps (which reads neither x nor w: they only give the dtype)."""
    B, C, H, W = g.shape
    K = w.shape[-1]
    gd = _dev(g, offset)
    gx = _dev(torch.empty_like(g), offset)
    gw = torch.empty((C, 1, K, K), dtype=g.dtype, device="cuda")
    _native.morpho_backward(op, IDENT, True, 0.0, x.cuda(), w.cuda(), 0, torch.as_tensor(taps).cuda(), gd, gx, gw, (B, C, C, 1, H, W, K, K))
    torch.cuda.synchronize()
    return (gx.cpu(), gw.cpu()) if tensors else (_np(gx), _np(gw))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("K", [3, 5])
@pytest.mark.parametrize("padding", PADDINGS)
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_band_forward_and_taps(op, padding, K, dtype):
    for si, (B, C, H, W) in enumerate(SHAPES):
        print(f"band forward op={op} {padding} {K}x{K} {dtype} shape {(B, C, H, W)}", flush=True)
        x = seeded(300 + si, B, C, H, W, dtype=dtype, kind="randn")
        w = seeded(310 + si, C, 1, K, K, dtype=dtype, kind="randn", scale=0.3)
        out, taps = _forward(op, padding, x, w, 0)
        ref, _ = O.morpho_forward(op, IDENT, O.PADDINGS[padding], PV, x.numpy(), w.numpy())
        assert np.array_equal(out, ref) and np.array_equal(np.signbit(out), np.signbit(ref)), si
        _, want_taps = _first_taps(op, padding, x.numpy(), w.numpy())
        assert np.array_equal(taps, want_taps), si
        out_t, taps_t = _forward(op, padding, x, w, 1)
        assert np.array_equal(out_t, out) and np.array_equal(np.signbit(out_t), np.signbit(out)) and np.array_equal(taps_t, taps), si


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_band_forward_special_values(op, dtype):
    """Ties on a zero element with signed zeros (the first tap's sign), NaN (never the extremum),
    +-inf inputs and an element of -inf taps (a pair that never improves keeps tap 0)."""
    B, C, H, W, K = 1, 3, 20, 24, 3
    x = seeded(320, B, C, H, W, dtype=dtype, kind="quant")
    x[:, :, ::3, ::2] = -0.0
    x[0, 0, 4, 5] = float("nan")
    x[0, 1, 7, 7] = float("inf")
    x[0, 1, 9, 11] = -float("inf")
    w = torch.zeros((C, 1, K, K), dtype=dtype)
    w[0, 0, 0, 0] = -0.0
    w[2] = -float("inf") if op == O.DILATION else float("inf")
    for padding in PADDINGS:
        print(f"band special values op={op} {padding} {dtype}", flush=True)
        out, taps = _forward(op, padding, x, w, 0)
        ref, _ = O.morpho_forward(op, IDENT, O.PADDINGS[padding], PV, x.numpy(), w.numpy())
        assert np.array_equal(out, ref, equal_nan=True) and np.array_equal(np.signbit(out), np.signbit(ref)), padding
        out_t, taps_t = _forward(op, padding, x, w, 1)
        assert np.array_equal(out_t, out, equal_nan=True) and np.array_equal(taps_t, taps), padding


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("K", [3, 5])
@pytest.mark.parametrize("op", [O.DILATION, O.EROSION])
def test_band_backward(op, K, dtype):
    for si, (B, C, H, W) in enumerate(SHAPES):
        print(f"band backward op={op} {K}x{K} {dtype} shape {(B, C, H, W)}", flush=True)
        x = seeded(330 + si, B, C, H, W, dtype=dtype, kind="randn")
        w = seeded(340 + si, C, 1, K, K, dtype=dtype, kind="randn", scale=0.3)
        g = seeded(350 + si, B, C, H, W, dtype=dtype, kind="randn")
        for padding in ("geodesic", "replicate"):
            _, taps = _forward(op, padding, x, w, 0)
            gx, gw = _backward(op, x, w, taps, g, 0)
            gx_t, gw_t = _backward(op, x, w, taps, g, 1)
            assert np.array_equal(gx, gx_t), (si, padding)
            assert normwise_error(gw, gw_t) <= TOL[dtype], (si, padding)
            want_gx, want_gw = O.morpho_backward(op, IDENT, O.PADDINGS[padding], PV, x.numpy(), w.numpy(), g.numpy())
            assert normwise_error(gx, want_gx) <= TOL[dtype], (si, padding)
            assert normwise_error(gw, want_gw) <= TOL[dtype], (si, padding)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K", [3, 5])
def test_band_backward_16bit(K, dtype):
    """16-bit gradients: the band gather reads and writes them directly; grad_input equals the tiled
    gather's bit for bit, grad_weight agrees within float32 rounding of its partial sums."""
    B, C, H, W = 2, 3, 37, 24
    print(f"band backward 16-bit {K}x{K} {dtype}", flush=True)
    x = seeded(360, B, C, H, W, kind="randn").to(dtype)
    w = seeded(361, C, 1, K, K, kind="randn", scale=0.3).to(dtype)
    g = seeded(362, B, C, H, W, kind="randn").to(dtype)
    taps = torch.empty((B, C, H, W), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(x, device="cuda")
    _native.morpho_forward(O.DILATION, IDENT, True, 0.0, x.cuda(), w.cuda(), 0, out, taps, (B, C, C, 1, H, W, K, K))
    gx, gw = _backward(O.DILATION, x, w, taps, g, 0, tensors=True)
    gx_t, gw_t = _backward(O.DILATION, x, w, taps, g, 1, tensors=True)
    assert torch.equal(gx.view(torch.int16), gx_t.view(torch.int16))
    assert normwise_error(gw.double().numpy(), gw_t.double().numpy()) <= 1e-2


def test_band_full_size_identity_through_the_operator():
    """configs[3]'s shape (32, 128, 112, 112) float64 through torch.ops.morphocore (the band kernels),
    equal to the tiled kernels' results on a one-element offset copy: output and grad_input bit for
    bit, grad_weight within 1e-12."""
    B, C, H, W, K = 32, 128, 112, 112, 3
    print("band kernels at configs[3]'s shape", flush=True)
    x = seeded(370, B, C, H, W, dtype=torch.float64, low=-1.0, scale=2.0)
    w = seeded(371, C, 1, K, K, dtype=torch.float64, kind="randn", scale=0.1)
    g = seeded(372, B, C, H, W, dtype=torch.float64, kind="randn")
    out, taps = _forward(O.DILATION, "replicate", x, w, 0)
    out_t, taps_t = _forward(O.DILATION, "replicate", x, w, 1)
    assert np.array_equal(out, out_t) and np.array_equal(taps, taps_t)
    gx, gw = _backward(O.DILATION, x, w, taps, g, 0)
    gx_t, gw_t = _backward(O.DILATION, x, w, taps, g, 1)
    assert np.array_equal(gx, gx_t)
    assert normwise_error(gw, gw_t) <= 1e-12
