"""The operators inside HIP graphs (torch.cuda.graph): every launch goes to torch's current stream, and
nothing in the native code allocates with hipMalloc, clears with hipMemsetAsync or synchronises the
device, so a captured forward, or a whole captured training step (forward and backward), replays the
same kernels on the graph's own memory. Each graph is replayed several times with new inputs copied
in, other eager work and synchronisations between the replays, and every replay is checked against
the eager result of the same inputs."""
import pytest
import torch

import morphocore_amd as mca

pytestmark = pytest.mark.gpu

F = mca.functional
DEV = "cuda"


def _inputs(seed, shape_x, shape_w, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape_x, generator=g, dtype=dtype).to(DEV), (torch.randn(*shape_w, generator=g, dtype=dtype) * 0.3).to(DEV)


def _warm(fn):
    """Warm-up on a side stream, as torch's graph capture expects."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()


def _STACK(x, w):
    """dilation(max) -> smorph(sum, alpha 2) -> erosion(min), one element for the three layers."""
    alpha = torch.full((w.shape[0], x.shape[1]), 2.0, dtype=x.dtype, device=DEV)
    return [("dilation", w, "max", "replicate"), ("smorph", w, alpha, "sum"), ("erosion", w, "min", "replicate")]


CASES = [
    ("dilation max 3x3", lambda x, w: F.dilation(x, w, "max", "replicate"), (4, 3, 64, 64), (16, 3, 3, 3)),
    ("erosion sum 5x5", lambda x, w: F.erosion(x, w, "sum", "geodesic"), (2, 8, 40, 96), (8, 8, 5, 5)),
    ("dilation identity 3x3 f64", lambda x, w: F.dilation(x, w, "identity", "replicate"), (2, 16, 48, 64), (16, 1, 3, 3)),
    ("erosion min 11x11", lambda x, w: F.erosion(x, w, "min", "zero"), (2, 4, 256, 512), (8, 4, 11, 11)),
    ("smorph mean 7x7", lambda x, w: F.smorph(x, w, torch.full((w.shape[0], x.shape[1]), 1.5, device=DEV), channel_merge_mode="mean"),
     (2, 4, 40, 80), (4, 4, 7, 7)),
    ("stack 5x5", lambda x, w: F.morpho_stack(x, _STACK(x, w)), (2, 4, 40, 80), (4, 4, 5, 5)),
    ("stack 5x5 chunks of one", lambda x, w: F.morpho_stack(x, _STACK(x, w), chunk=1), (3, 4, 40, 80), (4, 4, 5, 5)),
]


@pytest.mark.parametrize("name,fn,sx,sw", CASES, ids=[c[0] for c in CASES])
def test_captured_forward(name, fn, sx, sw):
    dtype = torch.float64 if "f64" in name else torch.float32
    print(f"graph forward {name}", flush=True)
    x, w = _inputs(1, sx, sw, dtype)
    sx_, sw_ = x.clone(), w.clone()
    with torch.no_grad():
        _warm(lambda: fn(sx_, sw_))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = fn(sx_, sw_)
        for k in range(4):
            xn, wn = _inputs(10 + k, sx, sw, dtype)
            sx_.copy_(xn)
            sw_.copy_(wn)
            graph.replay()
            eager_other = fn(xn * 0.5, wn)  # eager work between the replays
            torch.cuda.synchronize()
            want = fn(xn, wn)
            assert torch.equal(out, want), (name, k)
            del eager_other


@pytest.mark.parametrize("name,fn,sx,sw", CASES, ids=[c[0] for c in CASES])
def test_captured_training_step(name, fn, sx, sw):
    """Forward and backward captured together (the whole-step capture of torch.cuda.graph): outputs and
    both gradients of every replay against an eager step."""
    dtype = torch.float64 if "f64" in name else torch.float32
    print(f"graph step {name}", flush=True)
    x, w = _inputs(2, sx, sw, dtype)
    sx_, sw_ = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    g = torch.randn(sx[0], sw[0], sx[2], sx[3], dtype=dtype, device=DEV)

    def step():
        sx_.grad = None
        sw_.grad = None
        out = fn(sx_, sw_)
        out.backward(g)
        return out

    _warm(step)
    graph = torch.cuda.CUDAGraph()
    sx_.grad = None
    sw_.grad = None
    with torch.cuda.graph(graph):
        out = fn(sx_, sw_)
        out.backward(g)
    gx_static, gw_static = sx_.grad, sw_.grad
    for k in range(4):
        xn, wn = _inputs(20 + k, sx, sw, dtype)
        with torch.no_grad():
            sx_.copy_(xn)
            sw_.copy_(wn)
        graph.replay()
        got = (out.detach().clone(), gx_static.clone(), gw_static.clone())
        torch.cuda.synchronize()
        xe, we = xn.clone().requires_grad_(True), wn.clone().requires_grad_(True)
        oe = fn(xe, we)
        oe.backward(g)
        torch.cuda.synchronize()
        assert torch.equal(got[0], oe.detach()), (name, k, "output")
        # Sums of floating-point atomics may differ in their last bits between two runs.
        torch.testing.assert_close(got[1], xe.grad, rtol=1e-6, atol=1e-6 * float(xe.grad.abs().max()))
        torch.testing.assert_close(got[2], we.grad, rtol=1e-6, atol=1e-6 * float(we.grad.abs().max()))
