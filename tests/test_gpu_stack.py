"""Layer stacks (torch.ops.morphocore.morpho_stack, the C ABI's mca_stack_*, functional.morpho_stack,
nn.MorphoStack) against the oracle run layer by layer, and against the single operators.

The oracle chain applies the oracle's operators in turn (morpho_forward / smorph_forward, then the
backwards in reverse, each from the previous one's gradient); the stack's output must equal it bit
for bit (NaN positions equal). In float64 every gradient is within the float64 contract of the oracle
chain's. In float32 the gradients are compared with the same chain of the single HIP operators (each
pinned to the oracle by its own tests): within the float32 contract. A float32 chain's gradients also
meet the oracle chain's within 1e-5 norm-wise: each layer adds its own float32 rounding (1e-6 for one
operator) and the routed sums of a layer's element gradient can cancel, so the chain's bound is looser
than one operator's. Chunks of 1, 2 (a partial last chunk), more than the batch, and the default
(the whole batch) give the same values."""
import numpy as np
import pytest
import torch

import morphocore_amd as mca
from morphocore_amd import _native
from oracle import oracle as O
from tests.helpers import TOL, normwise_error, seeded

pytestmark = pytest.mark.gpu

F = mca.functional
DEV = "cuda"
KIND = {"dilation": 0, "erosion": 1, "smorph": 2}
PAD = {"zero": O.ZERO, "geodesic": O.GEODESIC, "constant": O.CONSTANT, "replicate": O.REPLICATE}

# name: (channels of the input, then per layer (kind, merge, out channels, K, padding or alpha)).
CHAINS = {
    "c5": (4, [("dilation", "max", 4, 5, "replicate"), ("smorph", "sum", 4, 5, 5.0), ("erosion", "min", 4, 5, "replicate")]),
    "c5_k11": (3, [("dilation", "max", 3, 11, "replicate"), ("smorph", "sum", 3, 11, 5.0), ("erosion", "min", 3, 11, "replicate")]),
    "mixed": (3, [("erosion", "sum", 5, 3, "geodesic"), ("dilation", "identity", 5, 5, "zero"), ("smorph", "max", 2, 3, -2.0),
                  ("dilation", "mean", 3, 7, "constant")]),
    "smorph_first": (2, [("smorph", "min", 3, 7, 1.5), ("smorph", "identity", 3, 5, -0.5), ("erosion", "max", 2, 3, "zero")]),
    "one_layer": (3, [("erosion", "min", 4, 5, "constant")]),
}


def _chain(name, dtype, seed, B=3, H=20, W=70):
    """Input, per-layer (kind, merge, weight as the operator receives it, alpha or None, padding code,
    padding value)."""
    cin, spec = CHAINS[name]
    x = seeded(seed, B, cin, H, W, dtype=dtype, kind="randn")
    layers = []
    for j, (kind, merge, cout, K, extra) in enumerate(spec):
        cw = 1 if merge == "identity" else cin
        w = seeded(seed + 10 + j, cout, cw, K, K, dtype=dtype, kind="randn", scale=0.3)
        if kind == "smorph":
            pairs = (cout,) if merge == "identity" else (cout, cin)
            alpha = torch.full(pairs, extra, dtype=dtype) + seeded(seed + 20 + j, *pairs, dtype=dtype, kind="randn", scale=0.1)
            layers.append((kind, merge, w, alpha, 0, 0.0))
        else:
            layers.append((kind, merge, w, None, PAD[extra], -0.25))
        cin = cout
    return x, layers


def _oracle_chain(x, layers, g):
    """Forward values and (grad_input, [grad_weight], [grad_alpha]) of the chain, by the oracle."""
    acts = [x]
    for kind, merge, w, alpha, pad, pv in layers:
        if kind == "smorph":
            acts.append(O.smorph_forward(O.MERGES[merge], acts[-1], w, alpha))
        else:
            acts.append(O.morpho_forward(O.DILATION if kind == "dilation" else O.EROSION, O.MERGES[merge], pad, pv, acts[-1], w)[0])
    gw, ga = [None] * len(layers), []
    for j in reversed(range(len(layers))):
        kind, merge, w, alpha, pad, pv = layers[j]
        if kind == "smorph":
            g, gw[j], a = O.smorph_backward(O.MERGES[merge], acts[j], w, alpha, g)
            ga.insert(0, a)
        else:
            g, gw[j] = O.morpho_backward(O.DILATION if kind == "dilation" else O.EROSION, O.MERGES[merge], pad, pv, acts[j], w, g)
    return acts[-1], g, gw, ga


def _stack_op(x, layers, chunk, save=True):
    """The chain through torch.ops.morphocore.morpho_stack; returns the output and the leaf tensors."""
    xd = x.to(DEV).requires_grad_(True)
    ws = [w.to(DEV).requires_grad_(True) for _, _, w, _, _, _ in layers]
    alphas = [a.to(DEV).requires_grad_(True) for _, _, _, a, _, _ in layers if a is not None]
    out = torch.ops.morphocore.morpho_stack(xd, ws, alphas, [KIND[k] for k, *_ in layers], [int(O.MERGES[m]) for _, m, *_ in layers],
                                            [p for *_, p, _ in layers], [v for *_, v in layers], save, chunk)
    return out, xd, ws, alphas


def _single_ops(x, layers):
    """The chain of single operators (torch.ops.morphocore.dilation / erosion / smorph)."""
    xd = x.to(DEV).requires_grad_(True)
    ws = [w.to(DEV).requires_grad_(True) for _, _, w, _, _, _ in layers]
    alphas = [a.to(DEV).requires_grad_(True) for _, _, _, a, _, _ in layers if a is not None]
    y, a = xd, 0
    for (kind, merge, _, _, pad, pv), w in zip(layers, ws):
        if kind == "smorph":
            y = torch.ops.morphocore.smorph(y, w, alphas[a], O.MERGES[merge])
            a += 1
        else:
            fn = torch.ops.morphocore.dilation if kind == "dilation" else torch.ops.morphocore.erosion
            y = fn(y, w, O.MERGES[merge], pad, pv, True, 0.0)
    return y, xd, ws, alphas


def _assert_bits(got, want):
    got, want = np.ascontiguousarray(got), np.ascontiguousarray(want)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), "NaN positions differ"
    assert np.array_equal(got[~nan], want[~nan]), f"values differ: max {np.max(np.abs(got[~nan] - want[~nan]))}"


@pytest.mark.parametrize("chunk", [0, 1, 2, 5])
@pytest.mark.parametrize("name", list(CHAINS))
def test_stack_float64_matches_oracle_chain(name, chunk):
    print(f"stack f64 {name} chunk {chunk}", flush=True)
    x, layers = _chain(name, torch.float64, 300)
    npl = [(k, m, w.numpy(), None if a is None else a.numpy(), p, v) for k, m, w, a, p, v in layers]
    out, xd, ws, alphas = _stack_op(x, layers, chunk)
    g = seeded(399, *out.shape, dtype=torch.float64, kind="randn")
    ref, gx, gw, ga = _oracle_chain(x.numpy(), npl, g.numpy())
    _assert_bits(out.detach().cpu().numpy(), ref)
    out.backward(g.to(DEV))
    assert normwise_error(xd.grad.cpu().numpy(), gx) <= TOL[torch.float64]
    for j, w in enumerate(ws):
        assert normwise_error(w.grad.cpu().numpy(), gw[j]) <= TOL[torch.float64], f"layer {j} weight"
    for a, want in zip(alphas, ga):
        assert normwise_error(a.grad.cpu().numpy(), want) <= TOL[torch.float64]


@pytest.mark.parametrize("save", [True, False])
@pytest.mark.parametrize("chunk", [0, 1, 2])
@pytest.mark.parametrize("name", list(CHAINS))
def test_stack_float32_matches_layers_and_oracle(name, chunk, save):
    print(f"stack f32 {name} chunk {chunk} save {save}", flush=True)
    x, layers = _chain(name, torch.float32, 500)
    out, xd, ws, alphas = _stack_op(x, layers, chunk, save)
    ref, rx, rws, ralphas = _single_ops(x, layers)
    _assert_bits(out.detach().cpu().numpy(), ref.detach().cpu().numpy())
    npl = [(k, m, w.numpy(), None if a is None else a.numpy(), p, v) for k, m, w, a, p, v in layers]
    g = seeded(599, *out.shape, kind="randn")
    oref, ogx, ogw, oga = _oracle_chain(x.numpy(), npl, g.numpy())
    _assert_bits(out.detach().cpu().numpy(), oref)
    out.backward(g.to(DEV))
    ref.backward(g.to(DEV))
    pairs = [(xd, rx, ogx)] + [(w, r, o) for w, r, o in zip(ws, rws, ogw)] + [(a, r, o) for a, r, o in zip(alphas, ralphas, oga)]
    for got, single, orc in pairs:
        assert normwise_error(got.grad.cpu().numpy(), single.grad.cpu().numpy()) <= TOL[torch.float32]
        assert normwise_error(got.grad.cpu().numpy(), orc) <= 1e-5


def test_stack_c_abi_partial_gradients():
    """Through the C ABI: the c5 chain with grad_input and the first layer's weight gradient not
    wanted (NULL), three chunks of one; the wanted gradients equal those of the all-gradients call."""
    print("stack C ABI", flush=True)
    x, layers = _chain("c5", torch.float32, 700)
    xd = x.to(DEV)
    ws = [w.to(DEV) for _, _, w, _, _, _ in layers]
    aps = [a.to(DEV).reshape(-1).contiguous() if a is not None else None for _, _, _, a, _, _ in layers]

    def specs(grads):
        out = []
        for j, (kind, merge, _, _, pad, pv) in enumerate(layers):
            s = dict(kind=KIND[kind], merge=int(O.MERGES[merge]), save=1, weight=ws[j])
            if kind == "smorph":
                s["alpha"] = aps[j]
            else:
                s["replicate"] = int(pad == O.REPLICATE)
                s["fill"] = O.fill_value(KIND[kind], pad, pv, np.float32)
            s.update(grads[j])
            out.append(s)
        return _native.stack_layers(out)

    full = [dict(grad_weight=torch.empty_like(w)) for w in ws]
    full[1]["grad_alpha"] = torch.empty_like(aps[1])
    part = [{}, dict(grad_weight=torch.empty_like(ws[1])), dict(grad_weight=torch.empty_like(ws[2]))]
    g = seeded(799, x.shape[0], ws[-1].shape[0], *x.shape[2:], kind="randn").to(DEV)
    results = []
    for grads, gin in ((full, torch.empty_like(xd)), (part, None)):
        arr = specs(grads)
        saved_b, bwd_b = _native.stack_plan(arr, torch.float32, tuple(x.shape), 1)
        saved = torch.empty(max(saved_b, 1), dtype=torch.uint8, device=DEV)
        ws_buf = torch.empty(max(bwd_b, 1), dtype=torch.uint8, device=DEV)
        out = torch.empty(x.shape[0], ws[-1].shape[0], *x.shape[2:], device=DEV)
        _native.stack_forward(arr, xd, out, saved, 1)
        _native.stack_backward(arr, xd, out, g, gin, saved, ws_buf, 1)
        torch.cuda.synchronize()
        results.append((out.cpu(), gin, grads))
    (o1, gin1, g1), (o2, _, g2) = results
    assert torch.equal(o1, o2)
    for j in (1, 2):  # sums of floating-point atomics may differ in their last bits between two runs
        assert normwise_error(g2[j]["grad_weight"].cpu().numpy(), g1[j]["grad_weight"].cpu().numpy()) <= TOL[torch.float32]
    npl = [(k, m, w.numpy(), None if a is None else a.numpy(), p, v) for k, m, w, a, p, v in layers]
    ref, gx, gw, ga = _oracle_chain(x.numpy(), npl, g.cpu().numpy())
    _assert_bits(o1.numpy(), ref)
    assert normwise_error(gin1.cpu().numpy(), gx) <= 1e-5
    for j in range(3):
        assert normwise_error(g1[j]["grad_weight"].cpu().numpy(), gw[j]) <= 1e-5
    assert normwise_error(g1[1]["grad_alpha"].cpu().numpy().reshape(ga[0].shape), ga[0]) <= 1e-5


def test_stack_empty_batch_and_no_gradient_graph():
    x, layers = _chain("c5", torch.float32, 800, B=0)
    out, xd, ws, alphas = _stack_op(x, layers, 0)
    assert out.shape == (0, 4, 20, 70)
    out.sum().backward()
    assert xd.grad.shape == xd.shape
    for t in ws + alphas:
        assert t.grad is not None and not t.grad.any()
    x, layers = _chain("c5", torch.float32, 801)
    with torch.no_grad():
        out, *_ = _stack_op(x, layers, 0)
    assert out.grad_fn is None


@pytest.mark.parametrize("shape,couts", [((2, 3, 0, 9), (4, 4)), ((2, 3, 6, 0), (4, 4)), ((2, 3, 6, 9), (0, 4)), ((2, 0, 6, 9), (4, 2))])
@pytest.mark.parametrize("merge", ["max", "sum", "mean"])
def test_stack_empty_planes_and_channels(shape, couts, merge):
    """Empty planes and a layer without channels: the values of the single operators (the merge's start
    value where a layer has no input channel) and their gradients (zero or empty)."""
    print(f"stack empty {shape} {couts} {merge}", flush=True)
    B, C, H, W = shape
    x = torch.randn(shape, dtype=torch.float64)
    ws = [torch.randn(couts[0], C, 3, 3, dtype=torch.float64), torch.randn(couts[1], couts[0], 3, 3, dtype=torch.float64)]
    layers = [("dilation", merge, ws[0], None, O.REPLICATE, 0.0), ("erosion", merge, ws[1], None, O.GEODESIC, 0.0)]
    out, xd, wd, _ = _stack_op(x, layers, 1)
    ref, rx, rws, _ = _single_ops(x, layers)
    assert out.shape == ref.shape
    assert torch.equal(out.isnan(), ref.isnan()) and torch.equal(out.nan_to_num(), ref.nan_to_num())
    g = torch.randn(out.shape, dtype=torch.float64, device=DEV)
    out.backward(g)
    ref.backward(g)
    for a, b in [(xd, rx)] + list(zip(wd, rws)):
        assert a.grad.shape == b.grad.shape
        torch.testing.assert_close(a.grad, b.grad, rtol=1e-12, atol=0)


def _modules(dtype):
    torch.manual_seed(5)
    d = mca.nn.Dilation(3, 4, 5, "max", "replicate", dtype=dtype)
    s = mca.nn.SMorph(4, 4, 5, "sum", init_alpha=3.0, dtype=dtype)
    e = mca.nn.Erosion(4, 2, 3, "min", "geodesic", dtype=dtype)
    with torch.no_grad():
        for m in (d, s, e):
            m.weight.copy_(torch.randn(m.weight.shape, dtype=m.weight.dtype) * 0.3)
    return [m.to(DEV) for m in (d, s, e)]


def test_nn_morpho_stack_equals_sequential():
    """nn.MorphoStack of Dilation -> SMorph -> Erosion modules: the same output as nn.Sequential of the
    same modules, bit for bit, and gradients within the contract; its parameters are the layers'."""
    mods = _modules(torch.float32)
    stack = mca.nn.MorphoStack(*mods, chunk=1)
    seq = torch.nn.Sequential(*mods)
    assert [n for n, _ in stack.named_parameters()] == [f"layers.{n}" for n, _ in seq.named_parameters()]
    x = seeded(901, 3, 3, 24, 40, kind="randn").to(DEV)
    out = stack(x)
    grads_stack = torch.autograd.grad(out, list(seq.parameters()), torch.ones_like(out))
    ref = seq(x)
    grads_seq = torch.autograd.grad(ref, list(seq.parameters()), torch.ones_like(ref))
    assert torch.equal(out, ref)
    for a, b in zip(grads_stack, grads_seq):
        assert normwise_error(a.cpu().numpy(), b.cpu().numpy()) <= TOL[torch.float32]


def test_nn_morpho_stack_runs_layers_for_dropout():
    """In training, a layer with weight dropout is not part of a stack: the forward calls the layers in
    turn, and with the same seed draws the same taps as nn.Sequential."""
    mods = _modules(torch.float32)
    mods[0].weight_dropout = 0.3
    stack = mca.nn.MorphoStack(*mods).train()
    seq = torch.nn.Sequential(*mods).train()
    x = seeded(902, 2, 3, 16, 30, kind="randn").to(DEV)
    torch.manual_seed(11)
    a = stack(x)
    torch.manual_seed(11)
    b = seq(x)
    assert torch.equal(a, b)


def test_nn_morpho_stack_calls_layers_with_hooks():
    """A forward hook on a layer runs: the stack then calls the layers in turn (same values)."""
    mods = _modules(torch.float32)
    seen = []
    handle = mods[1].register_forward_hook(lambda m, i, o: seen.append(o.shape))
    x = seeded(903, 2, 3, 16, 30, kind="randn").to(DEV)
    out = mca.nn.MorphoStack(*mods)(x)
    handle.remove()
    assert seen == [torch.Size([2, 4, 16, 30])]
    assert torch.equal(out, torch.nn.Sequential(*mods)(x))


def test_stack_rejects_bad_chains():
    x = torch.randn(2, 3, 8, 8, device=DEV)
    w = torch.randn(4, 2, 3, 3, device=DEV)
    with pytest.raises(RuntimeError, match="Input channels must match weight input channels"):
        torch.ops.morphocore.morpho_stack(x, [w], [], [0], [2], [3], [0.0], True, 0)
    with pytest.raises(RuntimeError, match="one alpha per smorph layer"):
        torch.ops.morphocore.morpho_stack(x, [torch.randn(4, 3, 3, 3, device=DEV)], [], [2], [2], [0], [0.0], True, 0)
    with pytest.raises(RuntimeError, match="Unsupported merge operation"):
        torch.ops.morphocore.morpho_stack(x, [torch.randn(4, 3, 3, 3, device=DEV)], [], [0], [4], [3], [0.0], True, 0)
    with pytest.raises(RuntimeError, match="not implemented for 'Half'"):
        torch.ops.morphocore.morpho_stack(x.half(), [torch.randn(4, 3, 3, 3, device=DEV).half()], [], [0], [2], [3], [0.0], True, 0)
    with pytest.raises(ValueError, match="Unknown layer kind"):
        F.morpho_stack(x, [("opening", w)])


@pytest.mark.parametrize("chunk", [0, 1])
def test_stack_full_size_c5(chunk):
    """BASELINE configs[4]'s chain at full size (8 x 64 x 512 x 512, 11 x 11 elements, alpha 5),
    through functional.morpho_stack, in one chunk and in chunks of one batch element: output bit for
    bit that of the three functional operators, and gradients within the float32 contract of theirs."""
    print(f"stack full-size c5 chunk {chunk}", flush=True)
    g = torch.Generator().manual_seed(0)
    x = (torch.rand(8, 64, 512, 512, generator=g)).to(DEV).requires_grad_(True)
    ws = [(torch.randn(64, 64, 11, 11, generator=g) * 0.05).to(DEV).requires_grad_(True) for _ in range(3)]
    alpha = torch.full((64, 64), 5.0, device=DEV, requires_grad=True)
    grad = torch.randn(8, 64, 512, 512, generator=g).to(DEV)
    params = [x] + ws + [alpha]
    out = F.morpho_stack(x, [("dilation", ws[0], "max", "replicate"), ("smorph", ws[1], alpha, "sum"), ("erosion", ws[2], "min", "replicate")],
                         chunk=chunk)
    got = torch.autograd.grad(out, params, grad)
    out = out.detach()
    y = F.erosion(F.smorph(F.dilation(x, ws[0], "max", "replicate"), ws[1], alpha, channel_merge_mode="sum"), ws[2], "min", "replicate")
    want = torch.autograd.grad(y, params, grad)
    assert torch.equal(out, y.detach())
    del out, y
    for name, a, b in zip(["x", "w1", "w2", "w3", "alpha"], got, want):
        err = float((a - b).abs().max() / b.abs().max())
        assert err <= TOL[torch.float32], f"{name}: {err}"


def _random_chain(seed, dtype):
    rng = np.random.default_rng(1000 + seed)
    B, C = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    H, W = int(rng.integers(3, 30)), int(rng.integers(3, 50))
    cin = C
    layers = []
    for j in range(int(rng.integers(1, 5))):
        kind = str(rng.choice(["dilation", "erosion", "smorph"]))
        merge = str(rng.choice(["max", "min", "sum", "mean", "identity"]))
        cout = cin if merge == "identity" else int(rng.integers(1, 5))
        KH, KW = int(rng.choice([1, 2, 3, 4, 5, 7])), int(rng.choice([1, 2, 3, 5, 6]))
        cw = 1 if merge == "identity" else cin
        w = seeded(2000 + 10 * seed + j, cout, cw, KH, KW, dtype=dtype, kind="randn", scale=0.3)
        if kind == "smorph":
            pairs = (cout,) if merge == "identity" else (cout, cin)
            alpha = seeded(3000 + 10 * seed + j, *pairs, dtype=dtype, kind="randn", scale=3.0)
            layers.append((kind, merge, w, alpha, 0, 0.0))
        else:
            pad = int(rng.choice([O.ZERO, O.GEODESIC, O.CONSTANT, O.REPLICATE]))
            layers.append((kind, merge, w, None, pad, float(rng.normal())))
        cin = cout
    chunk = int(rng.integers(0, B + 2))
    print(f"stack random chain {seed} {dtype}: {(B, C, H, W)} chunk {chunk} "
          f"{[(k, m, tuple(w.shape), p) for k, m, w, _, p, _ in layers]}", flush=True)
    return seeded(4000 + seed, B, C, H, W, dtype=dtype, kind="randn"), layers, chunk


@pytest.mark.parametrize("seed", range(16))
def test_stack_random_chains_float64(seed):
    """Seeded random chains: 1-4 layers of random kind, merge, padding, element shape (square, rectangular
    and even) and channel counts, random chunking, in float64 against the oracle chain: forward bit for
    bit, gradients within 1e-12."""
    x, layers, chunk = _random_chain(seed, torch.float64)
    npl = [(k, m, w.numpy(), None if a is None else a.numpy(), p, v) for k, m, w, a, p, v in layers]
    out, xd, ws, alphas = _stack_op(x, layers, chunk)
    g = seeded(5000 + seed, *out.shape, dtype=torch.float64, kind="randn")
    ref, gx, gw, ga = _oracle_chain(x.numpy(), npl, g.numpy())
    _assert_bits(out.detach().cpu().numpy(), ref)
    out.backward(g.to(DEV))
    assert normwise_error(xd.grad.cpu().numpy(), gx) <= TOL[torch.float64]
    for j, w in enumerate(ws):
        assert normwise_error(w.grad.cpu().numpy(), gw[j]) <= TOL[torch.float64], f"layer {j} weight"
    for a, want in zip(alphas, ga):
        assert normwise_error(a.grad.cpu().numpy(), want) <= TOL[torch.float64]


@pytest.mark.parametrize("seed", range(16))
def test_stack_random_chains_float32(seed):
    """The same random chains in float32 against the chain of single operators: forward bit for bit,
    gradients within 1e-6."""
    x, layers, chunk = _random_chain(seed, torch.float32)
    out, xd, ws, alphas = _stack_op(x, layers, chunk)
    ref, rx, rws, ralphas = _single_ops(x, layers)
    _assert_bits(out.detach().cpu().numpy(), ref.detach().cpu().numpy())
    g = seeded(6000 + seed, *out.shape, kind="randn").to(DEV)
    out.backward(g)
    ref.backward(g)
    for got, want in [(xd, rx)] + list(zip(ws, rws)) + list(zip(alphas, ralphas)):
        assert normwise_error(got.grad.cpu().numpy(), want.grad.cpu().numpy()) <= TOL[torch.float32]
