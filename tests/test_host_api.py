"""Host-side behaviour of the Python API that needs no GPU: the string enums, the operator schemas,
the argument checks and their messages (the reference's, see morpho_op_wrap.hxx, bindings.cpp,
reshaper.cpp, smorph_cpu_kernels.hxx), the module parameters, and that a CPU tensor is refused
rather than computed on a fallback path."""
import pytest
import torch

import morphocore_amd as mca
from morphocore_amd.functional import MorphoMerge, MorphoPadding, str_to_merge, str_to_padding

ops = torch.ops.morphocore


def test_enum_values_match_reference():
    assert [int(m) for m in (MorphoMerge.MAX, MorphoMerge.MIN, MorphoMerge.ADD, MorphoMerge.AVERAGE, MorphoMerge.SMOOTH,
                             MorphoMerge.IDENTITY)] == [0, 1, 2, 3, 4, 5]
    assert [int(p) for p in (MorphoPadding.ZERO, MorphoPadding.GEODESIC, MorphoPadding.CONSTANT, MorphoPadding.REPLICATE)] == [0, 1, 2, 3]
    assert str_to_merge("sum") == MorphoMerge.ADD and str_to_merge("mean") == MorphoMerge.AVERAGE
    assert str_to_padding("replicate") == MorphoPadding.REPLICATE


def test_unknown_strings_raise_value_error():
    x, w = torch.randn(1, 1, 8, 8), torch.zeros(1, 1, 3, 3)
    with pytest.raises(ValueError, match="Unknown padding mode"):
        mca.functional.dilation(x, w, padding_mode="reflect")
    with pytest.raises(ValueError, match="Unknown merge mode"):
        mca.functional.erosion(x, w, channel_merge_mode="average")


def test_schemas():
    assert "float padding_value=0., bool save_indices=True, float noise_scale=0." in str(ops.dilation.default._schema)
    assert str(ops.smorph.default._schema).startswith("morphocore::smorph(Tensor input, Tensor weight, Tensor alpha, int merge)")
    assert "Tensor beta" in str(ops.smorph_scm.default._schema)


def test_operator_argument_errors():
    x, w = torch.randn(2, 3, 8, 8), torch.zeros(4, 3, 3, 3)
    with pytest.raises(RuntimeError, match="Unknown merge mode 9"):
        ops.dilation(x, w, 9, 0)
    with pytest.raises(RuntimeError, match="Unknown padding mode 7"):
        ops.erosion(x, w, 0, 7)
    with pytest.raises(RuntimeError, match="Unsupported merge operation"):
        ops.dilation(x, w, 4, 0)
    with pytest.raises(RuntimeError, match="noise_scale must be non negative"):
        ops.dilation(x, w, 0, 0, 0.0, True, -0.1)
    with pytest.raises(RuntimeError, match="Input channels must match weight input channels"):
        ops.dilation(x, torch.zeros(4, 2, 3, 3), 2, 0)
    with pytest.raises(RuntimeError, match="Identity mode requires weight.shape\\[0\\] == input.shape\\[1\\]"):
        ops.dilation(x, torch.zeros(4, 1, 3, 3), 5, 0)
    with pytest.raises(RuntimeError, match="Identity mode requires weight.shape\\[1\\] == 1"):
        ops.dilation(x, torch.zeros(3, 3, 3, 3), 5, 0)
    with pytest.raises(RuntimeError, match="Invalid input tensor"):
        ops.dilation(torch.zeros(1, 1, 1, 2, 2), w, 0, 0)
    with pytest.raises(RuntimeError, match="Invalid weight tensor dimensions"):
        ops.dilation(x, torch.zeros(3, 3, 3), 0, 0)


def test_smorph_argument_errors():
    x = torch.randn(2, 3, 8, 8)
    w = torch.zeros(4, 3, 3, 3)
    with pytest.raises(RuntimeError, match="Alpha must have one value, or shape \\[out_channels, in_channels\\]"):
        ops.smorph(x, w, torch.zeros(5), 2)
    with pytest.raises(RuntimeError, match="Alpha must have one value, or shape \\[channels\\]"):
        ops.smorph(x, torch.zeros(3, 1, 3, 3), torch.zeros(4), 5)
    with pytest.raises(RuntimeError, match="Identity mode requires weight.shape\\[1\\] == 1, got 3"):
        ops.smorph(x, torch.zeros(3, 3, 3, 3), torch.zeros(3), 5)
    with pytest.raises(RuntimeError, match="Unsupported merge operation for smorph"):
        ops.smorph(x, w, torch.zeros(4, 3), 4)
    # smorph with beta: the SMOOTH channel merge (smorph_scm), one beta per output channel
    # (smorph_scm.cpp:33).
    with pytest.raises(RuntimeError, match="Beta must have shape \\[out_channels\\]"):
        mca.functional.smorph(x, w, torch.zeros(4, 3), beta=torch.zeros(4, 3))
    with pytest.raises(RuntimeError, match="Alpha must have one value, or shape \\[out_channels, in_channels\\]"):
        ops.smorph_scm(x, w, torch.zeros(4), torch.zeros(4))
    with pytest.raises(RuntimeError, match="runs on AMD GPUs"):
        ops.smorph_scm(x, w, torch.zeros(4, 3), torch.zeros(4))


def test_cpu_tensors_are_refused_not_computed():
    x, w = torch.randn(1, 2, 8, 8), torch.zeros(3, 2, 3, 3)
    with pytest.raises(RuntimeError, match="runs on AMD GPUs"):
        mca.functional.dilation(x, w, "max")
    with pytest.raises(RuntimeError, match="runs on AMD GPUs"):
        mca.functional.smorph(x, w, torch.zeros(3, 2))


def test_module_parameters():
    d = mca.nn.Dilation(3, 5, 7)
    assert d.weight.shape == (5, 3, 7, 7) and d.weight.dtype == torch.float32 and not d.weight.any()
    e = mca.nn.Erosion(4, 4, (3, 5), channel_merge_mode="identity", dtype=torch.float64)
    assert e.weight.shape == (4, 1, 3, 5) and e.weight.dtype == torch.float64
    with pytest.raises(ValueError, match="in_channels must be equal to out_channels"):
        mca.nn.Dilation(3, 4, 3, channel_merge_mode="identity")
    s = mca.nn.SMorph(3, 6, 5, init_alpha=2.0, dtype=torch.float64)
    assert s.alpha.shape == (6, 3) and s.alpha.dtype == torch.float64 and float(s.alpha[0, 0]) == 2.0
    assert s.weight.dtype == torch.float32  # the reference does not forward dtype to the weight
    assert s.beta is None
    s2 = mca.nn.SMorph(3, 3, 3, channel_merge_mode="identity", init_beta=1.0)
    assert s2.alpha.shape == (3, 1) and s2.beta.shape == (3, 3)
    assert set(dict(d.named_parameters())) == {"weight"} and set(dict(s.named_parameters())) == {"weight", "alpha"}


def test_saved_statistics_admission_rule():
    """The rule the smorph forward applies before it keeps its pair statistics: within the per-call
    cap, within the process budget together with every buffer still alive, and at most half of the
    memory still available (so later layers keep room for their activations)."""
    from morphocore_amd import _C

    GB = 1 << 30
    policy = _C.saved_stats_policy
    assert policy(10 * GB, 0, 100 * GB, 200 * GB)
    assert not policy(0, 0, 100 * GB, 200 * GB)  # nothing to save
    assert not policy(10 * GB, 95 * GB, 100 * GB, 200 * GB)  # over the process budget
    assert not policy(10 * GB, 0, 100 * GB, 19 * GB)  # more than half of what is available
    assert not policy(10 * GB, 0, 100 * GB, 200 * GB, 5 * GB)  # over the per-call cap
    assert not policy(1, 0, 100 * GB, 200 * GB, 0)  # cap 0 disables saving
    # A 3-layer stack of 30 GB layers under a 80 GB budget: the third layer recomputes.
    live, avail, admitted = 0, 250 * GB, []
    for _ in range(3):
        ok = policy(30 * GB, live, 80 * GB, avail)
        admitted.append(ok)
        if ok:
            live += 30 * GB
            avail -= 30 * GB
        avail -= 10 * GB  # the layer's output
    assert admitted == [True, True, False]


def _reference_dropout_loop(w, p):
    """The reference's loop (functional/dilation.py:78-87), for comparison."""
    keep = torch.rand_like(w) > p
    for i in range(w.shape[0]):
        for j in range(w.shape[1]):
            if not keep[i, j].any():
                flat = torch.randint(0, keep[i, j].numel(), (1,)).item()
                keep[i, j].view(-1)[flat] = True
    return keep


@pytest.mark.parametrize("shape,p", [((4, 3, 3, 3), 0.9), ((8, 8, 5, 5), 0.97), ((3, 1, 3, 5), 0.999), ((5, 4, 1, 1), 0.5),
                                     ((16, 16, 7, 7), 0.995), ((3, 5), 0.6)])
def test_dropout_mask_matches_the_reference_loop(shape, p):
    """One pass + one randint of n draws keeps exactly the taps of the reference's per-pair loop, seed
    for seed (the generator yields the same values for one call of n draws as for n calls of one), and
    leaves the generator in the same state."""
    from morphocore_amd.functional._dropout import dropout_keep

    w = torch.randn(*shape)
    for seed in range(5):
        torch.manual_seed(seed)
        ref = _reference_dropout_loop(w, p)
        after_ref = torch.rand(3)
        torch.manual_seed(seed)
        got = dropout_keep(w, p)
        after_got = torch.rand(3)
        assert torch.equal(got, ref)
        assert torch.equal(after_got, after_ref)
        rows = got.reshape(shape[0] * shape[1], -1)
        assert bool(rows.any(dim=1).all())


def test_dropout_mask_of_a_permuted_weight():
    """A weight that is not contiguous (a permuted view: rand_like keeps its strides) gets its one
    survivor per pair on the mask itself, at the tap the reference's loop draws, counted in the
    view's own (row, column) order; every pair keeps a tap."""
    from morphocore_amd.functional._dropout import dropout_keep

    base = torch.randn(6, 2, 5, 3)
    w = base.permute(0, 1, 3, 2)  # (6, 2, 3, 5), not contiguous
    assert not w.is_contiguous()
    for seed in range(4):
        torch.manual_seed(seed)
        ref = torch.rand_like(w) > 0.999
        for i in range(w.shape[0]):
            for j in range(w.shape[1]):
                if not ref[i, j].any():
                    flat = torch.randint(0, ref[i, j].numel(), (1,)).item()
                    ref[i, j, flat // w.shape[3], flat % w.shape[3]] = True
        torch.manual_seed(seed)
        got = dropout_keep(w, 0.999)
        assert torch.equal(got, ref)
        assert bool(got.reshape(12, -1).any(dim=1).all())


def test_composition_layers_construction():
    """Opening / Closing share one structuring element by default, which needs equal channel counts
    and the identity merge (reference nn/opening.py:104-140 messages); SigmaLayer has weight and
    alpha."""
    o = mca.nn.Opening(3, 3, 5)
    assert o.erosion.weight is o.dilation.weight and len(list(o.parameters())) == 1
    c = mca.nn.Closing(3, 8, 5, share_weights=False)
    assert len(list(c.parameters())) == 2 and c.dilation.channel_merge_mode == "sum"
    with pytest.raises(ValueError, match="in_channels == out_channels"):
        mca.nn.Opening(3, 8, 5)
    with pytest.raises(ValueError, match="channel_merge_mode='identity'"):
        mca.nn.Closing(3, 3, 5, channel_merge_mode="sum")
    s = mca.nn.SigmaLayer(3, 4, 3)
    assert [tuple(p.shape) for p in s.parameters()] == [(4, 3, 3, 3), (4, 3)]
    assert set(mca.functional.__all__) >= {"opening", "closing", "sigma_layer"}


class _RecordingOps:
    """Stands in for torch.ops.morphocore in the functional layer: records each operator call and
    returns a tensor of the output's shape (no kernel runs on the CPU)."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def op(x, *args):
            self.calls.append((name, args))
            w = args[0]
            return torch.zeros(x.shape[0], w.shape[0], *x.shape[2:], dtype=x.dtype)
        return op


@pytest.mark.parametrize("kind", ["opening", "closing"])
def test_fused_pair_routing(kind, monkeypatch):
    """Per-channel merges go to the fused operator (erosion's element flipped, each stage's dropout
    drawn first, noise only in training); dropout and noise together run the composition, whose draws
    interleave; other merges always run the composition."""
    import importlib

    _pair, dil_mod, ero_mod = (importlib.import_module(f"morphocore_amd.functional.{m}") for m in ("_pair", "dilation", "erosion"))
    rec = _RecordingOps()
    monkeypatch.setattr(_pair, "ops", rec)
    monkeypatch.setattr(ero_mod, "ops", rec)
    monkeypatch.setattr(dil_mod, "ops", rec)
    f = getattr(mca.functional, kind)
    x = torch.zeros(2, 3, 8, 9)
    w1 = torch.arange(27.0).reshape(3, 1, 3, 3)
    w2 = -torch.arange(27.0).reshape(3, 1, 3, 3)
    f(x, w1, w2, 'identity', 'geodesic', noise_scale=0.3)
    name, args = rec.calls[-1]
    assert name == "opening_closing" and len(rec.calls) == 1
    first, second = (args[0], args[1])
    if kind == "opening":
        assert torch.equal(first, w1.flip((-2, -1))) and torch.equal(second, w2) and args[2] == 1
    else:
        assert torch.equal(first, w1) and torch.equal(second, w2.flip((-2, -1))) and args[2] == 0
    assert args[-1] == 0.0  # noise only in training
    rec.calls.clear()
    f(x, w1, w2, 'identity', training=True, weight_dropout=0.5, noise_scale=0.3)
    assert [c[0] for c in rec.calls] == (["erosion", "dilation"] if kind == "opening" else ["dilation", "erosion"])
    rec.calls.clear()
    f(x, w1, w2, 'identity', training=True, weight_dropout=0.5)
    assert [c[0] for c in rec.calls] == ["opening_closing"]
    rec.calls.clear()
    f(x, torch.zeros(3, 3, 3, 3), w2, 'sum')
    assert [c[0] for c in rec.calls] == (["erosion", "dilation"] if kind == "opening" else ["dilation", "erosion"])


def test_fused_sigma_routing(monkeypatch):
    import importlib

    sig_mod, dil_mod, ero_mod = (importlib.import_module(f"morphocore_amd.functional.{m}") for m in ("sigma_layer", "dilation", "erosion"))
    rec = _RecordingOps()
    for m in (sig_mod, ero_mod, dil_mod):
        monkeypatch.setattr(m, "ops", rec)
    x = torch.zeros(2, 3, 8, 9)
    w = torch.arange(27.0).reshape(3, 1, 3, 3)
    a = torch.full((3, 1), 0.5)
    mca.functional.sigma_layer(x, w, a, 'identity')
    name, args = rec.calls[-1]
    assert name == "sigma_identity" and torch.equal(args[0], w.flip((-2, -1))) and torch.equal(args[1], w)
    assert torch.allclose(args[2], torch.sigmoid(a.mean(dim=1)))
    rec.calls.clear()
    mca.functional.sigma_layer(x, w, a.double(), 'identity')  # mixed dtypes: the composition
    assert [c[0] for c in rec.calls] == ["erosion", "dilation"]


@pytest.mark.parametrize("kind", ["Opening", "Closing"])
def test_fused_layer_keeps_sub_module_hooks(kind, monkeypatch):
    """nn.Opening / nn.Closing take the fused operator only when calling the two sub-modules would run
    nothing but their own forward: a forward hook, a pre-hook, a global hook or a subclass of a
    stage makes the layer call both sub-modules, as the reference's layers always do."""
    import importlib

    _pair, dil_mod, ero_mod = (importlib.import_module(f"morphocore_amd.functional.{m}") for m in ("_pair", "dilation", "erosion"))
    rec = _RecordingOps()
    for m in (_pair, dil_mod, ero_mod):
        monkeypatch.setattr(m, "ops", rec)
    x = torch.zeros(2, 3, 8, 9)
    layer = getattr(mca.nn, kind)(3, 3, 3)
    first, second = (layer.erosion, layer.dilation) if kind == "Opening" else (layer.dilation, layer.erosion)
    order = ["erosion", "dilation"] if kind == "Opening" else ["dilation", "erosion"]
    layer(x)
    assert [c[0] for c in rec.calls] == ["opening_closing"]
    seen = []
    for register in (lambda m: m.register_forward_hook(lambda *a: seen.append("hook")),
                     lambda m: m.register_forward_pre_hook(lambda *a: seen.append("pre"))):
        for m in (first, second):
            rec.calls.clear()
            h = register(m)
            layer(x)
            h.remove()
            assert [c[0] for c in rec.calls] == order
    assert len(seen) == 4
    rec.calls.clear()
    h = torch.nn.modules.module.register_module_forward_hook(lambda *a: None)
    try:
        layer(x)
    finally:
        h.remove()
    assert [c[0] for c in rec.calls] == order

    class Sub(type(second)):
        def forward(self, x):
            return super().forward(x) + 1.0

    sub = Sub(3, 3, 3, channel_merge_mode="identity")
    sub.weight = second.weight
    if kind == "Opening":
        layer.dilation = sub
    else:
        layer.erosion = sub
    rec.calls.clear()
    layer(x)
    assert [c[0] for c in rec.calls] == order
