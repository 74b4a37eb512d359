"""The stack executor's plan (C ABI mca_stack_plan_*), without a GPU: chain validation with the single
operators' messages, and the sizes of the saved state (the activations between layers, the winners and
the float32 smorph statistics, one region per batch chunk) and of the backward workspace."""
import ctypes

import pytest
import torch

from morphocore_amd import _native


def _layers(specs):
    arr = (_native.StackLayer * len(specs))()
    for a, s in zip(arr, specs):
        for k, v in s.items():
            setattr(a, k, v)
    return arr


def _plan(specs, shape, chunk=0, dtype=torch.float32):
    return _native.stack_plan(_layers(specs), dtype, shape, chunk)


def _layer(kind, merge, cout, cw, k, save=1):
    # A non-null weight / alpha address: the plan only checks that they are given.
    return dict(kind=kind, merge=merge, out_channels=cout, weight_channels=cw, kh=k, kw=k, weight=16, alpha=16, save=save)


C5 = [_layer(0, 0, 64, 64, 11), _layer(2, 2, 64, 64, 11), _layer(1, 1, 64, 64, 11)]


def _al(n):
    return (n + 255) // 256 * 256


def test_c5_saved_state_per_chunk():
    B, C, H, W = 8, 64, 512, 512
    act = B * C * H * W * 4                 # one float32 activation
    win = C * H * W * 4                     # packed winners of one batch element
    stats = 3 * C * C * H * W * 4           # ref, 1 / S, W / S per pair and pixel of one batch element
    saved, backward = _plan(C5, (B, C, H, W), chunk=1)
    # Chunks of one batch element: 8 regions each.
    assert saved == 2 * act + 2 * 8 * _al(win) + 8 * _al(stats)
    # The automatic chunk is the whole batch: one region each.
    assert _plan(C5, (B, C, H, W))[0] == 2 * act + 2 * _al(8 * win) + _al(8 * stats)
    # Chunks of 3: three regions sized for 3 elements (the last one holds 2).
    assert _plan(C5, (B, C, H, W), chunk=3)[0] == 2 * act + 2 * 3 * _al(3 * win) + 3 * _al(3 * stats)
    # The backward: two chunk gradient buffers, the largest layer workspace, a weight and an alpha
    # gradient of one chunk, and a double accumulator for each wanted gradient (none here).
    assert backward >= 2 * _al(C * H * W * 4) + _al(64 * 64 * 121 * 4) + _al(64 * 64 * 4)


def test_unsaved_layers_keep_only_activations():
    specs = [dict(s, save=0) for s in C5]
    B, C, H, W = 4, 64, 64, 64
    assert _plan(specs, (B, C, H, W))[0] == 2 * B * C * H * W * 4
    # float64: no smorph statistics, the winners still saved.
    saved, _ = _plan(C5, (B, C, H, W), dtype=torch.float64)
    assert saved == 2 * B * C * H * W * 8 + 2 * _al(B * C * H * W * 4)


def test_wanted_gradients_add_accumulators_for_several_chunks():
    specs = [dict(s) for s in C5]
    shape = (4, 64, 64, 64)
    _, base = _plan(specs, shape, chunk=1)
    specs[1]["grad_weight"] = 16
    specs[1]["grad_alpha"] = 16
    _, more = _plan(specs, shape, chunk=1)
    assert more == base + _al(64 * 64 * 121 * 8) + _al(64 * 64 * 8)
    # One chunk: the gradients are written in place, no accumulator.
    assert _plan(specs, shape, chunk=4)[1] == _plan(C5, shape, chunk=4)[1]


@pytest.mark.parametrize("specs,message", [
    ([_layer(0, 2, 4, 2, 3)], "does not match the 3 channels it reads"),
    ([_layer(0, 5, 4, 1, 3)], "does not match the 3 channels it reads"),
    ([_layer(3, 2, 4, 3, 3)], "Unknown layer kind 3 at layer 0"),
    ([_layer(0, 4, 4, 3, 3)], "Unsupported merge operation"),
    ([_layer(0, 9, 4, 3, 3)], "Unknown merge mode 9"),
    ([_layer(0, 2, 4, 3, 3), _layer(1, 2, 2, 3, 3)], "Layer 1: the structuring element does not match the 4 channels it reads"),
    ([dict(_layer(2, 2, 4, 3, 3), alpha=None)], "Layer 0: alpha must not be null"),
    ([dict(_layer(1, 2, 4, 3, 3), weight=None)], "Layer 0: weight must not be null"),
    ([dict(_layer(1, 2, 4, 3, 0))], "Invalid structuring element shape at layer 0"),
])
def test_rejects_bad_chains(specs, message):
    with pytest.raises(RuntimeError, match=message):
        _plan(specs, (2, 3, 8, 8))


def test_rejects_empty_chain_and_negative_chunk():
    lib = _native.lib()
    saved, backward = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.mca_stack_plan_f32(None, 0, 1, 1, 1, 1, 0, ctypes.byref(saved), ctypes.byref(backward)) == 1
    assert "at least one layer" in lib.mca_last_error().decode()
    with pytest.raises(RuntimeError, match="chunk must be non negative"):
        _plan(C5, (1, 64, 8, 8), chunk=-1)


def test_element_too_large_for_the_smorph_backward():
    """The forward still plans; the backward workspace is 0 (no backward for this element)."""
    saved, backward = _plan([_layer(2, 2, 2, 2, 101)], (1, 2, 128, 128))
    assert saved == 0 and backward == 0


def test_stack_layer_specs_and_module_checks():
    """The Python layers of the stack check their arguments before any device work."""
    import morphocore_amd as mca

    w = torch.zeros(2, 2, 3, 3)
    with pytest.raises(ValueError, match="Unknown layer kind"):
        mca.functional.morpho_stack(torch.zeros(1, 2, 4, 4), [("opening", w)])
    with pytest.raises(ValueError, match="A smorph layer is"):
        mca.functional.morpho_stack(torch.zeros(1, 2, 4, 4), [("smorph", w)])
    with pytest.raises(ValueError, match="A dilation layer is"):
        mca.functional.morpho_stack(torch.zeros(1, 2, 4, 4), [("dilation", w, "max", "zero", 0.0, 1)])
    with pytest.raises(ValueError, match="Unknown merge mode"):
        mca.functional.morpho_stack(torch.zeros(1, 2, 4, 4), [("erosion", w, "median")])
    with pytest.raises(ValueError, match="at least one layer"):
        mca.functional.morpho_stack(torch.zeros(1, 2, 4, 4), [])
    with pytest.raises(TypeError, match="takes Dilation, Erosion and SMorph layers"):
        mca.nn.MorphoStack(torch.nn.ReLU())
    with pytest.raises(ValueError, match="at least one layer"):
        mca.nn.MorphoStack()
    stack = mca.nn.MorphoStack(mca.nn.Dilation(2, 3, 3), mca.nn.SMorph(3, 3, 3), chunk=2)
    assert [n for n, _ in stack.named_parameters()] == ["layers.0.weight", "layers.1.weight", "layers.1.alpha"]


def test_forward_and_backward_check_their_buffers_first():
    """Buffer sizes are checked before any launch (so these run without a GPU)."""
    arr = _layers(C5)
    shape = (2, 64, 32, 32)
    saved, backward = _native.stack_plan(arr, torch.float32, shape)
    lib = _native.lib()
    P = ctypes.c_void_p
    assert lib.mca_stack_forward_f32(ctypes.cast(arr, P), 3, 16, 16, *shape, 0, 16, saved - 1, None) == 1
    assert "Saved-state buffer too small" in lib.mca_last_error().decode()
    assert lib.mca_stack_backward_f32(ctypes.cast(arr, P), 3, 16, 16, 16, None, *shape, 0, 16, saved, 16, backward - 1, None) == 1
    assert "Workspace too small" in lib.mca_last_error().decode()
    big = _layers([_layer(2, 2, 2, 2, 101)])
    assert lib.mca_stack_backward_f32(ctypes.cast(big, P), 1, 16, 16, 16, None, 1, 2, 128, 128, 0, 16, 0, 16, 1 << 20, None) == 1
    assert "too large for the smorph backward" in lib.mca_last_error().decode()
