"""A chain of dilation / erosion / smorph layers as one operator.

No reference counterpart: the reference chains its functional operators in Python, one operator call
and one autograd node per layer (morphocore/functional/dilation.py:89-91, smorph.py:72-75,
erosion.py:89-91). ``morpho_stack`` runs the same chain through the native stack executor
(``torch.ops.morphocore.morpho_stack``): one autograd node for the chain, each chunk of batch elements
through every layer before the next chunk, and a backward that holds one chunk of each intermediate
gradient instead of whole-batch tensors.
"""
from typing import Sequence

import torch

from ._ops import ops
from .merge_enum import str_to_merge, str_to_padding
from .smorph import w_tilde

_KINDS = {"dilation": 0, "erosion": 1, "smorph": 2}


def _spec(layer):
    kind = layer[0]
    if kind not in _KINDS:
        raise ValueError(f"Unknown layer kind: {kind}. Expected one of {sorted(_KINDS)}.")
    if kind == "smorph":
        if not 3 <= len(layer) <= 4:
            raise ValueError("A smorph layer is ('smorph', w, alpha[, channel_merge_mode])")
        merge = layer[3] if len(layer) > 3 else "sum"
        w, alpha = layer[1], layer[2]
        return _KINDS[kind], w_tilde(w, alpha, merge), alpha, str_to_merge(merge), 0, 0.0
    if not 2 <= len(layer) <= 5:
        raise ValueError(f"A {kind} layer is ('{kind}', w[, channel_merge_mode[, padding_mode[, padding_value]]])")
    merge, padding, value = (tuple(layer[2:]) + ("sum", "replicate", 0.0)[len(layer) - 2:])[:3]
    w = layer[1]
    # The erosion operator receives the flipped element, as functional.erosion passes it.
    w = w.flip((-2, -1)) if kind == "erosion" else w
    return _KINDS[kind], w, None, str_to_merge(merge), str_to_padding(padding), float(value)


def morpho_stack(x: torch.Tensor, layers: Sequence[tuple], save_indices: bool = True, chunk: int = 0) -> torch.Tensor:
    """Runs a chain of layers as one operator; the same values (bit for bit, winners included) as
    calling :func:`dilation`, :func:`erosion` and :func:`smorph` in turn, with gradients that agree
    within floating-point tolerance (each chunk's weight gradient is summed in chunk order).

    Parameters
    ----------
    x : [N, C, H, W] input on a HIP device, float32 or float64.
    layers : the chain, each layer a tuple
        ``('dilation', w, channel_merge_mode='sum', padding_mode='replicate', padding_value=0.0)``,
        ``('erosion', w, channel_merge_mode='sum', padding_mode='replicate', padding_value=0.0)`` or
        ``('smorph', w, alpha, channel_merge_mode='sum')``, with the single operators' shapes; layer l
        reads the previous layer's output channels. Weight dropout, weight noise and smorph's SMOOTH
        merge (``beta``) are not part of a stack: call the single operators for them.
    save_indices : keep each dilation's / erosion's winners and, in float32, each smorph layer's pair
        statistics for the backward (within the saved-statistics budget); otherwise it recomputes them.
    chunk : batch elements per chunk; 0 (the default) takes the whole batch, the fastest for these
        instruction-bound layers; a smaller chunk bounds the backward's intermediate gradients to one
        chunk (at some cost in time: each layer then launches once per chunk).
    """
    if len(layers) == 0:
        raise ValueError("morpho_stack needs at least one layer")
    specs = [_spec(layer) for layer in layers]
    kinds = [s[0] for s in specs]
    weights = [s[1] for s in specs]
    alphas = [s[2] for s in specs if s[0] == _KINDS["smorph"]]
    merges = [int(s[3]) for s in specs]
    paddings = [int(s[4]) for s in specs]
    values = [s[5] for s in specs]
    return ops.morpho_stack(x, weights, alphas, kinds, merges, paddings, values, save_indices, chunk)
