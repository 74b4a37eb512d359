"""Opening and closing with per-channel merges on both stages, as one fused operator call.

The reference composes opening / closing from two operator calls (functional/opening.py:96-101,
functional/closing.py:96-101). When the first stage also merges per channel ('identity', the form
nn.Opening / nn.Closing build with a shared structuring element), ``torch.ops.morphocore.opening_closing``
computes the same values in one kernel, keeping the intermediate image on chip. The random draws happen
in the composition's order: the first stage's dropout, then the second's, then the operator's noise
(first stage, then second). Only dropout and noise together would interleave differently (the
composition draws the first stage's noise before the second stage's dropout); that case runs the
composition itself.
"""
import torch

from ._dropout import drop_weights
from ._ops import ops
from .merge_enum import str_to_padding

# The reference's operation values (functional/csrc/cpp/morpho_op_enum.hpp:17-21).
DILATION = 0
EROSION = 1


def fused_pair(x: torch.Tensor, w_first: torch.Tensor, w_second: torch.Tensor, first_op: int, padding_mode: str, save_indices: bool,
               padding_value: float, weight_dropout: float, training: bool, noise_scale: float):
    """The fused opening (first_op erosion) or closing (first_op dilation), or None when the composition
    must run (dropout and noise together in training)."""
    drop = training and weight_dropout > 0.0
    noise = noise_scale if training else 0.0
    if drop and noise > 0.0:
        return None
    if drop:
        w_first = drop_weights(w_first, weight_dropout)
        w_second = drop_weights(w_second, weight_dropout)
    # The erosion's element is flipped, as functional.erosion passes it to its operator.
    if first_op == EROSION:
        w_first = w_first.flip((-2, -1))
    else:
        w_second = w_second.flip((-2, -1))
    return ops.opening_closing(x, w_first, w_second, first_op, str_to_padding(padding_mode), padding_value, save_indices, noise)


__all__ = ['fused_pair', 'DILATION', 'EROSION']
