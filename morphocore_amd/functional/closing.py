import torch

from ._pair import DILATION, fused_pair
from .dilation import dilation
from .erosion import erosion


def closing(x: torch.Tensor, w_dilation: torch.Tensor, w_erosion: torch.Tensor, channel_merge_mode: str = 'sum',
            padding_mode: str = 'replicate', save_indices: bool = True, padding_value: float = 0.0, weight_dropout: float = 0.0,
            training: bool = False, noise_scale: float = 0.0) -> torch.Tensor:
    """Morphological closing: a dilation, then a per-channel ('identity') erosion of its output.

    Same signature, defaults and semantics as the reference's ``morphocore.functional.closing``
    (morphocore/functional/closing.py:6-101); see :func:`morphocore_amd.functional.opening` (fused when
    both stages merge per channel).
    """
    if channel_merge_mode == 'identity':
        out = fused_pair(x, w_dilation, w_erosion, DILATION, padding_mode, save_indices, padding_value, weight_dropout, training,
                         noise_scale)
        if out is not None:
            return out
    dilated = dilation(x, w_dilation, channel_merge_mode, padding_mode, save_indices, weight_dropout=weight_dropout, training=training,
                       padding_value=padding_value, noise_scale=noise_scale)
    return erosion(dilated, w_erosion, 'identity', padding_mode, save_indices, weight_dropout=weight_dropout, training=training,
                   padding_value=padding_value, noise_scale=noise_scale)
