import torch

from ._pair import EROSION, fused_pair
from .dilation import dilation
from .erosion import erosion


def opening(x: torch.Tensor, w_erosion: torch.Tensor, w_dilation: torch.Tensor, channel_merge_mode: str = 'sum',
            padding_mode: str = 'replicate', save_indices: bool = True, padding_value: float = 0.0, weight_dropout: float = 0.0,
            training: bool = False, noise_scale: float = 0.0) -> torch.Tensor:
    """Morphological opening: an erosion, then a per-channel ('identity') dilation of its output.

    Same signature, defaults and semantics as the reference's ``morphocore.functional.opening``
    (morphocore/functional/opening.py:6-101): the erosion merges channels with ``channel_merge_mode``
    (w_erosion: [C_mid, C_in, K_h, K_w]), the dilation always uses 'identity' (w_dilation:
    [C_mid, 1, K_h, K_w]); both stages use the same padding, and in training each stage draws its own
    dropout mask and noise. When both stages merge per channel ('identity') the two run as one fused
    operator (``torch.ops.morphocore.opening_closing``), with the same values and random draws.
    """
    if channel_merge_mode == 'identity':
        out = fused_pair(x, w_erosion, w_dilation, EROSION, padding_mode, save_indices, padding_value, weight_dropout, training,
                         noise_scale)
        if out is not None:
            return out
    eroded = erosion(x, w_erosion, channel_merge_mode, padding_mode, save_indices, weight_dropout=weight_dropout, training=training,
                     padding_value=padding_value, noise_scale=noise_scale)
    return dilation(eroded, w_dilation, 'identity', padding_mode, save_indices, weight_dropout=weight_dropout, training=training,
                    padding_value=padding_value, noise_scale=noise_scale)
