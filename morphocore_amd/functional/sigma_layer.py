import torch

from .dilation import dilation
from .erosion import erosion


def sigma_layer(x: torch.Tensor, w: torch.Tensor, alpha: torch.Tensor, channel_merge_mode: str = 'sum', padding_mode: str = 'replicate',
                save_indices: bool = True, padding_value: float = 0.0, weight_dropout: float = 0.0, training: bool = False,
                noise_scale: float = 0.0) -> torch.Tensor:
    """Interpolation between erosion and dilation with one structuring element:
    Y = sigmoid(a) * dilation(x, w) + (1 - sigmoid(a)) * erosion(x, w), a = alpha.mean(dim=1) per output
    channel.

    Same signature, defaults and semantics as the reference's ``morphocore.functional.sigma_layer``
    (morphocore/functional/sigma_layer.py:7-83): the erosion is evaluated first, then the dilation
    (each with its own dropout mask and noise in training), and the blend is torch code, as there.
    """
    out_erosion = erosion(x, w, channel_merge_mode=channel_merge_mode, padding_mode=padding_mode, save_indices=save_indices,
                          padding_value=padding_value, weight_dropout=weight_dropout, training=training, noise_scale=noise_scale)
    out_dilation = dilation(x, w, channel_merge_mode=channel_merge_mode, padding_mode=padding_mode, save_indices=save_indices,
                            padding_value=padding_value, weight_dropout=weight_dropout, training=training, noise_scale=noise_scale)
    soft = torch.sigmoid(alpha.mean(dim=1))
    soft = soft.view(1, -1, 1, 1)
    return out_erosion * (1.0 - soft) + out_dilation * soft
