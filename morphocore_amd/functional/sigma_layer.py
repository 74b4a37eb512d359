import torch

from ._dropout import drop_weights
from ._ops import ops
from .dilation import dilation
from .erosion import erosion
from .merge_enum import str_to_padding


def sigma_layer(x: torch.Tensor, w: torch.Tensor, alpha: torch.Tensor, channel_merge_mode: str = 'sum', padding_mode: str = 'replicate',
                save_indices: bool = True, padding_value: float = 0.0, weight_dropout: float = 0.0, training: bool = False,
                noise_scale: float = 0.0) -> torch.Tensor:
    """Interpolation between erosion and dilation with one structuring element:
    Y = sigmoid(a) * dilation(x, w) + (1 - sigmoid(a)) * erosion(x, w), a = alpha.mean(dim=1) per output
    channel.

    Same signature, defaults and semantics as the reference's ``morphocore.functional.sigma_layer``
    (morphocore/functional/sigma_layer.py:7-83): the erosion is evaluated first, then the dilation
    (each with its own dropout mask and noise in training), and the blend is torch code, as there.
    With the 'identity' merge the two operations and the blend run as one fused operator
    (``torch.ops.morphocore.sigma_identity``), with the same values and random draws (dropout and
    noise together in training, whose draws the composition interleaves, run the composition).
    """
    drop = training and weight_dropout > 0.0
    noise = noise_scale if training else 0.0
    if channel_merge_mode == 'identity' and not (drop and noise > 0.0) and alpha.dtype == x.dtype == w.dtype:
        soft = torch.sigmoid(alpha.mean(dim=1))
        w_e = drop_weights(w, weight_dropout) if drop else w
        w_d = drop_weights(w, weight_dropout) if drop else w
        return ops.sigma_identity(x, w_e.flip((-2, -1)), w_d, soft, str_to_padding(padding_mode), padding_value, save_indices, noise)
    out_erosion = erosion(x, w, channel_merge_mode=channel_merge_mode, padding_mode=padding_mode, save_indices=save_indices,
                          padding_value=padding_value, weight_dropout=weight_dropout, training=training, noise_scale=noise_scale)
    out_dilation = dilation(x, w, channel_merge_mode=channel_merge_mode, padding_mode=padding_mode, save_indices=save_indices,
                            padding_value=padding_value, weight_dropout=weight_dropout, training=training, noise_scale=noise_scale)
    soft = torch.sigmoid(alpha.mean(dim=1))
    soft = soft.view(1, -1, 1, 1)
    return out_erosion * (1.0 - soft) + out_dilation * soft
