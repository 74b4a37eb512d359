import torch

from ._dropout import drop_weights
from ._ops import ops
from .merge_enum import str_to_merge, str_to_padding


def dilation(x: torch.Tensor, w: torch.Tensor, channel_merge_mode: str = 'sum', padding_mode: str = 'replicate',
             save_indices: bool = True, weight_dropout: float = 0.0, training: bool = False, padding_value: float = 0.0,
             noise_scale: float = 0.0) -> torch.Tensor:
    """Morphological dilation: out[b, o, h, w] = merge_i max_{kh, kw} (x[b, i, h + KH//2 - kh, w + KW//2 - kw] + w[o, i, kh, kw]).

    Same signature, defaults and semantics as the reference's ``morphocore.functional.dilation``
    (morphocore/functional/dilation.py:5-91).

    Parameters
    ----------
    x : input, [N, C_in, H, W] (also [C_in, H, W] or [H, W]); float32 or float64, on a HIP device.
    w : structuring element, [C_out, C_in, K_h, K_w] ([C, 1, K_h, K_w] for 'identity'), or [K_h, K_w].
    channel_merge_mode : 'sum', 'mean', 'max', 'min' or 'identity'.
    padding_mode : 'zero', 'geodesic' (-inf: the border never wins), 'constant' (``padding_value``)
        or 'replicate' (nearest edge pixel).
    save_indices : keep the winning (channel, tap) of 'max' / 'min' merges for the backward pass.
    weight_dropout : in training, probability of setting a tap of the structuring element to -inf;
        at least one tap of every (output, input) pair survives.
    training : dropout and noise apply only when True.
    padding_value : border value of 'constant' padding.
    noise_scale : in training, half width of the uniform noise added to a per-sample copy of ``w``.

    Returns
    -------
    torch.Tensor of shape [N, C_out, H, W] (the input's rank is kept).
    """
    if training and weight_dropout > 0.0:
        # The reference's draws and one-survivor rule, in its order (dilation.py:78-87), so that seeded
        # runs drop the same taps; one host synchronisation instead of one per channel pair.
        w = drop_weights(w, weight_dropout)

    return ops.dilation(x, w, str_to_merge(channel_merge_mode), str_to_padding(padding_mode), padding_value, save_indices,
                        noise_scale if training else 0.0)
