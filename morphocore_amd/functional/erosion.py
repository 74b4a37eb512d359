import torch

from ._dropout import drop_weights
from ._ops import ops
from .merge_enum import str_to_merge, str_to_padding


def erosion(x: torch.Tensor, w: torch.Tensor, channel_merge_mode: str = 'sum', padding_mode: str = 'replicate',
            save_indices: bool = True, weight_dropout: float = 0.0, training: bool = False, padding_value: float = 0.0,
            noise_scale: float = 0.0) -> torch.Tensor:
    """Morphological erosion: out[b, o, h, w] = merge_i min_{m, n} (x[b, i, h + m - KH//2, w + n - KW//2] - w[o, i, m, n]).

    Same signature, defaults and semantics as the reference's ``morphocore.functional.erosion``
    (morphocore/functional/erosion.py:5-91): the operator receives the flipped structuring element,
    so that the tap rule of the kernels reads the window in correlation order. Parameters as in
    :func:`morphocore_amd.functional.dilation`; 'geodesic' padding reads +inf here.
    """
    if training and weight_dropout > 0.0:
        # The reference's draws and one-survivor rule, in its order (dilation.py:78-87), so that seeded
        # runs drop the same taps; one host synchronisation instead of one per channel pair.
        w = drop_weights(w, weight_dropout)

    return ops.erosion(x, w.flip((-2, -1)), str_to_merge(channel_merge_mode), str_to_padding(padding_mode), padding_value,
                       save_indices, noise_scale if training else 0.0)
