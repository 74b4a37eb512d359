import torch
import torch.nn as nn

from ..functional._pair import EROSION, fused_pair
from .dilation import Dilation
from .erosion import Erosion
from ._plain import calls_forward_plainly

_SHARED = ('padding_mode', 'padding_value', 'save_indices', 'weight_dropout', 'noise_scale', 'training')


class Opening(nn.Module):
    """Learnable morphological opening (reference: morphocore/nn/opening.py:9-180): an erosion, then a
    per-channel ('identity') dilation.

    ``Opening(in_channels, out_channels, kernel_size, channel_merge_mode=None, padding_mode='replicate',
    dtype=torch.float32, save_indices=True, padding_value=0.0, share_weights=True, weight_dropout=0.0,
    noise_scale=0.0)``. With ``share_weights`` (the default) both stages use one structuring element,
    which makes the layer an algebraic opening (anti-extensive and idempotent with geodesic padding); it needs in_channels == out_channels and
    forces the 'identity' merge. ``share_weights=False`` gives the two stages independent parameters
    and lets the first one merge channels ('sum' by default).
    """

    def __init__(self, in_channels: int, out_channels: int, kernel_size, channel_merge_mode: str = None, padding_mode: str = "replicate",
                 dtype: torch.dtype = torch.float32, save_indices: bool = True, padding_value: float = 0.0, share_weights: bool = True,
                 weight_dropout: float = 0.0, noise_scale: float = 0.0):
        super().__init__()
        if type(kernel_size) is int:
            kernel_size = (kernel_size, kernel_size)
        if share_weights:
            if in_channels != out_channels:
                raise ValueError(
                    f"share_weights=True needs in_channels == out_channels, got {in_channels} and "
                    f"{out_channels}. Pass share_weights=False for two independent structuring elements."
                )
            if channel_merge_mode not in (None, 'identity'):
                raise ValueError(
                    f"share_weights=True forces channel_merge_mode='identity', got "
                    f"'{channel_merge_mode}'. Pass share_weights=False to merge channels instead."
                )
            channel_merge_mode = 'identity'
        elif channel_merge_mode is None:
            channel_merge_mode = 'sum'
        self.share_weights = share_weights
        common = dict(kernel_size=kernel_size, padding_mode=padding_mode, padding_value=padding_value, weight_dropout=weight_dropout,
                      noise_scale=noise_scale, dtype=dtype, save_indices=save_indices)
        self.erosion = Erosion(in_channels=in_channels, out_channels=out_channels, channel_merge_mode=channel_merge_mode, **common)
        self.dilation = Dilation(in_channels=out_channels, out_channels=out_channels, channel_merge_mode='identity', **common)
        if share_weights:
            self.dilation.weight = self.erosion.weight

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # Both stages per channel with the same settings: one fused operator call (same values and draws),
        # unless a hook or an override of a sub-module's forward expects the two calls.
        a, b = self.erosion, self.dilation
        if (a.channel_merge_mode == 'identity' and all(getattr(a, k) == getattr(b, k) for k in _SHARED)
                and calls_forward_plainly(a, Erosion) and calls_forward_plainly(b, Dilation)):
            out = fused_pair(x, a.weight, b.weight, EROSION, a.padding_mode, a.save_indices, a.padding_value, a.weight_dropout, a.training,
                             a.noise_scale)
            if out is not None:
                return out
        return b(a(x))
