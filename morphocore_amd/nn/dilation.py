import torch

from ..functional import dilation
from .morpho_module import MorphoModule


class Dilation(MorphoModule):
    """Learnable morphological dilation layer (reference: morphocore/nn/dilation.py:6-102).

    ``Dilation(in_channels, out_channels, kernel_size, channel_merge_mode='sum', padding_mode='replicate',
    dtype=torch.float32, save_indices=True, weight_dropout=0.0, padding_value=0.0, noise_scale=0.0)``;
    an int ``kernel_size`` means a square structuring element. The forward pass calls
    :func:`morphocore_amd.functional.dilation` with the module's training flag, so dropout and noise
    apply in training only.
    """

    def __init__(self, in_channels: int, out_channels: int, kernel_size: tuple, channel_merge_mode: str = "sum",
                 padding_mode: str = "replicate", dtype: torch.dtype = torch.float32, save_indices: bool = True,
                 weight_dropout: float = 0.0, padding_value: float = 0.0, noise_scale: float = 0.0):
        if type(kernel_size) is int:
            kernel_size = (kernel_size, kernel_size)
        self.save_indices = save_indices
        self.weight_dropout = weight_dropout
        self.noise_scale = noise_scale
        super().__init__(in_channels, out_channels, kernel_size, channel_merge_mode, padding_mode, dtype=dtype,
                         padding_value=padding_value)

    def forward(self, x):
        return dilation(x, self.weight, self.channel_merge_mode, self.padding_mode, self.save_indices, self.weight_dropout,
                        self.training, self.padding_value, self.noise_scale)
