import torch

from ..functional import sigma_layer
from .alpha_module import AlphaModule


class SigmaLayer(AlphaModule):
    """Learnable interpolation between erosion and dilation (reference: morphocore/nn/sigma_layer.py:6-80).

    ``SigmaLayer(in_channels, out_channels, kernel_size, channel_merge_mode='sum', padding_mode='replicate',
    init_alpha=0.0, dtype=torch.float32, save_indices=True, padding_value=0.0, weight_dropout=0.0,
    noise_scale=0.0)``: parameters ``weight`` and ``alpha`` as :class:`AlphaModule`; the forward is
    :func:`morphocore_amd.functional.sigma_layer` with the module's training flag.
    """

    def __init__(self, in_channels: int, out_channels: int, kernel_size: tuple, channel_merge_mode: str = "sum",
                 padding_mode: str = "replicate", init_alpha: float = 0.0, dtype: torch.dtype = torch.float32, save_indices: bool = True,
                 padding_value: float = 0.0, weight_dropout: float = 0.0, noise_scale: float = 0.0):
        if type(kernel_size) is int:
            kernel_size = (kernel_size, kernel_size)
        super().__init__(in_channels, out_channels, kernel_size, channel_merge_mode, init_alpha, dtype=dtype)
        self.save_indices = save_indices
        self.padding_mode = padding_mode
        self.padding_value = padding_value
        self.weight_dropout = weight_dropout
        self.noise_scale = noise_scale

    def forward(self, x):
        return sigma_layer(x, self.weight, self.alpha, self.channel_merge_mode, padding_mode=self.padding_mode, save_indices=self.save_indices,
                           padding_value=self.padding_value, weight_dropout=self.weight_dropout, training=self.training,
                           noise_scale=self.noise_scale)
