import torch
import torch.nn as nn

from ..functional import smorph
from .alpha_module import AlphaModule


class SMorph(AlphaModule):
    """Learnable smooth morphological layer (reference: morphocore/nn/smorph.py:6-112).

    ``SMorph(in_channels, out_channels, kernel_size, channel_merge_mode='sum', init_alpha=0.0,
    dtype=torch.float32, init_beta=None)``: parameters ``weight`` (zeros), ``alpha`` (``init_alpha``)
    and, when ``init_beta`` is given, ``beta`` of shape (out_channels, in_channels), which selects the
    SMOOTH channel merge (the smorph_scm operator). As in the reference, the operator takes one beta per
    output channel, so that shape runs only with in_channels == 1 (other widths raise "Beta must have
    shape [out_channels]"); :func:`morphocore_amd.functional.smorph` takes a [C_out] beta directly.
    Forward: :func:`morphocore_amd.functional.smorph`.
    """

    def __init__(self, in_channels: int, out_channels: int, kernel_size: tuple, channel_merge_mode: str = "sum",
                 init_alpha: float = 0.0, dtype: torch.dtype = torch.float32, init_beta: float = None):
        if type(kernel_size) is int:
            kernel_size = (kernel_size, kernel_size)
        super(SMorph, self).__init__(in_channels, out_channels, kernel_size, channel_merge_mode, init_alpha, dtype)
        if init_beta is not None:
            self.beta = nn.Parameter(torch.full((out_channels, in_channels), init_beta, dtype=dtype))
        else:
            self.beta = None

    def forward(self, x: torch.Tensor):
        return smorph(x=x, w=self.weight, alpha=self.alpha, beta=self.beta, channel_merge_mode=self.channel_merge_mode)
