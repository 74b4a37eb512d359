import torch

from ._ops import ops
from .merge_enum import str_to_merge


def w_tilde(w: torch.Tensor, alpha: torch.Tensor, channel_merge_mode: str = "sum") -> torch.Tensor:
    """The element the smorph operator receives: w blended with its flip by tanh(alpha), per pair,
    w~ = tanh(a) * ((1 - tanh(a)) / 2 * flip(w) + (1 + tanh(a)) / 2 * w), in torch operations so that
    autograd carries w~'s gradient back to w and alpha (morphocore/functional/smorph.py:56-70)."""
    if channel_merge_mode == 'identity' or alpha.dim() == 1:
        tanh_alpha = torch.tanh(alpha).view(-1, 1, 1, 1)
    else:
        tanh_alpha = torch.tanh(alpha).unsqueeze(-1).unsqueeze(-1)

    term1 = (1 + tanh_alpha) / 2
    term2 = (1 - tanh_alpha) / 2
    return tanh_alpha * (term2 * w.flip(dims=(-2, -1)) + term1 * w)


def smorph(x: torch.Tensor, w: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor = None,
           channel_merge_mode: str = "sum") -> torch.Tensor:
    """Smooth morphology: an alpha-softmax over each window, dilation-like for alpha -> +inf and
    erosion-like for alpha -> -inf.

    Same signature and semantics as the reference's ``morphocore.functional.smorph``
    (morphocore/functional/smorph.py:6-75). The structuring element is first blended with its flip,
    w~ = tanh(a) * ((1 - tanh(a)) / 2 * flip(w) + (1 + tanh(a)) / 2 * w), with torch operations (so
    that autograd carries the gradient of w~ back to w and alpha), then for every channel pair and
    output pixel, over the taps that read an in-image pixel (v = x + w~):
    out = sum_k exp(a (v_k - ref)) v_k / sum_k exp(a (v_k - ref)), ref = max v (a >= 0) or min v.

    Parameters
    ----------
    x : [N, C_in, H, W] input on a HIP device, float32 or float64.
    w : [C_out, C_in, K_h, K_w] structuring element ([C, 1, K_h, K_w] for 'identity').
    alpha : [C_out, C_in] (or [C_out] / [C, 1] for 'identity'), or a single value shared by all pairs.
    beta : [C_out], one value per output channel: selects the SMOOTH channel merge (the smorph_scm
        operator), a soft extremum of the pair outputs with temperature beta (max-like for beta > 0,
        min-like for beta < 0, their mean at 0); ``channel_merge_mode`` is then ignored.
    channel_merge_mode : 'sum', 'mean', 'max', 'min' or 'identity'.
    """
    w_tilde_alpha = w_tilde(w, alpha, channel_merge_mode)
    if beta is not None:
        return ops.smorph_scm(x, w_tilde_alpha, alpha, beta)
    return ops.smorph(x, w_tilde_alpha, alpha, str_to_merge(channel_merge_mode))
