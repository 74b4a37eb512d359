"""When a composed layer may replace its two sub-module calls by one fused operator call."""
import torch.nn as nn
from torch.nn.modules import module as _module

_HOOKS = ("_forward_hooks", "_forward_pre_hooks", "_backward_hooks", "_backward_pre_hooks")
_GLOBAL_HOOKS = ("_global_forward_hooks", "_global_forward_pre_hooks", "_global_backward_hooks", "_global_backward_pre_hooks")


def calls_forward_plainly(m: nn.Module, cls: type) -> bool:
    """Whether ``m(x)`` would run nothing but ``cls.forward``: ``m`` is exactly a ``cls`` (no subclass
    override, no ``forward`` set on the instance) and no module hook, its own or a global one, is
    registered. Otherwise the layer calls its sub-modules, as the reference's nn.Opening / nn.Closing
    always do (reference: morphocore/nn/opening.py:162-180)."""
    if type(m) is not cls or "forward" in m.__dict__:
        return False
    if any(getattr(m, h, None) for h in _HOOKS):
        return False
    return not any(getattr(_module, h, None) for h in _GLOBAL_HOOKS)
