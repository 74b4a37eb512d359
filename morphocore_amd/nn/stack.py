import torch
import torch.nn as nn

from ..functional import morpho_stack
from ._plain import calls_forward_plainly
from .dilation import Dilation
from .erosion import Erosion
from .smorph import SMorph


class MorphoStack(nn.Module):
    """A chain of Dilation / Erosion / SMorph layers run as one operator
    (:func:`morphocore_amd.functional.morpho_stack`). No reference counterpart: the reference chains such
    layers as separate modules (e.g. in ``nn.Sequential``), one operator call per layer.

    ``MorphoStack(*layers, chunk=0)``: the layers are ordinary ``Dilation``, ``Erosion`` and ``SMorph``
    modules (registered as ``layers``, so their parameters and state_dict entries are the layers' own).
    The forward pass gives the values of calling the layers in turn. A layer that a stack does not take
    (weight dropout or weight noise in training, SMorph's SMOOTH merge with ``beta``), or one whose call
    would run more than its class's forward (a hook, a subclass or an instance override of ``forward``),
    makes the forward call the layers one by one instead.
    """

    def __init__(self, *layers: nn.Module, chunk: int = 0):
        super().__init__()
        for layer in layers:
            if not isinstance(layer, (Dilation, Erosion, SMorph)):
                raise TypeError(f"MorphoStack takes Dilation, Erosion and SMorph layers, not {type(layer).__name__}")
        if not layers:
            raise ValueError("MorphoStack needs at least one layer")
        self.layers = nn.ModuleList(layers)
        self.chunk = chunk

    def _stackable(self) -> bool:
        for layer in self.layers:
            if not any(calls_forward_plainly(layer, cls) for cls in (Dilation, Erosion, SMorph)):
                return False
            if isinstance(layer, SMorph):
                if layer.beta is not None:
                    return False
            elif self.training and (layer.weight_dropout > 0.0 or layer.noise_scale > 0.0):
                return False
        return True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._stackable():
            for layer in self.layers:
                x = layer(x)
            return x
        specs = []
        save = True
        for layer in self.layers:
            if isinstance(layer, SMorph):
                specs.append(("smorph", layer.weight, layer.alpha, layer.channel_merge_mode))
            else:
                kind = "dilation" if isinstance(layer, Dilation) else "erosion"
                specs.append((kind, layer.weight, layer.channel_merge_mode, layer.padding_mode, layer.padding_value))
                save = save and layer.save_indices
        return morpho_stack(x, specs, save_indices=save, chunk=self.chunk)
