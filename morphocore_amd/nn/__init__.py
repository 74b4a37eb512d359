"""Layers (reference: morphocore/nn/__init__.py)."""
from .dilation import Dilation
from .erosion import Erosion
from .opening import Opening
from .closing import Closing
from .sigma_layer import SigmaLayer
from .smorph import SMorph
from .stack import MorphoStack
from .morpho_module import MorphoModule
from .alpha_module import AlphaModule

__all__ = ['Dilation', 'Erosion', 'Opening', 'Closing', 'SigmaLayer', 'SMorph', 'MorphoStack', 'MorphoModule', 'AlphaModule']
