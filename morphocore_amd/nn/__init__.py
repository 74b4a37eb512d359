"""Layers (reference: morphocore/nn/__init__.py)."""
from .dilation import Dilation
from .erosion import Erosion
from .smorph import SMorph
from .morpho_module import MorphoModule
from .alpha_module import AlphaModule

__all__ = ['Dilation', 'Erosion', 'SMorph', 'MorphoModule', 'AlphaModule']
