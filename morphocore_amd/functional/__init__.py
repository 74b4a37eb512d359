"""Functional operators (reference: morphocore/functional/__init__.py)."""
from .dilation import dilation
from .erosion import erosion
from .smorph import smorph
from .merge_enum import MorphoMerge, MorphoPadding, str_to_merge, str_to_padding
from ._ops import ops

__all__ = ['dilation', 'erosion', 'smorph', 'MorphoMerge', 'MorphoPadding', 'str_to_merge', 'str_to_padding', 'ops']
