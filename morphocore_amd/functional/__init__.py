"""Functional operators (reference: morphocore/functional/__init__.py)."""
from .dilation import dilation
from .erosion import erosion
from .opening import opening
from .closing import closing
from .sigma_layer import sigma_layer
from .smorph import smorph
from .stack import morpho_stack
from .merge_enum import MorphoMerge, MorphoPadding, str_to_merge, str_to_padding
from ._ops import ops

__all__ = ['dilation', 'erosion', 'opening', 'closing', 'sigma_layer', 'smorph', 'morpho_stack', 'MorphoMerge', 'MorphoPadding', 'str_to_merge',
           'str_to_padding', 'ops']
