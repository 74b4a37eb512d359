"""Channel-merge and padding modes: string names to the integer codes the operators take.

Same names, values and errors as the reference (morphocore/functional/merge_enum.py:4-70), which
shares the values with morpho_op_enum.hpp:17-35.
"""
from enum import IntEnum


class MorphoMerge(IntEnum):
    """How the per-input-channel results of one output channel are combined."""
    MAX = 0
    MIN = 1
    ADD = 2
    AVERAGE = 3
    SMOOTH = 4
    IDENTITY = 5


class MorphoPadding(IntEnum):
    """What a tap reads outside the image."""
    ZERO = 0
    GEODESIC = 1
    CONSTANT = 2
    REPLICATE = 3


_MERGE_MODES = {
    "max": MorphoMerge.MAX,
    "min": MorphoMerge.MIN,
    "sum": MorphoMerge.ADD,
    "mean": MorphoMerge.AVERAGE,
    "identity": MorphoMerge.IDENTITY,
}

_PADDING_MODES = {
    "zero": MorphoPadding.ZERO,
    "geodesic": MorphoPadding.GEODESIC,
    "constant": MorphoPadding.CONSTANT,
    "replicate": MorphoPadding.REPLICATE,
}


def str_to_merge(mode: str) -> MorphoMerge:
    """'max', 'min', 'sum', 'mean' or 'identity' to its MorphoMerge; ValueError otherwise."""
    try:
        return _MERGE_MODES[mode]
    except (KeyError, TypeError):
        raise ValueError(f"Unknown merge mode: {mode}") from None


def str_to_padding(mode: str) -> MorphoPadding:
    """'zero', 'geodesic', 'constant' or 'replicate' to its MorphoPadding; ValueError otherwise."""
    try:
        return _PADDING_MODES[mode]
    except (KeyError, TypeError):
        raise ValueError(f"Unknown padding mode: {mode}. Expected one of {sorted(_PADDING_MODES)}.") from None
