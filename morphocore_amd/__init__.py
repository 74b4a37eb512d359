"""morphocore_amd: morphocore's operator hot path (dilation, erosion, smorph) as hand-written HIP
kernels for AMD Instinct MI355X (gfx950), behind the reference package's Python API.

``morphocore_amd.functional`` and ``morphocore_amd.nn`` mirror ``morphocore.functional`` and
``morphocore.nn`` (reference: morphocore/functional/__init__.py, morphocore/nn/__init__.py); the
operators are registered as ``torch.ops.morphocore.{dilation,erosion,smorph}`` with the reference's
schemas (reference: morphocore/functional/csrc/cpp/bindings.cpp:130-138).
"""

__version__ = "0.13.1"

from . import functional, nn  # noqa: E402,F401
