"""Registers the operators with torch's dispatcher as ``torch.ops.morphocore.<name>``.

Same namespace, names and schemas as the reference (morphocore/functional/csrc/cpp/bindings.cpp:130-138),
registered for ``CompositeImplicitAutograd`` like the reference (bindings.cpp:142-148): the kernel runs
above autograd for every device and records its own backward through the autograd Functions in
``_autograd``. Call sites written against the reference's ``ops`` (morphocore/functional/_ops.py:6)
work unchanged.
"""
import torch

from . import _autograd

_SCHEMAS = {
    "dilation": "dilation(Tensor input, Tensor weight, int merge, int padding, float padding_value=0., bool save_indices=True, "
                "float noise_scale=0.) -> Tensor",
    "erosion": "erosion(Tensor input, Tensor weight, int merge, int padding, float padding_value=0., bool save_indices=True, "
               "float noise_scale=0.) -> Tensor",
    "smorph": "smorph(Tensor input, Tensor weight, Tensor alpha, int merge) -> Tensor",
    "smorph_scm": "smorph_scm(Tensor input, Tensor weight, Tensor alpha, Tensor beta) -> Tensor",
}


def _dilation(input, weight, merge, padding, padding_value=0.0, save_indices=True, noise_scale=0.0):
    return _autograd.morpho_operation(_autograd.DILATION, input, weight, merge, padding, padding_value, save_indices, noise_scale)


def _erosion(input, weight, merge, padding, padding_value=0.0, save_indices=True, noise_scale=0.0):
    return _autograd.morpho_operation(_autograd.EROSION, input, weight, merge, padding, padding_value, save_indices, noise_scale)


def _smorph(input, weight, alpha, merge):
    return _autograd.smorph_operation(input, weight, alpha, merge)


def _smorph_scm(input, weight, alpha, beta):
    return _autograd.smorph_scm_operation(input, weight, alpha, beta)


_LIBRARY = torch.library.Library("morphocore", "DEF")
for _name, _schema in _SCHEMAS.items():
    _LIBRARY.define(_schema)
_LIBRARY.impl("dilation", _dilation, "CompositeImplicitAutograd")
_LIBRARY.impl("erosion", _erosion, "CompositeImplicitAutograd")
_LIBRARY.impl("smorph", _smorph, "CompositeImplicitAutograd")
_LIBRARY.impl("smorph_scm", _smorph_scm, "CompositeImplicitAutograd")

ops = torch.ops.morphocore
