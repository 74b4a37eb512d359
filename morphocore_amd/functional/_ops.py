"""Loads the PyTorch-ROCm extension ``morphocore_amd._C``, which registers the operators with torch's
dispatcher as ``torch.ops.morphocore.<name>``.

Same namespace, names and schemas as the reference (morphocore/functional/csrc/cpp/bindings.cpp:130-138),
registered for ``CompositeImplicitAutograd`` like the reference (bindings.cpp:142-148): the C++
kernels run above autograd for every device and record their own backward through C++ autograd
Functions (morphocore_amd/csrc/torch_ops.cpp), whose device work is the gfx950 HIP library. Call sites
written against the reference's ``ops`` (morphocore/functional/_ops.py:6) work unchanged. A missing
extension is an error, never a fallback.
"""
import torch

try:
    from .. import _C  # noqa: F401  (loading the library runs the registrations)
except ImportError as exc:  # pragma: no cover - depends on the build
    raise RuntimeError(
        "morphocore_amd: the native extension morphocore_amd._C is not built; build it with "
        "`python setup.py build_ext --inplace` (or `python -c 'import __graft_entry__ as g; g.build()'`)"
    ) from exc

ops = torch.ops.morphocore
