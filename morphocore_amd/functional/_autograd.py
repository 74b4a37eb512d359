"""Host side of the operators: argument checks, rank handling, weight noise, and the autograd
Functions that call the native HIP kernels.

This is the Python restatement of the reference's C++ host layer:
``MorphoOperation<op, merge, kind>::forward/backward`` (morphocore/functional/csrc/cpp/morpho_op_wrap.hxx:24-211),
``Smorph<merge>::forward/backward`` (smorph.cpp:20-111), the int checks of bindings.cpp:15-27 and the
rank handling of reshaper.cpp:3-151. Same checks, same messages (raised as RuntimeError, which is what
a TORCH_CHECK becomes in Python), same saved state. The arithmetic runs only in the native library.
"""
from __future__ import annotations

import os

import torch

from .. import _native
from .merge_enum import MorphoMerge, MorphoPadding

DILATION, EROSION = 0, 1

# Max / min winners are saved only while the reference's CUDA grid could address every (batch,
# output channel) pair (morpho_op_wrap.hxx:65-66).
_MAX_GRID_DIM = 65535

# The per-pair taps of the sum / mean / identity merges (one byte per channel pair and output
# pixel) are kept for the backward pass up to this many bytes per call; beyond it the backward
# recomputes them. MORPHOCORE_AMD_SAVED_TAPS_LIMIT overrides it (bytes, 0 disables saving).
_SAVED_TAPS_LIMIT = int(os.environ.get("MORPHOCORE_AMD_SAVED_TAPS_LIMIT", 8 << 30))


def _should_save(merge: MorphoMerge, save_indices: bool, needs_grad: bool, B: int, Cout: int, nbytes: int) -> bool:
    """Whether the forward keeps its winners for the backward. The result never depends on it."""
    if not (save_indices and needs_grad):
        return False
    if merge in (MorphoMerge.MAX, MorphoMerge.MIN):
        return Cout * B < _MAX_GRID_DIM
    return nbytes <= _SAVED_TAPS_LIMIT


def _save_smorph_stats(nbytes: int, needs_grad: bool, device) -> bool:
    """Whether the smorph forward keeps its pair statistics (12 bytes per channel pair and output
    pixel; float32 with a 3x3, 5x5, 7x7 or 11x11 element) so that the backward need not recompute
    them: when they take at most half of the device memory still available (free, plus what torch's
    allocator holds unused). MORPHOCORE_AMD_SAVED_STATS_LIMIT caps them further (bytes, 0 disables
    saving). The result never depends on it."""
    if not needs_grad or nbytes <= 0:
        return False
    limit = os.environ.get("MORPHOCORE_AMD_SAVED_STATS_LIMIT")
    if limit is not None and nbytes > int(limit):
        return False
    free, _ = torch.cuda.mem_get_info(device)
    avail = free + torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
    return nbytes <= avail // 2


def to_merge(merge: int) -> MorphoMerge:
    """bindings.cpp:16-20."""
    merge = int(merge)
    if not (0 <= merge <= int(MorphoMerge.IDENTITY)):
        raise RuntimeError(f"Unknown merge mode {merge}")
    return MorphoMerge(merge)


def to_padding(padding: int) -> MorphoPadding:
    """bindings.cpp:23-27."""
    padding = int(padding)
    if not (0 <= padding <= int(MorphoPadding.REPLICATE)):
        raise RuntimeError(f"Unknown padding mode {padding}")
    return MorphoPadding(padding)


def fill_value(op: int, padding: MorphoPadding, padding_value: float) -> float:
    """Border value of the fill paddings (morpho_padding_policy.hpp:22-33): ZERO 0, CONSTANT the
    value, GEODESIC the identity element of the operation (-inf dilation, +inf erosion).
    REPLICATE reads the clamped edge pixel instead and ignores this value."""
    if padding == MorphoPadding.ZERO:
        return 0.0
    if padding == MorphoPadding.CONSTANT:
        return float(padding_value)
    if padding == MorphoPadding.GEODESIC:
        return float("-inf") if op == DILATION else float("inf")
    return 0.0


def input_to_4d(t: torch.Tensor) -> torch.Tensor:
    """TensorInputDim::To4DTensor (reshaper.cpp:3-55): [H, W] and [C, H, W] gain leading unit axes."""
    d = t.dim()
    if d == 4:
        return t
    if d == 3:
        return t.unsqueeze(0)
    if d == 2:
        return t.unsqueeze(0).unsqueeze(0)
    raise RuntimeError(f"Invalid input tensor: please give a 2D, 3D or 4D input tensor, received: {d} dimensions !")


def output_to_original(out: torch.Tensor, input_dims: int) -> torch.Tensor:
    """TensorInputDim::ToOriginalTensor (reshaper.cpp:57-81): undo the leading unit axes."""
    if input_dims == 3:
        return out.squeeze(0)
    if input_dims == 2:
        return out.squeeze(0).squeeze(0)
    return out


def weight_to_4d(t: torch.Tensor) -> torch.Tensor:
    """TensorWeightDim::To4DTensor (reshaper.cpp:84-130): a [KH, KW] weight is one pair."""
    d = t.dim()
    if d == 4:
        return t
    if d == 2:
        return t.unsqueeze(0).unsqueeze(0)
    raise RuntimeError(f"Invalid weight tensor dimensions: expected 2D, 3D, 4D or 5D tensor, received {d}D tensor")


def _check_4d(x4: torch.Tensor, w4: torch.Tensor) -> None:
    if x4.dim() != 4:
        raise RuntimeError("Input must be a 4d tensor (batch_size, in_channels, height, width)")
    if w4.dim() != 4:
        raise RuntimeError("Weight must be a 4d tensor (out_channels, in_channels, kernel_height, kernel_width)")


def _check_identity(x4: torch.Tensor, w4: torch.Tensor, smorph: bool) -> None:
    if w4.shape[0] != x4.shape[1]:
        raise RuntimeError("Identity mode requires weight.shape[0] == input.shape[1]")
    if w4.shape[1] != 1:
        raise RuntimeError("Identity mode requires weight.shape[1] == 1" + (f", got {w4.shape[1]}" if smorph else ""))


def _check_device(x4: torch.Tensor, *others: torch.Tensor, name: str) -> None:
    """The product path runs only on a HIP device; a CPU tensor is an error, never a fallback."""
    if not x4.is_cuda:
        raise RuntimeError(f"morphocore_amd: {name} runs on AMD GPUs (HIP devices); got an input on {x4.device}")
    if x4.dtype not in (torch.float32, torch.float64):
        raise RuntimeError(f'"{name}" not implemented for \'{str(x4.dtype).replace("torch.", "").capitalize()}\'')
    for t in others:
        if t.device != x4.device:
            raise RuntimeError(f"morphocore_amd: {name} expects every tensor on {x4.device}, got one on {t.device}")
        if t.dtype != x4.dtype:
            raise RuntimeError(f"expected scalar type {_scalar_name(x4.dtype)} but found {_scalar_name(t.dtype)}")


def _scalar_name(dtype: torch.dtype) -> str:
    return {torch.float32: "Float", torch.float64: "Double", torch.float16: "Half", torch.bfloat16: "BFloat16"}.get(dtype, str(dtype))


def _geom(x4: torch.Tensor, w4: torch.Tensor):
    B, Cin, H, W = x4.shape
    Cout, Cw, KH, KW = w4.shape
    return (int(B), int(Cin), int(Cout), int(Cw), int(H), int(W), int(KH), int(KW))


class _MorphoFunction(torch.autograd.Function):
    """MorphoOperation<op, merge, kind> (morpho_op_wrap.hxx:24-211) on 4-D, checked arguments."""

    @staticmethod
    def forward(ctx, x4, w4, op, merge, padding, padding_value, save_indices, noise_scale, needs_grad):
        geom = _geom(x4, w4)
        B, Cin, Cout, Cw, H, W, KH, KW = geom
        x4c = x4.contiguous()
        w4c = w4.contiguous()
        # Weight noise: one structuring element per batch element, drawn on the weight's device from
        # its generator exactly as morpho_op_wrap.hxx:55-64 draws it.
        sample_weight = None
        if noise_scale > 0.0:
            noise = (torch.rand((B, Cout, Cw, KH, KW), dtype=w4c.dtype, device=w4c.device) * 2.0 - 1.0) * noise_scale
            sample_weight = (w4c.unsqueeze(0) + noise).contiguous()
        kernel_weight = sample_weight if sample_weight is not None else w4c
        wbs = Cout * Cw * KH * KW if sample_weight is not None else 0
        nbytes = _native.indices_bytes(int(merge), geom)
        should_save = _should_save(merge, bool(save_indices), needs_grad, B, Cout, nbytes)
        out = torch.empty((B, Cout, H, W), dtype=x4c.dtype, device=x4c.device)
        # Layout per mca_morpho_indices_bytes: packed int32 winners (max / min) or per-pair taps.
        indices = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x4c.device) if should_save else None
        replicate = padding == MorphoPadding.REPLICATE
        fill = fill_value(op, padding, padding_value)
        _native.morpho_forward(op, int(merge), replicate, fill, x4c, kernel_weight, wbs, out, indices, geom)
        ctx.save_for_backward(x4c, w4c, indices, sample_weight)
        ctx.op, ctx.merge, ctx.padding, ctx.padding_value = op, int(merge), padding, padding_value
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x4, w4, indices, sample_weight = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        expected = list(x4.shape)
        expected[1] = w4.shape[0]
        if list(grad_output.shape) != expected:
            raise RuntimeError(f"grad_output shape mismatch: expected [{expected}] but got [{list(grad_output.shape)}]")
        if grad_output.device != x4.device:
            raise RuntimeError("grad_output must be on the same device as input")
        if grad_output.dtype != x4.dtype:
            raise RuntimeError("grad_output must have the same dtype as input")
        geom = _geom(x4, w4)
        B, Cin, Cout, Cw, H, W, KH, KW = geom
        kernel_weight = sample_weight if sample_weight is not None else w4
        wbs = Cout * Cw * KH * KW if sample_weight is not None else 0
        grad_input = torch.empty_like(x4)
        grad_weight = torch.empty_like(w4)
        replicate = ctx.padding == MorphoPadding.REPLICATE
        fill = fill_value(ctx.op, ctx.padding, ctx.padding_value)
        _native.morpho_backward(ctx.op, ctx.merge, replicate, fill, x4, kernel_weight, wbs, indices, grad_output, grad_input, grad_weight,
                                geom)
        return grad_input, grad_weight, None, None, None, None, None, None, None


def morpho_operation(op: int, input: torch.Tensor, weight: torch.Tensor, merge: int, padding: int, padding_value: float = 0.0,
                     save_indices: bool = True, noise_scale: float = 0.0) -> torch.Tensor:
    """Body of the ``dilation`` / ``erosion`` operators: bindings.cpp:59-101 then
    MorphoOperation::forward's checks (morpho_op_wrap.hxx:24-77)."""
    padding = to_padding(padding)
    merge = to_merge(merge)
    if merge == MorphoMerge.SMOOTH:
        raise RuntimeError("Unsupported merge operation")
    if not noise_scale >= 0.0:
        raise RuntimeError("noise_scale must be non negative")
    input_dims = input.dim()
    x4 = input_to_4d(input)
    w4 = weight_to_4d(weight)
    _check_4d(x4, w4)
    if x4.shape[1] != w4.shape[1] and merge != MorphoMerge.IDENTITY:
        raise RuntimeError("Input channels must match weight input channels")
    if merge == MorphoMerge.IDENTITY:
        _check_identity(x4, w4, smorph=False)
    _check_device(x4, w4, name="morpho_operation_forward_hip")
    needs_grad = torch.is_grad_enabled() and (input.requires_grad or weight.requires_grad)
    out = _MorphoFunction.apply(x4, w4, op, merge, padding, float(padding_value), bool(save_indices), float(noise_scale), needs_grad)
    return output_to_original(out, input_dims)


def smorph_pair_alphas(alpha: torch.Tensor, merge: MorphoMerge, Cin: int, Cout: int) -> torch.Tensor:
    """One alpha per channel pair, index o * Cin + i ([Cout] for IDENTITY), or one shared value
    broadcast to every pair (smorph_cpu_kernels.hxx:642-649)."""
    pairs = Cout if merge == MorphoMerge.IDENTITY else Cout * Cin
    if alpha.numel() != pairs and alpha.numel() != 1:
        shape = "[channels]" if merge == MorphoMerge.IDENTITY else "[out_channels, in_channels]"
        raise RuntimeError(f"Alpha must have one value, or shape {shape}")
    if alpha.numel() == pairs:
        return alpha.contiguous().reshape(pairs)
    return alpha.reshape(1).expand(pairs).contiguous()


class _SmorphFunction(torch.autograd.Function):
    """Smorph<merge> (smorph.cpp:20-111) on 4-D, checked arguments; `w4` is the blended w~."""

    @staticmethod
    def forward(ctx, x4, w4, alpha, merge, needs_grad):
        geom = _geom(x4, w4)
        B, Cin, Cout, Cw, H, W, KH, KW = geom
        x4c = x4.contiguous()
        w4c = w4.contiguous()
        alpha_pairs = smorph_pair_alphas(alpha, merge, Cin, Cout)
        out = torch.empty((B, Cout, H, W), dtype=x4c.dtype, device=x4c.device)
        stats = None
        nbytes = _native.smorph_stats_bytes(int(merge), x4c.dtype, geom)
        if _save_smorph_stats(nbytes, needs_grad, x4c.device):
            try:
                stats = torch.empty(nbytes // 4, dtype=torch.float32, device=x4c.device)
            except torch.cuda.OutOfMemoryError:
                stats = None  # fragmented memory: the backward recomputes them
        _native.smorph_forward(int(merge), x4c, w4c, alpha_pairs, out, geom, stats=stats)
        ctx.save_for_backward(out, alpha, x4c, w4c, stats)
        ctx.merge = merge
        return out

    @staticmethod
    def backward(ctx, grad_output):
        out, alpha, x4, w4, stats = ctx.saved_tensors
        geom = _geom(x4, w4)
        B, Cin, Cout, Cw, H, W, KH, KW = geom
        alpha_pairs = smorph_pair_alphas(alpha, ctx.merge, Cin, Cout)
        grad_output = grad_output.contiguous()
        if grad_output.dtype != x4.dtype:
            raise RuntimeError("grad_output must have the same dtype as input")
        grad_input = torch.empty_like(x4)
        grad_weight = torch.empty_like(w4)
        grad_alpha_pairs = torch.empty_like(alpha_pairs)
        _native.smorph_backward(int(ctx.merge), x4, w4, alpha_pairs, out, grad_output, grad_input, grad_weight, grad_alpha_pairs, geom,
                                stats=stats)
        # A single alpha shared by every pair receives the gradient of all of them (smorph.cpp:96-98).
        if alpha.numel() == grad_alpha_pairs.numel():
            grad_alpha = grad_alpha_pairs.view_as(alpha)
        else:
            grad_alpha = grad_alpha_pairs.sum().view_as(alpha)
        return grad_input, grad_weight, grad_alpha, None, None


def smorph_operation(input: torch.Tensor, weight: torch.Tensor, alpha: torch.Tensor, merge: int) -> torch.Tensor:
    """Body of the ``smorph`` operator: bindings.cpp:109-120 then Smorph::forward's checks
    (smorph.cpp:20-47, smorph_cpu_kernels.hxx:642-649)."""
    merge = to_merge(merge)
    if merge == MorphoMerge.SMOOTH:
        raise RuntimeError("Unsupported merge operation for smorph")
    input_dims = input.dim()
    x4 = input_to_4d(input)
    w4 = weight_to_4d(weight)
    _check_4d(x4, w4)
    if merge == MorphoMerge.IDENTITY:
        _check_identity(x4, w4, smorph=True)
    elif x4.shape[1] != w4.shape[1]:
        raise RuntimeError("Input channels must match weight input channels")
    smorph_pair_alphas(alpha, merge, int(x4.shape[1]), int(w4.shape[0]))
    _check_device(x4, w4, alpha, name="smorph_forward_hip")
    # Inside Function.forward autograd is off: whether a backward can follow is decided here.
    needs_grad = torch.is_grad_enabled() and (input.requires_grad or weight.requires_grad or alpha.requires_grad)
    out = _SmorphFunction.apply(x4, w4, alpha, merge, needs_grad)
    return output_to_original(out, input_dims)


def smorph_scm_operation(input, weight, alpha, beta):
    """The SMOOTH channel merge (smorph_scm, reference smorph_scm.cpp) is not provided."""
    raise NotImplementedError("morphocore_amd does not implement smorph_scm (smorph with beta, the SMOOTH channel merge)")
