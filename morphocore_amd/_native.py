"""ctypes binding of the C ABI in ``include/morphocore_amd.h`` (``libmorphocore_amd.so``).

The library holds the gfx950 kernels; nothing here computes. Every call enqueues work on the
current HIP stream of the tensors' device, which is what the reference's CUDA launchers do with
``getCurrentCUDAStream()`` (reference: morphocore/functional/csrc/cuda/morpho_cuda_launch.cuh).
A missing library is an error, never a fallback.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmorphocore_amd.so")

# Every symbol include/morphocore_amd.h declares.
EXPORTS = (
    "mca_version",
    "mca_last_error",
    "mca_morpho_indices_bytes",
    "mca_morpho_forward_f32",
    "mca_morpho_forward_f64",
    "mca_morpho_backward_workspace_size_f32",
    "mca_morpho_backward_workspace_size_f64",
    "mca_morpho_backward_f32",
    "mca_morpho_backward_f64",
    "mca_morpho_backward_noalloc_f32",
    "mca_morpho_forward_f16",
    "mca_morpho_forward_bf16",
    "mca_morpho_backward_workspace_size_f16",
    "mca_morpho_backward_workspace_size_bf16",
    "mca_morpho_backward_f16",
    "mca_morpho_backward_bf16",
    "mca_smorph_forward_f32",
    "mca_smorph_forward_f64",
    "mca_smorph_backward_workspace_size_f32",
    "mca_smorph_backward_workspace_size_f64",
    "mca_smorph_backward_f32",
    "mca_smorph_backward_f64",
    "mca_smorph_stats_bytes_f32",
    "mca_smorph_forward_stats_f32",
    "mca_smorph_backward_stats_f32",
    "mca_smorph_scm_forward_workspace_size_f32",
    "mca_smorph_scm_forward_workspace_size_f64",
    "mca_smorph_scm_forward_f32",
    "mca_smorph_scm_forward_f64",
    "mca_smorph_scm_backward_workspace_size_f32",
    "mca_smorph_scm_backward_workspace_size_f64",
    "mca_smorph_scm_backward_f32",
    "mca_smorph_scm_backward_f64",
    "mca_smorph_scm_stats_bytes_f32",
    "mca_smorph_scm_forward_stats_f32",
    "mca_smorph_scm_backward_stats_f32",
    "mca_noise_sample_weights_f32",
    "mca_noise_sample_weights_f64",
    "mca_morpho_pair_supported",
    "mca_morpho_pair_forward_f32",
    "mca_morpho_pair_forward_f64",
    "mca_morpho_pair_backward_workspace_size_f32",
    "mca_morpho_pair_backward_workspace_size_f64",
    "mca_morpho_pair_backward_f32",
    "mca_morpho_pair_backward_f64",
    "mca_morpho_sigma_forward_f32",
    "mca_morpho_sigma_forward_f64",
    "mca_morpho_sigma_backward_workspace_size_f32",
    "mca_morpho_sigma_backward_workspace_size_f64",
    "mca_morpho_sigma_backward_f32",
    "mca_morpho_sigma_backward_f64",
    "mca_stack_plan_f32",
    "mca_stack_plan_f64",
    "mca_stack_forward_f32",
    "mca_stack_forward_f64",
    "mca_stack_backward_f32",
    "mca_stack_backward_f64",
    "mca_probe_smorph_exp_f32",
    "mca_probe_smorph_exp_f64",
)

_lib = None


class StackLayer(ctypes.Structure):
    """mca_stack_layer: one layer of a stack (kind 0 dilation, 1 erosion, 2 smorph)."""
    _fields_ = [("kind", ctypes.c_int), ("merge", ctypes.c_int), ("replicate", ctypes.c_int), ("save", ctypes.c_int),
                ("fill", ctypes.c_double), ("out_channels", ctypes.c_int64), ("weight_channels", ctypes.c_int64),
                ("kh", ctypes.c_int64), ("kw", ctypes.c_int64), ("weight", ctypes.c_void_p), ("alpha", ctypes.c_void_p),
                ("grad_weight", ctypes.c_void_p), ("grad_alpha", ctypes.c_void_p)]

_I, _I64, _P, _SZ = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
_GEOM = [_I64] * 8


def lib() -> ctypes.CDLL:
    """Load the native library (once). Raises RuntimeError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"morphocore_amd: native library {LIB_PATH} is not built; build it with "
            "`python setup.py build_ext --inplace` or `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    so = ctypes.CDLL(LIB_PATH)
    so.mca_version.restype = ctypes.c_char_p
    so.mca_version.argtypes = []
    so.mca_last_error.restype = ctypes.c_char_p
    so.mca_last_error.argtypes = []
    so.mca_morpho_indices_bytes.argtypes = [_I] + _GEOM
    so.mca_morpho_indices_bytes.restype = _SZ
    for sfx, real in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
        f = getattr(so, f"mca_morpho_forward_{sfx}")
        f.argtypes = [_I, _I, _I, real, _P, _P, _I64, _P, _P] + _GEOM + [_P]
        f.restype = _I
        f = getattr(so, f"mca_morpho_backward_workspace_size_{sfx}")
        f.argtypes = [_I, _I] + _GEOM
        f.restype = _SZ
        f = getattr(so, f"mca_morpho_backward_{sfx}")
        f.argtypes = [_I, _I, _I, real, _P, _P, _I64, _P, _P, _P, _P] + _GEOM + [_P, _SZ, _P]
        f.restype = _I
        f = getattr(so, f"mca_smorph_forward_{sfx}")
        f.argtypes = [_I, _P, _P, _P, _P] + _GEOM + [_P]
        f.restype = _I
        f = getattr(so, f"mca_smorph_backward_workspace_size_{sfx}")
        f.argtypes = [_I] + _GEOM
        f.restype = _SZ
        f = getattr(so, f"mca_smorph_backward_{sfx}")
        f.argtypes = [_I, _P, _P, _P, _P, _P, _P, _P, _P] + _GEOM + [_P, _SZ, _P]
        f.restype = _I
        for d in ("forward", "backward"):
            f = getattr(so, f"mca_smorph_scm_{d}_workspace_size_{sfx}")
            f.argtypes = list(_GEOM)
            f.restype = _SZ
        f = getattr(so, f"mca_probe_smorph_exp_{sfx}")
        f.argtypes = [_P, _P, _I64, _P]
        f.restype = _I
        f = getattr(so, f"mca_smorph_scm_forward_{sfx}")
        f.argtypes = [_P] * 6 + _GEOM + [_P, _SZ, _P]
        f.restype = _I
        f = getattr(so, f"mca_smorph_scm_backward_{sfx}")
        f.argtypes = [_P] * 11 + _GEOM + [_P, _SZ, _P]
        f.restype = _I
    for sfx, real in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
        f = getattr(so, f"mca_noise_sample_weights_{sfx}")
        f.argtypes = [_P, _P, real, _P, _I64, _I64, _P]
        f.restype = _I
    for sfx in ("f16", "bf16"):
        f = getattr(so, f"mca_morpho_forward_{sfx}")
        f.argtypes = [_I, _I, _I, ctypes.c_float, _P, _P, _I64, _P, _P] + _GEOM + [_P]
        f.restype = _I
        f = getattr(so, f"mca_morpho_backward_workspace_size_{sfx}")
        f.argtypes = [_I, _I] + _GEOM
        f.restype = _SZ
        f = getattr(so, f"mca_morpho_backward_{sfx}")
        f.argtypes = [_I, _I, _I, ctypes.c_float, _P, _P, _I64, _P, _P, _P, _P] + _GEOM + [_P, _SZ, _P]
        f.restype = _I
    _PGEOM = [_I64] * 6
    so.mca_morpho_pair_supported.argtypes = [_I64, _I64]
    so.mca_morpho_pair_supported.restype = _I
    for sfx, real in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
        f = getattr(so, f"mca_morpho_pair_forward_{sfx}")
        f.argtypes = [_I, _I, real, real, _P, _P, _P, _I64, _P, _P, _P] + _PGEOM + [_P]
        f.restype = _I
        f = getattr(so, f"mca_morpho_pair_backward_workspace_size_{sfx}")
        f.argtypes = list(_PGEOM)
        f.restype = _SZ
        f = getattr(so, f"mca_morpho_pair_backward_{sfx}")
        f.argtypes = [_I, _P, _P, _P, _P, _P, _P] + _PGEOM + [_P, _SZ, _P]
        f.restype = _I
        f = getattr(so, f"mca_morpho_sigma_forward_{sfx}")
        f.argtypes = [_I, real, real, _P, _P, _P, _I64, _P, _P, _P, _P] + _PGEOM + [_P]
        f.restype = _I
        f = getattr(so, f"mca_morpho_sigma_backward_workspace_size_{sfx}")
        f.argtypes = list(_PGEOM)
        f.restype = _SZ
        f = getattr(so, f"mca_morpho_sigma_backward_{sfx}")
        f.argtypes = [_I, real, real, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P] + _PGEOM + [_P, _SZ, _P]
        f.restype = _I
    so.mca_morpho_backward_noalloc_f32.argtypes = [_I, _I, _I, ctypes.c_float, _P, _P, _I64, _P, _P, _P, _P] + _GEOM + [_P]
    so.mca_morpho_backward_noalloc_f32.restype = _I
    so.mca_smorph_stats_bytes_f32.argtypes = [_I] + _GEOM
    so.mca_smorph_stats_bytes_f32.restype = _SZ
    so.mca_smorph_forward_stats_f32.argtypes = [_I, _P, _P, _P, _P, _P] + _GEOM + [_P]
    so.mca_smorph_forward_stats_f32.restype = _I
    so.mca_smorph_backward_stats_f32.argtypes = [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P] + _GEOM + [_P, _SZ, _P]
    so.mca_smorph_backward_stats_f32.restype = _I
    so.mca_smorph_scm_stats_bytes_f32.argtypes = list(_GEOM)
    so.mca_smorph_scm_stats_bytes_f32.restype = _SZ
    so.mca_smorph_scm_forward_stats_f32.argtypes = [_P] * 7 + _GEOM + [_P]
    so.mca_smorph_scm_forward_stats_f32.restype = _I
    so.mca_smorph_scm_backward_stats_f32.argtypes = [_P] * 12 + _GEOM + [_P, _SZ, _P]
    so.mca_smorph_scm_backward_stats_f32.restype = _I
    _SHAPE = [_I64] * 5  # B, C, H, W, chunk
    for sfx in ("f32", "f64"):
        f = getattr(so, f"mca_stack_plan_{sfx}")
        f.argtypes = [_P, _I] + _SHAPE + [_P, _P]
        f.restype = _I
        f = getattr(so, f"mca_stack_forward_{sfx}")
        f.argtypes = [_P, _I, _P, _P] + _SHAPE + [_P, _SZ, _P]
        f.restype = _I
        f = getattr(so, f"mca_stack_backward_{sfx}")
        f.argtypes = [_P, _I, _P, _P, _P, _P] + _SHAPE + [_P, _SZ, _P, _SZ, _P]
        f.restype = _I
    _lib = so
    return so


def version() -> str:
    return lib().mca_version().decode()


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().mca_last_error().decode())


def _sfx(t: torch.Tensor) -> str:
    if t.dtype == torch.float32:
        return "f32"
    if t.dtype == torch.float64:
        return "f64"
    if t.dtype == torch.float16:
        return "f16"
    if t.dtype == torch.bfloat16:
        return "bf16"
    raise RuntimeError(f"morphocore_amd supports float32, float64, float16 and bfloat16 tensors, got {t.dtype}")


def _ptr(t):
    return None if t is None else t.data_ptr()


# The current stream's raw handle of a device index: torch's direct accessor (a few hundred ns) when
# this torch build has it, else the Stream object's handle (a few microseconds, the launch-bound
# configurations feel it).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def indices_bytes(merge, geom) -> int:
    """Bytes of the winners the forward can save for this merge (C ABI mca_morpho_indices_bytes):
    packed int32 per output pixel for max / min, one tap per channel pair and pixel otherwise."""
    return int(lib().mca_morpho_indices_bytes(merge, *geom))


def morpho_forward(op, merge, replicate, fill, x, weight, weight_batch_stride, out, indices, geom):
    """Enqueue the dilation / erosion forward (C ABI mca_morpho_forward_*)."""
    f = getattr(lib(), f"mca_morpho_forward_{_sfx(x)}")
    _check(f(op, merge, int(replicate), fill, _ptr(x), _ptr(weight), weight_batch_stride, _ptr(out), _ptr(indices), *geom, _stream(x)))


def morpho_backward(op, merge, replicate, fill, x, weight, weight_batch_stride, indices, grad_out, grad_in, grad_w, geom):
    """Enqueue the dilation / erosion backward (C ABI mca_morpho_backward_*), workspace from torch."""
    so, sfx = lib(), _sfx(x)
    nbytes = getattr(so, f"mca_morpho_backward_workspace_size_{sfx}")(merge, int(indices is not None), *geom)
    ws = _workspace(nbytes, x.device)
    f = getattr(so, f"mca_morpho_backward_{sfx}")
    _check(f(op, merge, int(replicate), fill, _ptr(x), _ptr(weight), weight_batch_stride, _ptr(indices), _ptr(grad_out), _ptr(grad_in),
             _ptr(grad_w), *geom, _ptr(ws), ws.numel(), _stream(x)))


# Device scratch each GPU holds for the no-allocation backward (MCA_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20


def morpho_backward_noalloc(op, merge, replicate, fill, x, weight, weight_batch_stride, indices, grad_out, grad_in, grad_w, geom):
    """Enqueue the float32 dilation / erosion backward that allocates nothing (C ABI
    mca_morpho_backward_noalloc_f32): its workspace is the library's per-GPU device scratch."""
    _check(lib().mca_morpho_backward_noalloc_f32(op, merge, int(replicate), fill, _ptr(x), _ptr(weight), weight_batch_stride,
                                                 _ptr(indices), _ptr(grad_out), _ptr(grad_in), _ptr(grad_w), *geom, _stream(x)))


def smorph_stats_bytes(merge, dtype, geom) -> int:
    """Bytes of the pair statistics the smorph forward can save for its backward (C ABI
    mca_smorph_stats_bytes_f32); 0 when the configuration has no such path (float64, other sizes)."""
    if dtype != torch.float32:
        return 0
    return int(lib().mca_smorph_stats_bytes_f32(merge, *geom))


def smorph_forward(merge, x, weight, alpha_pairs, out, geom, stats=None):
    """Enqueue the smorph forward (C ABI mca_smorph_forward_*); with `stats` (a float32 buffer of
    smorph_stats_bytes bytes) the pair statistics are saved too (mca_smorph_forward_stats_f32)."""
    if stats is not None:
        _check(lib().mca_smorph_forward_stats_f32(merge, _ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(out), _ptr(stats), *geom,
                                                  _stream(x)))
        return
    f = getattr(lib(), f"mca_smorph_forward_{_sfx(x)}")
    _check(f(merge, _ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(out), *geom, _stream(x)))


def smorph_backward(merge, x, weight, alpha_pairs, out, grad_out, grad_in, grad_w, grad_alpha, geom, stats=None):
    """Enqueue the smorph backward (C ABI mca_smorph_backward_*, or mca_smorph_backward_stats_f32 with
    the forward's saved `stats`), workspace from torch."""
    so, sfx = lib(), _sfx(x)
    nbytes = getattr(so, f"mca_smorph_backward_workspace_size_{sfx}")(merge, *geom)
    ws = _workspace(nbytes, x.device)
    if stats is not None:
        _check(so.mca_smorph_backward_stats_f32(merge, _ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(out), _ptr(stats), _ptr(grad_out),
                                                _ptr(grad_in), _ptr(grad_w), _ptr(grad_alpha), *geom, _ptr(ws), ws.numel(), _stream(x)))
        return
    f = getattr(so, f"mca_smorph_backward_{sfx}")
    _check(f(merge, _ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(out), _ptr(grad_out), _ptr(grad_in), _ptr(grad_w), _ptr(grad_alpha),
             *geom, _ptr(ws), ws.numel(), _stream(x)))


def smorph_scm_stats_bytes(dtype, geom) -> int:
    """Bytes of the pair statistics the smorph_scm forward can save for its backward (C ABI
    mca_smorph_scm_stats_bytes_f32); 0 when the configuration has no such path."""
    if dtype != torch.float32:
        return 0
    return int(lib().mca_smorph_scm_stats_bytes_f32(*geom))


def smorph_scm_forward(x, weight, alpha_pairs, beta, out, merge_stats, geom, pair_stats=None):
    """Enqueue smorph with the SMOOTH merge (C ABI mca_smorph_scm_forward_*), workspace from torch;
    `merge_stats` (2 * B * Cout * H * W values, or None) receives the soft merge's ref and 1 / sum.
    With `pair_stats` (float32, smorph_scm_stats_bytes bytes) the pair statistics are saved too
    (mca_smorph_scm_forward_stats_f32, no workspace)."""
    so, sfx = lib(), _sfx(x)
    if pair_stats is not None:
        _check(so.mca_smorph_scm_forward_stats_f32(_ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(beta), _ptr(out), _ptr(merge_stats),
                                                   _ptr(pair_stats), *geom, _stream(x)))
        return
    ws = _workspace(getattr(so, f"mca_smorph_scm_forward_workspace_size_{sfx}")(*geom), x.device)
    f = getattr(so, f"mca_smorph_scm_forward_{sfx}")
    _check(f(_ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(beta), _ptr(out), _ptr(merge_stats), *geom, _ptr(ws), ws.numel(), _stream(x)))


def smorph_scm_backward(x, weight, alpha_pairs, beta, out, merge_stats, grad_out, grad_in, grad_w, grad_alpha, grad_beta, geom,
                        pair_stats=None):
    """Enqueue the smorph_scm backward (C ABI mca_smorph_scm_backward_*, or
    mca_smorph_scm_backward_stats_f32 with the forward's saved `pair_stats`), workspace from torch."""
    so, sfx = lib(), _sfx(x)
    ws = _workspace(getattr(so, f"mca_smorph_scm_backward_workspace_size_{sfx}")(*geom), x.device)
    if pair_stats is not None:
        _check(so.mca_smorph_scm_backward_stats_f32(_ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(beta), _ptr(out), _ptr(merge_stats),
                                                    _ptr(pair_stats), _ptr(grad_out), _ptr(grad_in), _ptr(grad_w), _ptr(grad_alpha),
                                                    _ptr(grad_beta), *geom, _ptr(ws), ws.numel(), _stream(x)))
        return
    f = getattr(so, f"mca_smorph_scm_backward_{sfx}")
    _check(f(_ptr(x), _ptr(weight), _ptr(alpha_pairs), _ptr(beta), _ptr(out), _ptr(merge_stats), _ptr(grad_out), _ptr(grad_in), _ptr(grad_w),
             _ptr(grad_alpha), _ptr(grad_beta), *geom, _ptr(ws), ws.numel(), _stream(x)))


def noise_sample_weights(weight, uniform, scale, out):
    """Enqueue the per-sample elements of weight noise (C ABI mca_noise_sample_weights_*): out[b] =
    weight + (uniform[b] * 2 - 1) * scale with torch's roundings; uniform and out [B, *weight.shape]."""
    f = getattr(lib(), f"mca_noise_sample_weights_{_sfx(weight)}")
    _check(f(_ptr(weight), _ptr(uniform), scale, _ptr(out), uniform.shape[0], weight.numel(), _stream(weight)))


def morpho_pair_supported(KH, KW) -> bool:
    """Whether the fused opening / closing has kernels for this element (C ABI mca_morpho_pair_supported)."""
    return bool(lib().mca_morpho_pair_supported(KH, KW))


def morpho_pair_forward(first_op, replicate, fill_first, fill_second, x, w_first, w_second, weight_batch_stride, out, taps_first,
                        taps_second, pgeom):
    """Enqueue the fused opening / closing forward (C ABI mca_morpho_pair_forward_*); pgeom = (B, C, H, W, KH, KW)."""
    f = getattr(lib(), f"mca_morpho_pair_forward_{_sfx(x)}")
    _check(f(first_op, int(replicate), fill_first, fill_second, _ptr(x), _ptr(w_first), _ptr(w_second), weight_batch_stride, _ptr(out),
             _ptr(taps_first), _ptr(taps_second), *pgeom, _stream(x)))


def morpho_pair_backward(first_op, taps_first, taps_second, grad_out, grad_in, grad_w_first, grad_w_second, pgeom):
    """Enqueue the fused opening / closing backward (C ABI mca_morpho_pair_backward_*), workspace from torch."""
    so, sfx = lib(), _sfx(grad_out)
    ws = _workspace(getattr(so, f"mca_morpho_pair_backward_workspace_size_{sfx}")(*pgeom), grad_out.device)
    f = getattr(so, f"mca_morpho_pair_backward_{sfx}")
    _check(f(first_op, _ptr(taps_first), _ptr(taps_second), _ptr(grad_out), _ptr(grad_in), _ptr(grad_w_first), _ptr(grad_w_second), *pgeom,
             _ptr(ws), ws.numel(), _stream(grad_out)))


def morpho_sigma_forward(replicate, fill_erosion, fill_dilation, x, w_erosion, w_dilation, weight_batch_stride, soft, out, taps_erosion,
                         taps_dilation, pgeom):
    """Enqueue the fused sigma_layer forward, 'identity' merge (C ABI mca_morpho_sigma_forward_*)."""
    f = getattr(lib(), f"mca_morpho_sigma_forward_{_sfx(x)}")
    _check(f(int(replicate), fill_erosion, fill_dilation, _ptr(x), _ptr(w_erosion), _ptr(w_dilation), weight_batch_stride, _ptr(soft),
             _ptr(out), _ptr(taps_erosion), _ptr(taps_dilation), *pgeom, _stream(x)))


def morpho_sigma_backward(replicate, fill_erosion, fill_dilation, x, w_erosion, w_dilation, weight_batch_stride, soft, taps_erosion,
                          taps_dilation, grad_out, grad_in, grad_w_erosion, grad_w_dilation, grad_terms, pgeom):
    """Enqueue the fused sigma_layer backward (C ABI mca_morpho_sigma_backward_*), workspace from torch."""
    so, sfx = lib(), _sfx(x)
    ws = _workspace(getattr(so, f"mca_morpho_sigma_backward_workspace_size_{sfx}")(*pgeom), x.device)
    f = getattr(so, f"mca_morpho_sigma_backward_{sfx}")
    _check(f(int(replicate), fill_erosion, fill_dilation, _ptr(x), _ptr(w_erosion), _ptr(w_dilation), weight_batch_stride, _ptr(soft),
             _ptr(taps_erosion), _ptr(taps_dilation), _ptr(grad_out), _ptr(grad_in), _ptr(grad_w_erosion), _ptr(grad_w_dilation),
             _ptr(grad_terms), *pgeom, _ptr(ws), ws.numel(), _stream(x)))


def probe_smorph_exp(x, y):
    """y = the smorph kernels' exponential of x, elementwise (C ABI mca_probe_smorph_exp_*; tests)."""
    _check(getattr(lib(), f"mca_probe_smorph_exp_{_sfx(x)}")(_ptr(x), _ptr(y), x.numel(), _stream(x)))


def stack_layers(specs):
    """A ctypes array of mca_stack_layer from dicts with the fields of StackLayer (tensors for weight,
    alpha, grad_weight, grad_alpha; missing fields 0 / NULL)."""
    arr = (StackLayer * len(specs))()
    for a, spec in zip(arr, specs):
        for k, v in spec.items():
            setattr(a, k, v.data_ptr() if isinstance(v, torch.Tensor) else v)
        w = spec["weight"]
        a.out_channels, a.weight_channels, a.kh, a.kw = w.shape
    return arr


def stack_plan(layers, dtype, shape, chunk=0):
    """(saved bytes, backward workspace bytes) of a stack (C ABI mca_stack_plan_*); shape = (B, C, H, W)."""
    saved, backward = ctypes.c_size_t(0), ctypes.c_size_t(0)
    f = getattr(lib(), "mca_stack_plan_f64" if dtype == torch.float64 else "mca_stack_plan_f32")
    _check(f(ctypes.cast(layers, _P), len(layers), *shape, chunk, ctypes.byref(saved), ctypes.byref(backward)))
    return saved.value, backward.value


def stack_forward(layers, x, out, saved, chunk=0):
    """Enqueue a stack's forward (C ABI mca_stack_forward_*) into `out`, its saved state into `saved`."""
    f = getattr(lib(), f"mca_stack_forward_{_sfx(x)}")
    _check(f(ctypes.cast(layers, _P), len(layers), _ptr(x), _ptr(out), *x.shape, chunk, _ptr(saved), saved.numel(), _stream(x)))


def stack_backward(layers, x, out, grad_out, grad_in, saved, workspace, chunk=0):
    """Enqueue a stack's backward (C ABI mca_stack_backward_*): grad_in (or None) and the layers'
    grad_weight / grad_alpha buffers."""
    f = getattr(lib(), f"mca_stack_backward_{_sfx(x)}")
    _check(f(ctypes.cast(layers, _P), len(layers), _ptr(x), _ptr(out), _ptr(grad_out), _ptr(grad_in), *x.shape, chunk, _ptr(saved),
             saved.numel(), _ptr(workspace), workspace.numel(), _stream(x)))
