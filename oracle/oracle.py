"""CPU oracle for the morphocore hot path — TEST INFRASTRUCTURE ONLY.

Two independent restatements of the reference's CPU semantics:

* ``C`` — ctypes bindings of ``oracle/libmorpho_oracle.so`` (``morpho_oracle.c``), a plain C
  restatement of the reference CPU extension, fast enough for the configs' parity sizes.
* ``brute`` — numpy brute force for tiny inputs, built like the reference's own test references
  (``tests/functional/utils.py:6-49``, ``tests/functional/test_padding.py:9-45``), used to pin ``C``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
module. The product (``morphocore_amd``) never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmorpho_oracle.so")

# Same ints as the reference (morpho_op_enum.hpp:17-35, merge_enum.py:4-19).
MAX, MIN, ADD, AVERAGE, SMOOTH, IDENTITY = 0, 1, 2, 3, 4, 5
ZERO, GEODESIC, CONSTANT, REPLICATE = 0, 1, 2, 3
DILATION, EROSION = 0, 1

MERGES = {"max": MAX, "min": MIN, "sum": ADD, "mean": AVERAGE, "identity": IDENTITY}
PADDINGS = {"zero": ZERO, "geodesic": GEODESIC, "constant": CONSTANT, "replicate": REPLICATE}

_lib = None


def build() -> str:
    """Compile the C oracle in place (gcc, seconds)."""
    subprocess.run(["make", "-s", "-f", os.path.join(HERE, "Makefile")], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        i64, i32, p = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        geom = [i64] * 8
        for sfx, real in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
            f = getattr(_lib, f"oracle_morpho_forward_{sfx}")
            f.argtypes = [i32, i32, i32, real, p, p, i64, p, p] + geom
            f.restype = i32
            f = getattr(_lib, f"oracle_morpho_backward_{sfx}")
            f.argtypes = [i32, i32, i32, real, p, p, i64, p, p, p, p] + geom
            f.restype = i32
            f = getattr(_lib, f"oracle_smorph_forward_{sfx}")
            f.argtypes = [i32, p, p, p, p] + geom
            f.restype = i32
            f = getattr(_lib, f"oracle_smorph_backward_{sfx}")
            f.argtypes = [i32, p, p, p, p, p, p, p] + geom
            f.restype = i32
            f = getattr(_lib, f"oracle_smorph_scm_forward_{sfx}")
            f.argtypes = [p, p, p, p, p] + geom
            f.restype = i32
            f = getattr(_lib, f"oracle_smorph_scm_backward_{sfx}")
            f.argtypes = [p, p, p, p, p, p, p, p, p] + geom
            f.restype = i32
        _lib.oracle_set_abs_terms.argtypes = [i32]
        _lib.oracle_set_abs_terms.restype = None
        _lib.oracle_expf.argtypes = [ctypes.c_float]
        _lib.oracle_expf.restype = ctypes.c_float
        _lib.oracle_exp.argtypes = [ctypes.c_double]
        _lib.oracle_exp.restype = ctypes.c_double
        _lib.oracle_expf_array.argtypes = [p, p, i64]
        _lib.oracle_expf_array.restype = None
        _lib.oracle_exp_array.argtypes = [p, p, i64]
        _lib.oracle_exp_array.restype = None
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _sfx(dtype) -> str:
    if dtype == np.float32:
        return "f32"
    if dtype == np.float64:
        return "f64"
    raise TypeError(f"oracle supports float32 and float64, got {dtype}")


def fill_value(op: int, padding: int, padding_value: float, dtype) -> float:
    """morpho_fill_value (morpho_padding_policy.hpp:22-33): ZERO 0, CONSTANT the value cast to T,
    GEODESIC the neutral element (-inf dilation, +inf erosion); REPLICATE never reads it."""
    if padding == ZERO:
        return 0.0
    if padding == CONSTANT:
        return float(np.asarray(padding_value, dtype=dtype))
    return -np.inf if op == DILATION else np.inf


def _geom(x, w, sample_weight):
    B, Cin, H, W = x.shape
    wt = w if sample_weight is None else sample_weight[0]
    Cout, Cw, KH, KW = wt.shape
    return B, Cin, Cout, Cw, H, W, KH, KW


def morpho_forward(op, merge, padding, padding_value, x, w, save_indices=False, sample_weight=None):
    """Op-level forward (kernel-facing weight: erosion callers pass the flipped weight).

    ``x`` [B,Cin,H,W]; ``w`` [Cout,Cw,KH,KW]; ``sample_weight`` optional [B,Cout,Cw,KH,KW].
    Returns ``(out, indices or None)``."""
    x = np.ascontiguousarray(x)
    dtype = x.dtype
    wt = np.ascontiguousarray(w if sample_weight is None else sample_weight, dtype=dtype)
    B, Cin, Cout, Cw, H, W, KH, KW = _geom(x, w, sample_weight)
    out = np.empty((B, Cout, H, W), dtype=dtype)
    idx = np.empty((B, Cout, H, W), dtype=np.int32) if save_indices else None
    stride = Cout * Cw * KH * KW if sample_weight is not None else 0
    fn = getattr(lib(), f"oracle_morpho_forward_{_sfx(dtype)}")
    rc = fn(op, merge, int(padding == REPLICATE), fill_value(op, padding, padding_value, dtype), _ptr(x), _ptr(wt), stride,
            _ptr(out), _ptr(idx), B, Cin, Cout, Cw, H, W, KH, KW)
    if rc != 0:
        raise RuntimeError(f"oracle_morpho_forward failed ({rc})")
    return out, idx


def morpho_backward(op, merge, padding, padding_value, x, w, grad_out, indices=None, sample_weight=None):
    """Op-level backward. Returns ``(grad_input, grad_weight)``; grad_weight has w's shape."""
    x = np.ascontiguousarray(x)
    dtype = x.dtype
    wt = np.ascontiguousarray(w if sample_weight is None else sample_weight, dtype=dtype)
    grad_out = np.ascontiguousarray(grad_out, dtype=dtype)
    B, Cin, Cout, Cw, H, W, KH, KW = _geom(x, w, sample_weight)
    gx = np.empty_like(x)
    gw = np.empty((Cout, Cw, KH, KW), dtype=dtype)
    stride = Cout * Cw * KH * KW if sample_weight is not None else 0
    idx = None if indices is None else np.ascontiguousarray(indices, dtype=np.int32)
    fn = getattr(lib(), f"oracle_morpho_backward_{_sfx(dtype)}")
    rc = fn(op, merge, int(padding == REPLICATE), fill_value(op, padding, padding_value, dtype), _ptr(x), _ptr(wt), stride,
            _ptr(idx), _ptr(grad_out), _ptr(gx), _ptr(gw), B, Cin, Cout, Cw, H, W, KH, KW)
    if rc != 0:
        raise RuntimeError(f"oracle_morpho_backward failed ({rc})")
    return gx, gw


def pair_alphas(alpha, merge, Cin, Cout):
    """smorph_pair_alphas (smorph_cpu_kernels.hxx:642-649): one alpha per pair, or one shared."""
    alpha = np.asarray(alpha)
    pairs = Cout if merge == IDENTITY else Cout * Cin
    if alpha.size == pairs:
        return np.ascontiguousarray(alpha.reshape(pairs))
    if alpha.size == 1:
        return np.full(pairs, alpha.reshape(()), dtype=alpha.dtype)
    raise ValueError("Alpha must have one value per pair or one value")


def smorph_forward(merge, x, w_tilde, alpha):
    """Op-level smorph forward: ``w_tilde`` is the already blended weight (functional/smorph.py:56-70)."""
    x = np.ascontiguousarray(x)
    dtype = x.dtype
    w_tilde = np.ascontiguousarray(w_tilde, dtype=dtype)
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w_tilde.shape
    a = np.ascontiguousarray(pair_alphas(alpha, merge, Cin, Cout), dtype=dtype)
    out = np.empty((B, Cout, H, W), dtype=dtype)
    fn = getattr(lib(), f"oracle_smorph_forward_{_sfx(dtype)}")
    rc = fn(merge, _ptr(x), _ptr(w_tilde), _ptr(a), _ptr(out), B, Cin, Cout, Cw, H, W, KH, KW)
    if rc != 0:
        raise RuntimeError(f"oracle_smorph_forward failed ({rc})")
    return out


def smorph_backward(merge, x, w_tilde, alpha, grad_out):
    """Op-level smorph backward. Returns ``(grad_input, grad_w_tilde, grad_alpha)`` with grad_alpha
    shaped like ``alpha`` (a shared alpha receives the sum over pairs, smorph.cpp:96-98)."""
    x = np.ascontiguousarray(x)
    dtype = x.dtype
    w_tilde = np.ascontiguousarray(w_tilde, dtype=dtype)
    grad_out = np.ascontiguousarray(grad_out, dtype=dtype)
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w_tilde.shape
    alpha = np.asarray(alpha)
    a = np.ascontiguousarray(pair_alphas(alpha, merge, Cin, Cout), dtype=dtype)
    gx = np.empty_like(x)
    gw = np.empty_like(w_tilde)
    ga = np.empty_like(a)
    fn = getattr(lib(), f"oracle_smorph_backward_{_sfx(dtype)}")
    rc = fn(merge, _ptr(x), _ptr(w_tilde), _ptr(a), _ptr(grad_out), _ptr(gx), _ptr(gw), _ptr(ga), B, Cin, Cout, Cw, H, W, KH, KW)
    if rc != 0:
        raise RuntimeError(f"oracle_smorph_backward failed ({rc})")
    if alpha.size != a.size:
        ga = np.asarray(ga.sum(dtype=np.float64), dtype=dtype).reshape(alpha.shape)
    else:
        ga = ga.reshape(alpha.shape)
    return gx, gw, ga


def smorph_scm_forward(x, w_tilde, alpha, beta):
    """Op-level smorph with the SMOOTH channel merge (the smorph_scm operator, smorph_scm.cpp:13-53):
    ``beta`` holds one value per output channel; ``alpha`` one per pair or one shared value."""
    x = np.ascontiguousarray(x)
    dtype = x.dtype
    w_tilde = np.ascontiguousarray(w_tilde, dtype=dtype)
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w_tilde.shape
    a = np.ascontiguousarray(pair_alphas(alpha, SMOOTH, Cin, Cout), dtype=dtype)
    b = np.ascontiguousarray(np.asarray(beta, dtype=dtype).reshape(-1))
    if b.size != Cout:
        raise ValueError("Beta must have shape [out_channels]")
    out = np.empty((B, Cout, H, W), dtype=dtype)
    rc = getattr(lib(), f"oracle_smorph_scm_forward_{_sfx(dtype)}")(_ptr(x), _ptr(w_tilde), _ptr(a), _ptr(b), _ptr(out), B, Cin, Cout, Cw,
                                                                   H, W, KH, KW)
    if rc != 0:
        raise RuntimeError(f"oracle_smorph_scm_forward failed ({rc})")
    return out


def smorph_scm_backward(x, w_tilde, alpha, beta, grad_out):
    """Op-level smorph_scm backward (smorph_scm.cpp:55-96). Returns ``(grad_input, grad_w_tilde,
    grad_alpha, grad_beta)``, grad_alpha shaped like ``alpha`` (a shared alpha receives the sum over
    pairs) and grad_beta like ``beta``."""
    x = np.ascontiguousarray(x)
    dtype = x.dtype
    w_tilde = np.ascontiguousarray(w_tilde, dtype=dtype)
    grad_out = np.ascontiguousarray(grad_out, dtype=dtype)
    B, Cin, H, W = x.shape
    Cout, Cw, KH, KW = w_tilde.shape
    alpha = np.asarray(alpha)
    beta = np.asarray(beta)
    a = np.ascontiguousarray(pair_alphas(alpha, SMOOTH, Cin, Cout), dtype=dtype)
    b = np.ascontiguousarray(beta.astype(dtype).reshape(-1))
    gx, gw, ga, gb = np.empty_like(x), np.empty_like(w_tilde), np.empty_like(a), np.empty_like(b)
    rc = getattr(lib(), f"oracle_smorph_scm_backward_{_sfx(dtype)}")(_ptr(x), _ptr(w_tilde), _ptr(a), _ptr(b), _ptr(grad_out), _ptr(gx),
                                                                    _ptr(gw), _ptr(ga), _ptr(gb), B, Cin, Cout, Cw, H, W, KH, KW)
    if rc != 0:
        raise RuntimeError(f"oracle_smorph_scm_backward failed ({rc})")
    if alpha.size != a.size:
        ga = np.asarray(ga.sum(dtype=np.float64), dtype=dtype).reshape(alpha.shape)
    else:
        ga = ga.reshape(alpha.shape)
    return gx, gw, ga, gb.reshape(beta.shape)


def smorph_term_magnitudes(merge, x, w_tilde, alpha, grad_out):
    """Test helper, no counterpart in the reference: for the weight and alpha gradients of smorph_backward
    (shaped like them), the sums of the magnitudes of their terms (every routed tap's c, every pixel's and
    tap's pg (v - ref)(v - out)): ``(weight magnitudes, alpha magnitudes)``, the scale against which the
    float32 error of those sums, whose terms can cancel far below their size, is measured."""
    lib().oracle_set_abs_terms(1)
    try:
        r = smorph_backward(merge, x, w_tilde, alpha, grad_out)
        return r[1], r[2]
    finally:
        lib().oracle_set_abs_terms(0)


def smorph_scm_term_magnitudes(x, w_tilde, alpha, beta, grad_out):
    """As smorph_term_magnitudes for smorph_scm_backward: ``(weight, alpha, beta magnitudes)``, the beta
    terms being each pixel's and pair's q (c - ref)(c - out) g."""
    lib().oracle_set_abs_terms(1)
    try:
        r = smorph_scm_backward(x, w_tilde, alpha, beta, grad_out)
        return r[1], r[2], r[3]
    finally:
        lib().oracle_set_abs_terms(0)


# ----------------------------------------------------------------------------------------------
# Functional-level helpers: what morphocore.functional computes before it calls the op.
# ----------------------------------------------------------------------------------------------

def smorph_w_tilde(w, alpha, merge_name):
    """w~ = tanh a * ((1 - tanh a)/2 * flip(w) + (1 + tanh a)/2 * w) (functional/smorph.py:56-70),
    computed with torch on the CPU exactly as the reference's Python does. Pinned by closed forms
    (tests/test_oracle.py: alpha 0 and +-20, tanh alpha = +-1/2 by hand, every alpha shape, the
    derivatives in w and alpha), which planted mistakes fail."""
    import torch

    wt = torch.as_tensor(w)
    at = torch.as_tensor(alpha)
    if merge_name == "identity" or at.dim() == 1:
        tanh_alpha = torch.tanh(at).view(-1, 1, 1, 1)
    else:
        tanh_alpha = torch.tanh(at).unsqueeze(-1).unsqueeze(-1)
    term1 = (1 + tanh_alpha) / 2
    term2 = (1 - tanh_alpha) / 2
    return (tanh_alpha * (term2 * wt.flip(dims=(-2, -1)) + term1 * wt)).numpy()


# ----------------------------------------------------------------------------------------------
# numpy brute force (tiny inputs), independent of the C restatement.
# ----------------------------------------------------------------------------------------------

class brute:
    """Shifted-copy numpy brute force, following the reference tests' construction."""

    @staticmethod
    def padded(plane, KH, KW, padding, fill):
        pad_h, pad_w = KH // 2, KW // 2
        if padding == REPLICATE:
            return np.pad(plane, ((pad_h, pad_h), (pad_w, pad_w)), mode="edge")
        return np.pad(plane, ((pad_h, pad_h), (pad_w, pad_w)), mode="constant", constant_values=fill)

    @staticmethod
    def pair(plane, wpair, op, padding, fill):
        """Per-pair extremum and first arg tap (tap (kh,kw) reads (h+pad_h-kh, w+pad_w-kw))."""
        H, W = plane.shape
        KH, KW = wpair.shape
        pad_h, pad_w = KH // 2, KW // 2
        p = brute.padded(plane, KH, KW, padding, fill)
        best = np.full((H, W), -np.inf if op == DILATION else np.inf, dtype=plane.dtype)
        arg = np.zeros((H, W), dtype=np.int32)
        for kh in range(KH):
            for kw in range(KW):
                ys, xs = 2 * pad_h - kh, 2 * pad_w - kw
                shifted = p[ys:ys + H, xs:xs + W]
                v = shifted + wpair[kh, kw] if op == DILATION else shifted - wpair[kh, kw]
                better = v > best if op == DILATION else v < best
                best = np.where(better, v, best)
                arg = np.where(better, kh * KW + kw, arg)
        return best, arg

    @staticmethod
    def forward(op, merge, padding, padding_value, x, w):
        B, Cin, H, W = x.shape
        Cout = w.shape[0]
        fill = fill_value(op, padding, padding_value, x.dtype)
        out = np.empty((B, Cout, H, W), dtype=x.dtype)
        idx = np.zeros((B, Cout, H, W), dtype=np.int32)
        lowest = np.finfo(x.dtype).min
        for b in range(B):
            for o in range(Cout):
                if merge == IDENTITY:
                    out[b, o], _ = brute.pair(x[b, o], w[o, 0], op, padding, fill)
                    continue
                m = np.full((H, W), lowest if merge == MAX else (-lowest if merge == MIN else 0), dtype=x.dtype)
                win = np.zeros((H, W), dtype=np.int32)
                for i in range(Cin):
                    best, arg = brute.pair(x[b, i], w[o, i], op, padding, fill)
                    if merge in (MAX, MIN):
                        better = np.ones_like(best, dtype=bool) if i == 0 else (best > m if merge == MAX else best < m)
                        win = np.where(better, (i << 16) | arg, win)
                        m = np.maximum(m, best) if merge == MAX else np.minimum(m, best)
                    else:
                        m = m + best
                out[b, o] = m / x.dtype.type(Cin) if merge == AVERAGE else m
                idx[b, o] = win
        return out, idx

    @staticmethod
    def smorph_pair(plane, wpair, alpha):
        """Soft extremum over in-image taps, with numpy's exp."""
        H, W = plane.shape
        KH, KW = wpair.shape
        pad_h, pad_w = KH // 2, KW // 2
        vals, valid = [], []
        for kh in range(KH):
            for kw in range(KW):
                ys = np.arange(H)[:, None] + pad_h - kh
                xs = np.arange(W)[None, :] + pad_w - kw
                ok = (ys >= 0) & (ys < H) & (xs >= 0) & (xs < W)
                v = plane[np.clip(ys, 0, H - 1), np.clip(xs, 0, W - 1)] + wpair[kh, kw]
                vals.append(v)
                valid.append(ok)
        v = np.stack(vals)
        ok = np.stack(valid)
        if alpha >= 0:
            ref = np.where(ok, v, -np.inf).max(axis=0)
        else:
            ref = np.where(ok, v, np.inf).min(axis=0)
        e = np.where(ok, np.exp((v - ref) * alpha), 0)
        S = e.sum(axis=0)
        return (e * v).sum(axis=0) / S


def exp_array(x):
    """The reference's vector exponential (morpho_cpu_simd.hpp:127-169) over a float32 / float64 array."""
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    fn = lib().oracle_expf_array if x.dtype == np.float32 else lib().oracle_exp_array
    fn(_ptr(x), _ptr(y), x.size)
    return y
