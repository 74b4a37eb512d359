"""Shared helpers of the tests: seeded inputs and the norm-wise error the gradient checks use."""
import os

import numpy as np
import torch


def normwise_error(actual, expected) -> float:
    """max |actual - expected| / max |expected| (0 when both are zero); non-finite entries must match."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    fin = np.isfinite(e)
    assert np.array_equal(fin, np.isfinite(a)), "non-finite entries differ"
    assert np.array_equal(a[~fin], e[~fin]) or np.all(np.isnan(a[~fin]) == np.isnan(e[~fin]))
    if not fin.any():
        return 0.0
    scale = np.max(np.abs(e[fin]))
    diff = np.max(np.abs(a[fin] - e[fin]))
    if scale == 0.0:
        return float(diff)
    return float(diff / scale)


# Tolerances of the parity contract: relative 1e-6 (float32) and 1e-12 (float64), measured norm-wise.
TOL = {np.float32: 1e-6, np.float64: 1e-12, torch.float32: 1e-6, torch.float64: 1e-12}


def seeded(seed, *shape, dtype=torch.float32, kind="rand", scale=1.0, low=0.0):
    g = torch.Generator().manual_seed(seed)
    if kind == "rand":
        t = torch.rand(*shape, generator=g, dtype=torch.float64) * scale + low
    elif kind == "randn":
        t = torch.randn(*shape, generator=g, dtype=torch.float64) * scale
    elif kind == "quant":
        t = torch.randint(0, 16, shape, generator=g).to(torch.float64) / 16.0
    else:
        raise ValueError(kind)
    return t.to(dtype)


REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref", "libmorphocore_ref.so")


def reference_run(kind, timeout=600, **arrays):
    """Runs the reference's own CPU extension (oracle/_ref, built from its sources) on `arrays` in a
    child process (oracle/ref_run.py; it registers the product's torch.ops namespace) on up to 16 host
    threads, and returns its outputs as a dict of arrays."""
    import subprocess
    import sys
    import tempfile

    threads = min(16, len(os.sched_getaffinity(0)))
    with tempfile.TemporaryDirectory() as d:
        src, dst = os.path.join(d, "in.npz"), os.path.join(d, "out.npz")
        np.savez(src, kind=np.array(kind), threads=np.array(threads), **arrays)
        script = os.path.join(os.path.dirname(REF_LIB), os.pardir, "ref_run.py")
        r = subprocess.run([sys.executable, script, src, dst], capture_output=True, text=True, timeout=timeout)
        assert r.returncode == 0, f"reference run failed: {r.stderr[-2000:]}"
        with np.load(dst) as f:
            return {k: f[k] for k in f.files}
