"""Runs the reference's own CPU extension on inputs read from an .npz file, in a process of its own —
TEST INFRASTRUCTURE ONLY.

The extension is oracle/_ref/libmorphocore_ref.so, built from the reference sources by
oracle/Makefile.ref. It registers the same torch.ops namespace as the product, so the tests that check
the HIP kernels against it at sizes the C oracle is too slow for start this script as a child process
(tests/helpers.py: reference_run) and read its results back.

Usage: python oracle/ref_run.py IN.npz OUT.npz
  IN holds "kind" ("smorph" or "smorph_scm"), "threads" and the operator's arguments: x, wt (the
  element the operator receives, w~), alpha, grad (the output gradient), and merge (the reference's
  int) for smorph or beta for smorph_scm.
  OUT receives out, grad_input, grad_weight (of wt), grad_alpha and, for smorph_scm, grad_beta.
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB = os.path.join(HERE, "_ref", "libmorphocore_ref.so")


def main(src, dst):
    import numpy as np
    import torch

    inp = np.load(src)
    torch.set_num_threads(int(inp["threads"]))
    torch.ops.load_library(REF_LIB)
    ops = torch.ops.morphocore
    kind = str(inp["kind"])
    if kind not in ("smorph", "smorph_scm"):
        raise ValueError(f"unknown kind {kind}")
    x = torch.from_numpy(inp["x"]).requires_grad_(True)
    wt = torch.from_numpy(inp["wt"]).requires_grad_(True)
    alpha = torch.from_numpy(inp["alpha"]).requires_grad_(True)
    extra = {}
    if kind == "smorph":
        out = ops.smorph(x, wt, alpha, int(inp["merge"]))
    else:
        beta = torch.from_numpy(inp["beta"]).requires_grad_(True)
        out = ops.smorph_scm(x, wt, alpha, beta)
    out.backward(torch.from_numpy(inp["grad"]))
    if kind == "smorph_scm":
        extra["grad_beta"] = beta.grad.numpy()
    np.savez(dst, out=out.detach().numpy(), grad_input=x.grad.numpy(), grad_weight=wt.grad.numpy(), grad_alpha=alpha.grad.numpy(), **extra)


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
