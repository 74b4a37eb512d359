"""Runs the reference's own CPU extension on inputs read from an .npz file, in a process of its own —
TEST INFRASTRUCTURE ONLY.

The extension is oracle/_ref/libmorphocore_ref.so, built from the reference sources by
oracle/Makefile.ref. It registers the same torch.ops namespace as the product, so the tests that check
the HIP kernels against it at sizes the C oracle is too slow for start this script as a child process
(tests/helpers.py: reference_run) and read its results back.

Usage: python oracle/ref_run.py IN.npz OUT.npz
  IN holds "kind" ("smorph"), "threads" and the operator's arguments; for smorph: x, wt (the element
  the operator receives, w~), alpha, grad (the output gradient), merge (the reference's int).
  OUT receives out, grad_input, grad_weight (of wt) and grad_alpha.
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
    if kind != "smorph":
        raise ValueError(f"unknown kind {kind}")
    x = torch.from_numpy(inp["x"]).requires_grad_(True)
    wt = torch.from_numpy(inp["wt"]).requires_grad_(True)
    alpha = torch.from_numpy(inp["alpha"]).requires_grad_(True)
    out = ops.smorph(x, wt, alpha, int(inp["merge"]))
    out.backward(torch.from_numpy(inp["grad"]))
    np.savez(dst, out=out.detach().numpy(), grad_input=x.grad.numpy(), grad_weight=wt.grad.numpy(), grad_alpha=alpha.grad.numpy())


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
