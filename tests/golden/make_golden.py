"""Writes tests/golden/ref_vectors.npz: input / output vectors of the reference's own CPU extension.

The extension is built from the reference sources by oracle/Makefile.ref into
oracle/_ref/libmorphocore_ref.so; this script loads it (torch.ops.load_library) and records, for
seeded small inputs, the forward outputs and the gradients of every operator, merge, padding and
dtype the hot path covers. The fixture holds data only (inputs and expected outputs); the tests pin
the oracle, and through it the HIP kernels, against it.

Run in a container that has the reference build:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libmorphocore_ref.so")
OUT = os.path.join(HERE, "ref_vectors.npz")

MERGES = {"max": 0, "min": 1, "sum": 2, "mean": 3, "identity": 5}
PADDINGS = {"zero": 0, "geodesic": 1, "constant": 2, "replicate": 3}
PADDING_VALUE = 0.25


def gen(seed, *shape, dtype, kind="randn", scale=1.0):
    g = torch.Generator().manual_seed(seed)
    if kind == "quant":
        t = torch.randint(0, 16, shape, generator=g).to(torch.float64) / 16.0
    else:
        t = torch.randn(*shape, generator=g, dtype=torch.float64) * scale
    return t.to(dtype)


def morpho_case(ops, op, merge, padding, dtype, x, w, g, save_indices):
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    fn = ops.dilation if op == "dilation" else ops.erosion
    # Kernel-facing weight: the op receives w as is (functional.erosion would flip it first).
    out = fn(xr, wr, MERGES[merge], PADDINGS[padding], PADDING_VALUE, save_indices, 0.0)
    out.backward(g)
    return out.detach(), xr.grad, wr.grad


def smorph_case(ops, merge, x, wt, alpha, g):
    xr = x.clone().requires_grad_(True)
    wr = wt.clone().requires_grad_(True)
    ar = alpha.clone().requires_grad_(True)
    out = ops.smorph(xr, wr, ar, MERGES[merge])
    out.backward(g)
    return out.detach(), xr.grad, wr.grad, ar.grad


def smorph_scm_case(ops, x, wt, alpha, beta, g):
    xr = x.clone().requires_grad_(True)
    wr = wt.clone().requires_grad_(True)
    ar = alpha.clone().requires_grad_(True)
    br = beta.clone().requires_grad_(True)
    out = ops.smorph_scm(xr, wr, ar, br)
    out.backward(g)
    return out.detach(), xr.grad, wr.grad, ar.grad, br.grad


def main():
    if not os.path.exists(REF_LIB):
        sys.exit(f"{REF_LIB} is missing: build it with make -f oracle/Makefile.ref")
    torch.set_num_threads(1)
    torch.ops.load_library(REF_LIB)
    ops = torch.ops.morphocore
    arrays = {}
    B, Cin, Cout, H, W, KH, KW = 2, 3, 4, 7, 9, 3, 5
    for dtype, dname in ((torch.float32, "f32"), (torch.float64, "f64")):
        x = gen(1, B, Cin, H, W, dtype=dtype)
        xq = gen(2, B, Cin, H, W, dtype=dtype, kind="quant")
        g = gen(3, B, Cout, H, W, dtype=dtype)
        gi = gen(4, B, Cin, H, W, dtype=dtype)  # output gradient of the identity merge (Cout = Cin)
        w = gen(5, Cout, Cin, KH, KW, dtype=dtype, scale=0.3)
        wi = gen(6, Cin, 1, KH, KW, dtype=dtype, scale=0.3)
        arrays.update({f"{dname}/x": x.numpy(), f"{dname}/xq": xq.numpy(), f"{dname}/g": g.numpy(), f"{dname}/gi": gi.numpy(),
                       f"{dname}/w": w.numpy(), f"{dname}/wi": wi.numpy()})
        paddings = PADDINGS if dtype == torch.float32 else ("geodesic", "replicate")
        for op in ("dilation", "erosion"):
            for merge in MERGES:
                for padding in paddings:
                    for variant, xin in (("rand", x), ("quant", xq)):
                        if variant == "quant" and padding not in ("geodesic", "replicate"):
                            continue
                        ident = merge == "identity"
                        wt = wi if ident else w
                        if variant == "quant":
                            wt = torch.zeros_like(wt)
                        out, gx, gw = morpho_case(ops, op, merge, padding, dtype, xin, wt, gi if ident else g, True)
                        key = f"{dname}/morpho/{op}/{merge}/{padding}/{variant}"
                        arrays[key + "/out"] = out.numpy()
                        arrays[key + "/gx"] = gx.numpy()
                        arrays[key + "/gw"] = gw.numpy()
        for merge in MERGES:
            ident = merge == "identity"
            wt = gen(7, *((Cin, 1, KH, KW) if ident else (Cout, Cin, KH, KW)), dtype=dtype, scale=0.1)
            arrays[f"{dname}/smorph/{merge}/w"] = wt.numpy()
            pairs = Cin if ident else Cout * Cin
            for aname, alpha in (("neg", torch.full((pairs,), -2.0, dtype=dtype)), ("zero", torch.zeros(pairs, dtype=dtype)),
                                 ("mixed", gen(8, pairs, dtype=dtype, scale=3.0)), ("shared", torch.tensor(0.7, dtype=dtype))):
                if aname != "shared":
                    alpha = alpha.reshape((Cin,) if ident else (Cout, Cin))
                out, gx, gw, ga = smorph_case(ops, merge, x, wt, alpha, gi if ident else g)
                key = f"{dname}/smorph/{merge}/{aname}"
                arrays[key + "/alpha"] = alpha.numpy()
                arrays[key + "/out"] = out.numpy()
                arrays[key + "/gx"] = gx.numpy()
                arrays[key + "/gw"] = gw.numpy()
                arrays[key + "/ga"] = ga.numpy()
        # smorph_scm: the SMOOTH channel merge, one beta per output channel (smorph_scm.cpp:33).
        wt = gen(9, Cout, Cin, KH, KW, dtype=dtype, scale=0.1)
        arrays[f"{dname}/scm/w"] = wt.numpy()
        alphas = {"mixed": gen(10, Cout, Cin, dtype=dtype, scale=3.0), "shared": torch.tensor(-0.8, dtype=dtype)}
        betas = {"pos": torch.full((Cout,), 2.0, dtype=dtype), "neg": torch.full((Cout,), -3.0, dtype=dtype),
                 "zero": torch.zeros(Cout, dtype=dtype), "mixed": gen(11, Cout, dtype=dtype, scale=10.0)}
        for aname, alpha in alphas.items():
            for bname, beta in betas.items():
                out, gx, gw, ga, gb = smorph_scm_case(ops, x, wt, alpha, beta, g)
                key = f"{dname}/scm/{aname}/{bname}"
                arrays[key + "/alpha"] = alpha.numpy()
                arrays[key + "/beta"] = beta.numpy()
                arrays[key + "/out"] = out.numpy()
                arrays[key + "/gx"] = gx.numpy()
                arrays[key + "/gw"] = gw.numpy()
                arrays[key + "/ga"] = ga.numpy()
                arrays[key + "/gb"] = gb.numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(arrays)} arrays to {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
