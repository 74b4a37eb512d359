"""CPU baseline leg of bench.py — TEST / MEASUREMENT INFRASTRUCTURE ONLY.

Times forward + backward of a bounded sample of a bench workload on the host cores, with the
reference's own CPU extension (oracle/_ref/libmorphocore_ref.so, built from the reference sources by
oracle/Makefile.ref) when it is present, else with the C oracle (oracle/libmorpho_oracle.so). Runs in
its own process (the reference extension registers the same torch.ops namespace as the product), and
prints one JSON object:
  {"seconds_per_step": s, "output_elements": n, "kind": "reference"|"port", "threads": t, "steps": k}

Usage: python oracle/cpu_baseline.py '<json spec>' where the spec holds
  kind: "morpho" | "smorph" | "stack" | "pair" | "sigma" | "scm", op: "dilation"|"erosion" (pair: the first stage), merge, padding,
  dtype: "f32"|"f64",
  x: [B,C,H,W], w: [Cout,Cw,KH,KW], alpha (smorph), threads, min_seconds.
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
REF_LIB = os.path.join(HERE, "_ref", "libmorphocore_ref.so")

MERGES = {"max": 0, "min": 1, "sum": 2, "mean": 3, "identity": 5}
PADDINGS = {"zero": 0, "geodesic": 1, "constant": 2, "replicate": 3}


def _inputs(spec, torch):
    # 16-bit workloads: the reference has no 16-bit path; it runs float32 on the same (rounded) values.
    dtype = torch.float64 if spec.get("dtype") == "f64" else torch.float32
    g = torch.Generator().manual_seed(0)
    x = (torch.rand(*spec["x"], generator=g, dtype=torch.float64) * spec.get("x_scale", 1.0) + spec.get("x_low", 0.0)).to(dtype)
    if spec.get("dtype") in ("f16", "bf16"):
        x = x.to(getattr(torch, "float16" if spec["dtype"] == "f16" else "bfloat16")).to(dtype)
    ws = [(torch.randn(*spec["w"], generator=g, dtype=torch.float64) * spec.get("w_std", 0.1)).to(dtype)
          for _ in range(3 if spec["kind"] == "stack" else 1)]
    return x, ws, dtype


def run_reference(spec, threads):
    import torch

    torch.set_num_threads(threads)
    torch.ops.load_library(REF_LIB)
    ops = torch.ops.morphocore
    x, ws, dtype = _inputs(spec, torch)
    merge, padding = MERGES.get(spec.get("merge", "sum")), PADDINGS.get(spec.get("padding", "replicate"))

    def step():
        xr = x.clone().requires_grad_(True)
        wr = [w.clone().requires_grad_(True) for w in ws]
        if spec["kind"] == "morpho":
            if spec["op"] == "dilation":
                out = ops.dilation(xr, wr[0], merge, padding, 0.0, True, 0.0)
            else:
                out = ops.erosion(xr, wr[0].flip((-2, -1)), merge, padding, 0.0, True, 0.0)
        elif spec["kind"] == "smorph":
            a = torch.full(spec["alpha_shape"], spec["alpha"], dtype=dtype, requires_grad=True)
            t = torch.tanh(a).unsqueeze(-1).unsqueeze(-1) if a.dim() == 2 else torch.tanh(a).view(-1, 1, 1, 1)
            wt = t * ((1 - t) / 2 * wr[0].flip(dims=(-2, -1)) + (1 + t) / 2 * wr[0])
            out = ops.smorph(xr, wt, a, merge)
        elif spec["kind"] == "scm":
            # smorph with a beta: the SMOOTH channel merge (functional/smorph.py:72-73).
            a = torch.full((x.shape[1], x.shape[1]), 1.0, dtype=dtype, requires_grad=True)
            beta = torch.full((wr[0].shape[0],), 1.0, dtype=dtype, requires_grad=True)
            t = torch.tanh(a).unsqueeze(-1).unsqueeze(-1)
            wt = t * ((1 - t) / 2 * wr[0].flip(dims=(-2, -1)) + (1 + t) / 2 * wr[0])
            out = ops.smorph_scm(xr, wt, a, beta)
        elif spec["kind"] == "pair":
            # The reference's opening / closing with per-channel merges and one shared element
            # (functional/opening.py:96-101).
            ero = lambda v: ops.erosion(v, wr[0].flip((-2, -1)), MERGES["identity"], padding, 0.0, True, 0.0)  # noqa: E731
            dil = lambda v: ops.dilation(v, wr[0], MERGES["identity"], padding, 0.0, True, 0.0)  # noqa: E731
            out = dil(ero(xr)) if spec["op"] == "erosion" else ero(dil(xr))
        elif spec["kind"] == "sigma":
            # The reference's sigma_layer, per-channel merge (functional/sigma_layer.py:73-83).
            a = torch.full((x.shape[1], 1), 0.3, dtype=dtype, requires_grad=True)
            e = ops.erosion(xr, wr[0].flip((-2, -1)), MERGES["identity"], padding, 0.0, True, 0.0)
            d = ops.dilation(xr, wr[0], MERGES["identity"], padding, 0.0, True, 0.0)
            soft = torch.sigmoid(a.mean(dim=1)).view(1, -1, 1, 1)
            out = e * (1.0 - soft) + d * soft
        else:
            a = torch.full((x.shape[1], x.shape[1]), 5.0, dtype=dtype, requires_grad=True)
            y = ops.dilation(xr, wr[0], MERGES["max"], padding, 0.0, True, 0.0)
            t = torch.tanh(a).unsqueeze(-1).unsqueeze(-1)
            wt = t * ((1 - t) / 2 * wr[1].flip(dims=(-2, -1)) + (1 + t) / 2 * wr[1])
            y = ops.smorph(y, wt, a, MERGES["sum"])
            out = ops.erosion(y, wr[2].flip((-2, -1)), MERGES["min"], padding, 0.0, True, 0.0)
        out.backward(torch.ones_like(out))
        return out.numel() * (3 if spec["kind"] == "stack" else 1)

    return step


def run_port(spec, threads):
    os.environ["OMP_NUM_THREADS"] = str(threads)
    sys.path.insert(0, ROOT)
    import numpy as np
    import torch

    from oracle import oracle as O

    x, ws, dtype = _inputs(spec, torch)
    xn = x.numpy()
    wn = [w.numpy() for w in ws]
    merge, padding = MERGES.get(spec.get("merge", "sum")), PADDINGS.get(spec.get("padding", "replicate"))

    def step():
        if spec["kind"] == "morpho":
            op = O.DILATION if spec["op"] == "dilation" else O.EROSION
            w = wn[0] if op == O.DILATION else np.ascontiguousarray(wn[0][:, :, ::-1, ::-1])
            out, idx = O.morpho_forward(op, merge, padding, 0.0, xn, w, save_indices=merge in (0, 1))
            O.morpho_backward(op, merge, padding, 0.0, xn, w, np.ones_like(out), indices=idx)
            return out.size
        if spec["kind"] == "smorph":
            alpha = np.full(spec["alpha_shape"], spec["alpha"], dtype=xn.dtype)
            wt = O.smorph_w_tilde(wn[0], alpha, spec.get("merge", "sum"))
            out = O.smorph_forward(merge, xn, wt, alpha)
            O.smorph_backward(merge, xn, wt, alpha, np.ones_like(out))
            return out.size
        if spec["kind"] == "pair":
            ops_ = (O.EROSION, O.DILATION) if spec["op"] == "erosion" else (O.DILATION, O.EROSION)
            wk = {O.DILATION: wn[0], O.EROSION: np.ascontiguousarray(wn[0][:, :, ::-1, ::-1])}
            mid, _ = O.morpho_forward(ops_[0], MERGES["identity"], padding, 0.0, xn, wk[ops_[0]])
            out, _ = O.morpho_forward(ops_[1], MERGES["identity"], padding, 0.0, mid, wk[ops_[1]])
            gm, _ = O.morpho_backward(ops_[1], MERGES["identity"], padding, 0.0, mid, wk[ops_[1]], np.ones_like(out))
            O.morpho_backward(ops_[0], MERGES["identity"], padding, 0.0, xn, wk[ops_[0]], gm)
            return out.size
        raise ValueError("the port baseline covers single operators and the opening / closing pair")

    return step


def main():
    spec = json.loads(sys.argv[1])
    threads = int(spec.get("threads", os.cpu_count() or 1))
    kind = "reference" if os.path.exists(REF_LIB) else "port"
    step = run_reference(spec, threads) if kind == "reference" else run_port(spec, threads)
    n = step()  # warm-up (also loads the library and faults in the buffers)
    steps, t0 = 0, time.perf_counter()
    while True:
        n = step()
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= float(spec.get("min_seconds", 10.0)) or steps >= int(spec.get("max_steps", 1000)):
            break
    print(json.dumps({"seconds_per_step": elapsed / steps, "output_elements": n, "kind": kind, "threads": threads, "steps": steps}))


if __name__ == "__main__":
    main()
