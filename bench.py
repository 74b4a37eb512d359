"""Benchmark of the morphocore_amd hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1..5] [--no-cpu-baseline]

A step is one forward + backward pass of the configuration's operator(s) over one batch of synthetic,
seeded input already resident in HBM (default configs[1], "C2"). The timed
region is exactly K steps between device synchronisations. Prints one JSON line with the whole-job
throughput in output elements per second, the roofline of the dominant kernel (measured with HIP
events on the stream the kernels run on, torch's current stream) and the CPU baseline (the
reference's own CPU extension, or the C oracle, on a bounded sample on the host cores, in a child
process).
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fwd+bwd output-elements/sec at 1 GPU; % of HBM/VALU roofline; CPU ratio"

# MI355X published peaks.
PEAK_FP32_TFLOPS = 157.3
PEAK_FP64_TFLOPS = 78.6
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    1: dict(name="dilation fwd+bwd fp32 merge=max", kind="morpho", op="dilation", merge="max", dtype="f32", x=(4, 3, 64, 64),
            w=(16, 3, 3, 3), x_dist=("rand", 0.0, 1.0), w_std=0.1, bound="valu",
            sample=dict(x=(4, 3, 64, 64))),
    2: dict(name="erosion fwd+bwd fp32 merge=sum", kind="morpho", op="erosion", merge="sum", dtype="f32", x=(16, 32, 128, 128),
            w=(32, 32, 5, 5), x_dist=("rand", 0.0, 1.0), w_std=0.05, bound="valu",
            sample=dict(x=(16, 32, 128, 128))),
    3: dict(name="smorph fwd+bwd fp32 merge=mean, alpha in {-20,-1,0,1,20}", kind="smorph", merge="mean", dtype="f32",
            x=(8, 64, 256, 256), w=(64, 64, 7, 7), x_dist=("randn", 0.0, 1.0), w_std=0.1, alphas=(-20.0, -1.0, 0.0, 1.0, 20.0),
            bound="valu", sample=dict(x=(1, 64, 128, 128))),
    4: dict(name="dilation fwd+bwd fp64 merge=identity", kind="morpho", op="dilation", merge="identity", dtype="f64",
            x=(32, 128, 112, 112), w=(128, 1, 3, 3), x_dist=("rand", -1.0, 2.0), w_std=0.1, bound="hbm",
            sample=dict(x=(4, 128, 112, 112))),
    5: dict(name="dilation(max) -> smorph(alpha=5,sum) -> erosion(min) fwd+bwd fp32", kind="stack", dtype="f32", x=(8, 64, 512, 512),
            w=(64, 64, 11, 11), x_dist=("rand", 0.0, 1.0), w_std=0.05, bound="valu", sample=dict(x=(1, 64, 128, 128))),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


def taps(cfg, x_shape=None):
    B, Cin, H, W = x_shape or cfg["x"]
    Cout, Cw, KH, KW = cfg["w"]
    cin_eff = 1 if cfg.get("merge") == "identity" else Cin
    return B * Cout * H * W * cin_eff * KH * KW


def work(cfg):
    """Algorithmic work of one forward and one backward launch (flop, or bytes for the HBM-bound
    config): every tap counts, border included; a max-plus tap is 2 flop, a smorph tap 8 flop forward
    and 18 flop backward; the backward of a per-pair merge adds the routing add of every pair."""
    B, Cin, H, W = cfg["x"]
    Cout = cfg["w"][0]
    t = taps(cfg)
    if cfg["kind"] == "morpho":
        if cfg["bound"] == "hbm":
            esz = 8 if cfg["dtype"] == "f64" else 4
            n_in, n_out = B * Cin * H * W, B * Cout * H * W
            return {"fwd": (n_in + n_out) * esz, "bwd": (2 * n_in + n_out) * esz, "unit": "bytes"}
        bwd = 2 * t + (2 * B * Cout * Cin * H * W if cfg["merge"] in ("sum", "mean") else 0)
        return {"fwd": 2 * t, "bwd": bwd, "unit": "flop"}
    if cfg["kind"] == "smorph":
        n = len(cfg["alphas"])
        return {"fwd": 8 * t * n, "bwd": 18 * t * n, "unit": "flop"}
    # stack: two max-plus layers and one smorph layer.
    return {"fwd": 2 * t + 8 * t + 2 * t, "bwd": 2 * t + 18 * t + 2 * t, "unit": "flop"}


def make_inputs(cfg, torch, dev):
    dtype = torch.float64 if cfg["dtype"] == "f64" else torch.float32
    g = torch.Generator().manual_seed(0)
    kind, low, scale = cfg["x_dist"]
    x = torch.rand(*cfg["x"], generator=g, dtype=dtype) * scale + low if kind == "rand" else torch.randn(*cfg["x"], generator=g, dtype=dtype)
    nw = 3 if cfg["kind"] == "stack" else 1
    ws = [torch.randn(*cfg["w"], generator=g, dtype=dtype) * cfg["w_std"] for _ in range(nw)]
    return x.to(dev), [w.to(dev) for w in ws], dtype


def build_step(cfg, torch, mca, x, ws, dtype, dev):
    """Returns step() -> (fwd_event_pair, bwd_event_pair) and the output elements per step."""
    F = mca.functional
    xr = x.requires_grad_(True)
    wr = [w.requires_grad_(True) for w in ws]
    B, Cin, H, W = cfg["x"]
    Cout = cfg["w"][0]
    gen = torch.Generator(device=dev).manual_seed(1)
    grad = torch.randn((B, Cout, H, W), generator=gen, dtype=dtype, device=dev)

    if cfg["kind"] == "smorph":
        alphas = [torch.full((Cout, Cin), a, dtype=dtype, device=dev, requires_grad=True) for a in cfg["alphas"]]

        def fwd():
            return [F.smorph(xr, wr[0], a, channel_merge_mode=cfg["merge"]) for a in alphas]

        def bwd(outs):
            torch.autograd.backward(outs, [grad] * len(outs))

        n_out = B * Cout * H * W * len(alphas)
    elif cfg["kind"] == "stack":
        alpha = torch.full((Cout, Cin), 5.0, dtype=dtype, device=dev, requires_grad=True)

        def fwd():
            y = F.dilation(xr, wr[0], "max", "replicate")
            y = F.smorph(y, wr[1], alpha, channel_merge_mode="sum")
            return [F.erosion(y, wr[2], "min", "replicate")]

        def bwd(outs):
            torch.autograd.backward(outs, [grad])

        n_out = 3 * B * Cout * H * W
    else:
        op = F.dilation if cfg["op"] == "dilation" else F.erosion

        def fwd():
            return [op(xr, wr[0], cfg["merge"], "replicate")]

        def bwd(outs):
            torch.autograd.backward(outs, [grad])

        n_out = B * Cout * H * W

    params = [xr] + wr

    def step(events=None):
        for p in params:
            p.grad = None
        if events is not None:
            events[0].record()
        outs = fwd()
        if events is not None:
            events[1].record()
        bwd(outs)
        if events is not None:
            events[2].record()

    return step, n_out


def cpu_baseline(cfg, seconds):
    threads = min(len(os.sched_getaffinity(0)), 16)
    sx = cfg["sample"]["x"]
    spec = dict(kind=cfg["kind"], op=cfg.get("op", "dilation"), merge=cfg.get("merge", "sum"), padding="replicate", dtype=cfg["dtype"],
                x=list(sx), w=list(cfg["w"]), w_std=cfg["w_std"], x_low=cfg["x_dist"][1], x_scale=cfg["x_dist"][2], threads=threads,
                min_seconds=seconds, max_steps=50)
    if cfg["kind"] == "smorph":
        spec.update(alpha=1.0, alpha_shape=[cfg["w"][0], cfg["x"][1]])
    r = subprocess.run([sys.executable, os.path.join(ROOT, "oracle", "cpu_baseline.py"), json.dumps(spec)], capture_output=True, text=True,
                       timeout=600)
    if r.returncode != 0:
        return {"value": None, "unit": "output-elements/s", "cores": threads, "kind": None, "sample": "failed: " + r.stderr[-300:]}
    res = json.loads(r.stdout.strip().splitlines()[-1])
    desc = f"x {tuple(sx)}, w {tuple(cfg['w'])}, fwd+bwd, {res['steps']} steps after one warm-up"
    if cfg["kind"] == "smorph":
        desc += ", alpha = 1 (one point of the sweep)"
    return {"value": res["output_elements"] / res["seconds_per_step"], "unit": "output-elements/s", "cores": res["threads"],
            "kind": res["kind"], "sample": desc}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch

    import morphocore_amd as mca
    from morphocore_amd import _native

    _native.lib()
    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x, ws, dtype = make_inputs(cfg, torch, dev)
    step, n_out = build_step(cfg, torch, mca, x, ws, dtype, dev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(events[k])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in events) / args.steps
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in events) / args.steps
    ms_per_step = wall * 1000.0 / args.steps

    wk = work(cfg)
    if cfg["bound"] == "hbm":
        achieved = wk["bwd"] / (bwd_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "traffic": None}
    else:
        peak = PEAK_FP64_TFLOPS if cfg["dtype"] == "f64" else PEAK_FP32_TFLOPS
        achieved = wk["bwd"] / (bwd_ms * 1e-3) / 1e12
        roof = {"bound": "valu", "achieved": achieved, "peak": peak, "unit": "TFLOP/s", "frac": achieved / peak, "traffic": None}
    roof["kernel"] = "backward entry (mca_*_backward: dominant kernel plus its zero-fill and slot reduction)"
    roof["fwd_achieved"] = (wk["fwd"] / (fwd_ms * 1e-3)) / (1e9 if cfg["bound"] == "hbm" else 1e12)

    line = {
        "metric": METRIC,
        "value": n_out / (ms_per_step * 1e-3),
        "unit": "output-elements/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "fwd_ms": fwd_ms,
        "bwd_ms": bwd_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if cfg["dtype"] == "f64" else "f32",
        "data": "synthetic (seeded torch generators), inputs resident in HBM",
        "config": {"workload": f"configs[{args.config - 1}]: {cfg['name']}", "x": list(cfg["x"]), "w": list(cfg["w"]), "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
