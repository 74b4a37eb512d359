"""Benchmark of the morphocore_amd hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1..9] [--no-cpu-baseline] [--no-extra]

K and W default per config (DEFAULT_STEPS below): enough steps for steady clocks on the
millisecond-scale configs, one or two on the half-second ones, so every default run ends in minutes.

A step is one forward + backward pass of the configuration's operator(s) over one batch of synthetic,
seeded input already resident in HBM. The default is configs[4], the
3-layer 8x64x512x512 11x11 stack: BASELINE.json's metric names no configuration, and this is the
largest one that fits one GPU. After it, the default run also times configs[2] (the smorph alpha
sweep the north star's target is stated on) and reports it under "configs2_step" (--no-extra
skips it). The timed region is exactly K steps between device synchronisations.

Prints one JSON line with the whole-job throughput in output elements per second, the roofline of
the config's dominant kernel (launched through the C ABI after the timed region and timed with HIP
events on torch's current stream, the stream it runs on; HBM traffic and VALU instruction counts
from the committed rocprofv3 counter summaries) and the CPU baseline (the reference's own CPU
extension, or the C oracle, on a bounded sample on the host cores, in a child process).

--config 1..5 are BASELINE.json's configs[0..4]. --config 6 and 7 are workloads of the fused
compositions at configs[3]'s float64 shape, per-channel merges and one 3x3 element: the opening
(nn.Opening's default form) and sigma_layer, each as one fused operator; their lines also carry the
same step run as the reference's composition of operators ("composition_step"). --config 8 is
configs[3] in float16 (16-bit storage, float32 arithmetic; the reference has no 16-bit path, so its
CPU baseline runs float32 on the same values). --config 9 is smorph with the SMOOTH channel merge
(smorph_scm, a beta per output channel) at configs[2]'s shape, alpha 1 and beta 1.

--kernel-only and --copy-calibration launch only the dominant kernel, or a plain device copy, for
rocprofv3 counter runs.
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
    6: dict(name="opening fwd+bwd fp64 (erosion -> dilation, merge=identity, one shared element), fused", kind="pair", first="erosion",
            dtype="f64", x=(32, 128, 112, 112), w=(128, 1, 3, 3), x_dist=("rand", -1.0, 2.0), w_std=0.1, bound="hbm",
            sample=dict(x=(4, 128, 112, 112)), key="pair_opening_f64"),
    7: dict(name="sigma_layer fwd+bwd fp64 (erosion and dilation blended, merge=identity), fused", kind="sigma", dtype="f64",
            x=(32, 128, 112, 112), w=(128, 1, 3, 3), x_dist=("rand", -1.0, 2.0), w_std=0.1, bound="hbm",
            sample=dict(x=(4, 128, 112, 112)), key="sigma_identity_f64"),
    8: dict(name="dilation fwd+bwd fp16 merge=identity", kind="morpho", op="dilation", merge="identity", dtype="f16",
            x=(32, 128, 112, 112), w=(128, 1, 3, 3), x_dist=("rand", -1.0, 2.0), w_std=0.1, bound="hbm",
            sample=dict(x=(4, 128, 112, 112)), key="dilation_identity_f16"),
    9: dict(name="smorph_scm fwd+bwd fp32 (SMOOTH merge, alpha 1, beta 1)", kind="scm", dtype="f32", x=(8, 64, 256, 256),
            w=(64, 64, 7, 7), x_dist=("randn", 0.0, 1.0), w_std=0.1, bound="valu", sample=dict(x=(1, 64, 64, 64)),
            key="smorph_scm_f32"),
}

# Bench dtypes: torch dtype and bytes per element.
DTYPES = {"f64": ("float64", 8), "f32": ("float32", 4), "f16": ("float16", 2), "bf16": ("bfloat16", 2)}


def esize(cfg):
    return DTYPES[cfg["dtype"]][1]


def config_key(config):
    """Name of a config in the committed profile records and the bench line."""
    return CONFIGS[config].get("key", f"configs[{config - 1}]")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None, help="timed steps (default: per config, DEFAULT_STEPS)")
    p.add_argument("--warmup", type=int, default=None, help="untimed warmup steps (default: per config, DEFAULT_STEPS)")
    p.add_argument("--config", type=int, default=5, choices=sorted(CONFIGS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true", help="do not also time configs[2] after the default configs[4]")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--kernel-only", action="store_true",
                   help="launch only the config's dominant kernel --steps times (for rocprofv3 counter runs)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="copy a MIB-sized device buffer --steps times (scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = p.parse_args()
    steps, warmup = DEFAULT_STEPS[args.config]
    if args.kernel_only or args.copy_calibration:
        steps, warmup = 10, 0
    if args.steps is None:
        args.steps = steps
    if args.warmup is None:
        args.warmup = warmup
    return args


# Default timed and warmup steps per config: about a tenth of a second to two seconds of timed work,
# after enough warmup (~20 ms or one step of GPU work) for the clocks to settle; a 10-step run of a
# millisecond-scale config reads ~8% high (configs[1]: 1.00 against 0.93 ms per step).
DEFAULT_STEPS = {1: (500, 50), 2: (100, 20), 3: (3, 1), 4: (200, 20), 5: (2, 1), 6: (200, 20), 7: (200, 20), 8: (200, 20), 9: (2, 1)}


def taps(cfg, x_shape=None):
    B, Cin, H, W = x_shape or cfg["x"]
    Cout, Cw, KH, KW = cfg["w"]
    cin_eff = 1 if cfg.get("merge") == "identity" else Cin
    return B * Cout * H * W * cin_eff * KH * KW


def make_inputs(cfg, torch, dev):
    dtype = getattr(torch, DTYPES[cfg["dtype"]][0])
    gdt = torch.float64 if dtype == torch.float64 else torch.float32  # 16-bit inputs: drawn in float32, then rounded
    g = torch.Generator().manual_seed(0)
    kind, low, scale = cfg["x_dist"]
    x = torch.rand(*cfg["x"], generator=g, dtype=gdt) * scale + low if kind == "rand" else torch.randn(*cfg["x"], generator=g, dtype=gdt)
    x = x.to(dtype)
    nw = 3 if cfg["kind"] == "stack" else 1
    ws = [(torch.randn(*cfg["w"], generator=g, dtype=gdt) * cfg["w_std"]).to(dtype) for _ in range(nw)]
    return x.to(dev), [w.to(dev) for w in ws], dtype


def build_step(cfg, torch, mca, x, ws, dtype, dev):
    """Returns step(events=None), the output elements per step and the number of phases per step."""
    F = mca.functional
    xr = x.requires_grad_(True)
    wr = [w.requires_grad_(True) for w in ws]
    B, Cin, H, W = cfg["x"]
    Cout = cfg["w"][0]
    gen = torch.Generator(device=dev).manual_seed(1)
    grad = torch.randn((B, Cout, H, W), generator=gen, dtype=torch.float64 if dtype == torch.float64 else torch.float32,
                       device=dev).to(dtype)

    # A step is a list of (forward, backward) phases: one per alpha of the smorph sweep (each alpha's
    # backward runs before the next alpha's forward, so one alpha's saved state is live at a time),
    # one for the other configs.
    if cfg["kind"] == "smorph":
        alphas = [torch.full((Cout, Cin), a, dtype=dtype, device=dev, requires_grad=True) for a in cfg["alphas"]]

        def phase(a):
            return (lambda: [F.smorph(xr, wr[0], a, channel_merge_mode=cfg["merge"])]), (lambda outs: torch.autograd.backward(outs, [grad]))

        phases = [phase(a) for a in alphas]
        n_out = B * Cout * H * W * len(alphas)
        params = [xr] + wr + alphas
    elif cfg["kind"] == "stack":
        alpha = torch.full((Cout, Cin), 5.0, dtype=dtype, device=dev, requires_grad=True)

        def fwd():
            y = F.dilation(xr, wr[0], "max", "replicate")
            y = F.smorph(y, wr[1], alpha, channel_merge_mode="sum")
            return [F.erosion(y, wr[2], "min", "replicate")]

        phases = [(fwd, lambda outs: torch.autograd.backward(outs, [grad]))]
        n_out = 3 * B * Cout * H * W
        params = [xr] + wr + [alpha]
    elif cfg["kind"] in ("pair", "pair_composition"):
        # One structuring element shared by both stages (nn.Opening / nn.Closing's default).
        first, second = (F.erosion, F.dilation) if cfg["first"] == "erosion" else (F.dilation, F.erosion)
        fused = F.opening if cfg["first"] == "erosion" else F.closing
        if cfg["kind"] == "pair":
            fwd = lambda: [fused(xr, wr[0], wr[0], "identity", "replicate")]  # noqa: E731
        else:
            fwd = lambda: [second(first(xr, wr[0], "identity", "replicate"), wr[0], "identity", "replicate")]  # noqa: E731
        phases = [(fwd, lambda outs: torch.autograd.backward(outs, [grad]))]
        n_out = B * Cout * H * W
        params = [xr] + wr
    elif cfg["kind"] == "scm":
        alpha = torch.full((Cout, Cin), 1.0, dtype=dtype, device=dev, requires_grad=True)
        beta = torch.full((Cout,), 1.0, dtype=dtype, device=dev, requires_grad=True)
        phases = [((lambda: [F.smorph(xr, wr[0], alpha, beta)]), lambda outs: torch.autograd.backward(outs, [grad]))]
        n_out = B * Cout * H * W
        params = [xr] + wr + [alpha, beta]
    elif cfg["kind"] in ("sigma", "sigma_composition"):
        alpha = torch.full((Cout, 1), 0.3, dtype=dtype, device=dev, requires_grad=True)
        if cfg["kind"] == "sigma":
            fwd = lambda: [F.sigma_layer(xr, wr[0], alpha, "identity", "replicate")]  # noqa: E731
        else:
            def fwd():
                e = F.erosion(xr, wr[0], "identity", "replicate")
                d = F.dilation(xr, wr[0], "identity", "replicate")
                soft = torch.sigmoid(alpha.mean(dim=1)).view(1, -1, 1, 1)
                return [e * (1.0 - soft) + d * soft]
        phases = [(fwd, lambda outs: torch.autograd.backward(outs, [grad]))]
        n_out = B * Cout * H * W
        params = [xr] + wr + [alpha]
    else:
        op = F.dilation if cfg["op"] == "dilation" else F.erosion
        phases = [(lambda: [op(xr, wr[0], cfg["merge"], "replicate")]), (lambda outs: torch.autograd.backward(outs, [grad]))]
        phases = [tuple(phases)]
        n_out = B * Cout * H * W
        params = [xr] + wr

    def step(events=None):
        """One step; `events` (3 HIP events per phase) brackets each phase's forward and backward."""
        for p in params:
            p.grad = None
        for k, (fwd, bwd) in enumerate(phases):
            if events is not None:
                events[3 * k].record()
            outs = fwd()
            if events is not None:
                events[3 * k + 1].record()
            bwd(outs)
            del outs
            if events is not None:
                events[3 * k + 2].record()

    return step, n_out, len(phases)


MERGE_CODE = {"max": 0, "min": 1, "sum": 2, "mean": 3, "identity": 5}


def dominant(cfg, torch, native, x, ws, dtype, dev):
    """The kernel a config's roofline is quoted on (the largest share of its step on MI355X),
    launched through the C ABI on torch's current stream with the step's own inputs, and its
    algorithmic work per launch (all taps, border included; a max-plus tap 2 flop, a smorph
    backward tap 18 flop; HBM bytes: x, w, out and saved taps once)."""
    B, Cin, H, W = cfg["x"]
    Cout, Cw, KH, KW = cfg["w"]
    geom = (B, Cin, Cout, Cw, H, W, KH, KW)
    t = taps(cfg)
    esz = esize(cfg)
    if cfg["kind"] == "pair":
        # The fused forward: x read once, the output and one tap byte per stage written once.
        first = 1 if cfg["first"] == "erosion" else 0
        pg = (B, Cin, H, W, KH, KW)
        out = torch.empty_like(x)
        tp = torch.empty((2, B, Cin, H, W), dtype=torch.uint8, device=dev)
        w1 = ws[0].flip((-2, -1)).contiguous() if first == 1 else ws[0]
        w2 = ws[0] if first == 1 else ws[0].flip((-2, -1)).contiguous()
        fills = (float("inf"), float("-inf")) if first == 1 else (float("-inf"), float("inf"))

        def launch():
            native.morpho_pair_forward(first, True, fills[0], fills[1], x, w1, w2, 0, out, tp[0], tp[1], pg)

        what = f"fused {cfg['first']} -> identity pair forward (mca_morpho_pair_forward, one kernel)"
        return launch, (2 * B * Cin * H * W * esz + 2 * B * Cin * H * W + 2 * ws[0].numel() * esz), "bytes", what
    if cfg["kind"] == "scm":
        # The SMOOTH merge's backward, the larger part of its step, as the operator runs it: from the forward's saved
        # pair statistics when it would save them (float32 static two-row kernel at 7x7), else recomputing them; 18
        # flop per tap either way (the smorph backward's algorithmic work), 10 executed from saved statistics. The
        # soft merge's per-pixel work is not counted.
        from morphocore_amd import _C

        a_p = torch.full((Cout * Cin,), 1.0, dtype=dtype, device=dev)
        beta = torch.full((Cout,), 1.0, dtype=dtype, device=dev)
        wt = ws[0]
        out = torch.empty((B, Cout, H, W), dtype=dtype, device=dev)
        mst = torch.empty((2, B, Cout, H, W), dtype=dtype, device=dev)
        nbytes = native.smorph_scm_stats_bytes(dtype, geom)
        pst = torch.empty((nbytes // 4,), dtype=torch.float32, device=dev) if _C.saved_stats_admit(nbytes, dev.index or 0) else None
        native.smorph_scm_forward(x, wt, a_p, beta, out, mst, geom, pair_stats=pst)
        gen = torch.Generator(device=dev).manual_seed(2)
        grad = torch.randn((B, Cout, H, W), generator=gen, dtype=dtype, device=dev)
        gx, gw, ga, gb = torch.empty_like(x), torch.empty_like(wt), torch.empty_like(a_p), torch.empty_like(beta)

        def launch():
            native.smorph_scm_backward(x, wt, a_p, beta, out, mst, grad, gx, gw, ga, gb, geom, pair_stats=pst)

        if pst is not None:
            launch.executed_work = 10 * t
            return launch, 18 * t, "flop", ("smorph_scm backward, alpha 1, beta 1, from the forward's saved pair statistics "
                                            "(mca_smorph_scm_backward_stats_f32: kernels + reductions)")
        return launch, 18 * t, "flop", "smorph_scm backward, alpha 1, beta 1 (mca_smorph_scm_backward_f32: kernels + reductions)"
    if cfg["kind"] == "sigma":
        # The fused forward: x read once, the output and one tap byte per operation written once.
        pg = (B, Cin, H, W, KH, KW)
        out = torch.empty_like(x)
        tp = torch.empty((2, B, Cin, H, W), dtype=torch.uint8, device=dev)
        we = ws[0].flip((-2, -1)).contiguous()
        soft = torch.full((Cout,), 0.574442516811659, dtype=dtype, device=dev)

        def launch():
            native.morpho_sigma_forward(True, float("inf"), float("-inf"), x, we, ws[0], 0, soft, out, tp[0], tp[1], pg)

        what = "fused sigma_layer forward, identity merge (mca_morpho_sigma_forward, one kernel)"
        return launch, (2 * B * Cin * H * W * esz + 2 * B * Cin * H * W + 2 * ws[0].numel() * esz), "bytes", what
    if cfg["kind"] == "morpho":
        op = 0 if cfg["op"] == "dilation" else 1
        merge = MERGE_CODE[cfg["merge"]]
        out = torch.empty((B, Cout, H, W), dtype=dtype, device=dev)
        idx = torch.empty(native.indices_bytes(merge, geom), dtype=torch.uint8, device=dev)

        def launch():
            native.morpho_forward(op, merge, True, 0.0, x, ws[0], 0, out, idx, geom)

        what = f"{cfg['op']} forward, merge {cfg['merge']}, saving winners (mca_morpho_forward, one kernel)"
        if cfg["bound"] == "hbm":
            work = (B * Cin * H * W + B * Cout * H * W + ws[0].numel()) * esz + idx.numel()
            return launch, work, "bytes", what
        return launch, 2 * t, "flop", what
    # smorph (C3) or the stack's smorph layer (C5): its backward.
    merge = MERGE_CODE[cfg.get("merge", "sum")]
    a = 1.0 if cfg["kind"] == "smorph" else 5.0
    w = ws[0] if cfg["kind"] == "smorph" else ws[1]
    alpha = torch.full((Cout * Cin,), a, dtype=dtype, device=dev)
    out = torch.empty((B, Cout, H, W), dtype=dtype, device=dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    grad = torch.randn((B, Cout, H, W), generator=gen, dtype=dtype, device=dev)
    gx, gw, ga = torch.empty_like(x), torch.empty_like(w), torch.empty_like(alpha)
    # The step's own choice: the forward saves the pair statistics when the operator would.
    from morphocore_amd import _C

    nbytes = native.smorph_stats_bytes(merge, dtype, geom)
    stats = torch.empty(nbytes // 4, dtype=torch.float32, device=dev) if _C.saved_stats_admit(nbytes, dev.index or 0) else None
    native.smorph_forward(merge, x, w, alpha, out, geom, stats=stats)

    def launch():
        native.smorph_backward(merge, x, w, alpha, out, grad, gx, gw, ga, geom, stats=stats)

    if stats is not None:
        # The backward's algorithmic work is 18 flop per tap (recomputation of ref, S and W 8, exponential 1,
        # routing 9); from the saved statistics the kernel executes the exponential and the routing only: 10.
        what = (f"smorph backward, merge {cfg.get('merge', 'sum')}, alpha {a:g}, from the forward's saved pair statistics "
                "(mca_smorph_backward_stats_f32: kernel + zero-fill + slot reduction)")
        launch.executed_work = 10 * t
        return launch, 18 * t, "flop", what
    what = f"smorph backward, merge {cfg.get('merge', 'sum')}, alpha {a:g} (mca_smorph_backward: kernel + zero-fill + slot reduction)"
    return launch, 18 * t, "flop", what


def step_work(cfg):
    """Algorithmic work of one whole step (forward + backward), the convention of the dominant
    kernel's: (work, "flop" | "bytes"), or None for configs[0] (launch bound). Max-plus taps 2 flop;
    smorph forward taps 8 flop, backward taps 18 (recomputation included, whatever the kernels do);
    the identity config's bytes: x and out forward, x, grad_out and grad_x backward."""
    t = taps(cfg)
    B, Cin, H, W = cfg["x"]
    Cout = cfg["w"][0]
    if cfg["kind"] == "morpho" and cfg.get("bound") == "hbm":
        esz = esize(cfg)
        return 5 * B * Cin * H * W * esz, "bytes"
    if cfg["kind"] == "pair":
        # Forward: x read, output and two tap bytes written; backward: grad_out and two tap bytes
        # read, grad_x written.
        esz = esize(cfg)
        return B * Cin * H * W * (4 * esz + 4), "bytes"
    if cfg["kind"] == "sigma":
        # Forward: x read, output and two tap bytes written; backward: x, grad_out and two tap bytes
        # read, grad_x written.
        esz = esize(cfg)
        return B * Cin * H * W * (5 * esz + 4), "bytes"
    if cfg["kind"] == "morpho":
        return (None if B * Cout * H * W < (1 << 20) else (4 * t + 2 * B * Cout * Cin * H * W, "flop"))
    if cfg["kind"] == "smorph":
        return 26 * t * len(cfg["alphas"]), "flop"
    if cfg["kind"] == "scm":
        return 26 * t, "flop"
    return 2 * t + 26 * t + 2 * t, "flop"  # stack: dilation, smorph, erosion (index scatters not counted)


def time_launches(torch, launch, target_s=1.0, max_n=50):
    """Average duration of back-to-back launches between two HIP events on the current stream.

    A spin kernel queued ahead of the first event keeps the GPU busy while the host queues the n
    launches, so that the events bracket kernels that run back to back and not the host's launch
    gaps (which exceed the kernel time of the smallest configurations)."""
    s = torch.cuda.current_stream()
    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(s)
    launch()
    e1.record(s)
    host_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    n = max(1, min(max_n, int(target_s * 1000.0 / max(e0.elapsed_time(e1), 1e-3))))
    # Spin-kernel clock rate, then a spin covering twice the host time of n launches (at most 0.5 s).
    e0.record(s)
    torch.cuda._sleep(1 << 20)
    e1.record(s)
    torch.cuda.synchronize()
    cycles_per_ms = (1 << 20) / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(min(500.0, 2.0 * n * host_s * 1e3 + 1.0) * cycles_per_ms))
    e0.record(s)
    for _ in range(n):
        launch()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n, n


def profile_record(config):
    """The committed rocprofv3 counter record of a config's dominant kernel (profiles/traffic.json),
    or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(config_key(config))


def measured_traffic(config):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by what it reads for a plain copy), or None."""
    rec = profile_record(config)
    if not rec:
        return None
    return (rec["fetch_kib"] * rec["fetch_scale"] + rec["write_kib"] * rec["write_scale"]) * 1024.0


def instruction_ceiling(config, cfg, roof, dwork):
    """The VALU instruction ceiling of a VALU-bound dominant kernel: the rate its algorithmic flop
    would reach if every SIMD issued one of the kernel's own wave64 VALU instructions every 2 cycles
    (the full FP32 issue rate the 157.3 TFLOP/s peak assumes, at its 2.4 GHz), from the committed
    SQ_INSTS_VALU count per launch: peak * flop per tap / (2 * VALU lane-instructions per tap).
    `ceiling_frac` = achieved / ceiling says how close the kernel issues to that rate."""
    rec = profile_record(config)
    if not rec or "valu_insts" not in rec or roof["bound"] != "valu":
        return None
    t = taps(cfg)
    per_tap = rec["valu_insts"] * 64.0 / t
    ceiling = roof["peak"] * (dwork / t) / (2.0 * per_tap)
    return {"ceiling": ceiling, "unit": "TFLOP/s", "valu_insts_per_tap": per_tap, "ceiling_frac": roof["achieved"] / ceiling,
            "source": rec.get("profile")}


def host_cpu():
    """nproc, the cores this process may run on, and the CPU model of the host."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "cpu_model": model}


def cpu_baseline(cfg, seconds):
    threads = min(len(os.sched_getaffinity(0)), 16)
    sx = cfg["sample"]["x"]
    spec = dict(kind=cfg["kind"], op=cfg.get("op", cfg.get("first", "dilation")), merge=cfg.get("merge", "sum"), padding="replicate", dtype=cfg["dtype"],
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
    if cfg["dtype"] in ("f16", "bf16"):
        desc += ", in float32 (the reference has no 16-bit path) on the same 16-bit values"
    if cfg["kind"] == "smorph":
        desc += ", alpha = 1 (one point of the sweep)"
    out = {"value": res["output_elements"] / res["seconds_per_step"], "unit": "output-elements/s", "cores": res["threads"],
           "kind": res["kind"], "sample": desc}
    out.update(host_cpu())
    return out


def run_steps(cfg, torch, mca, dev, steps, warmup):
    """Builds a config's inputs, runs `warmup` untimed steps, then times exactly `steps` steps between
    device synchronisations. Returns the timing and the step's state (inputs)."""
    x, ws, dtype = make_inputs(cfg, torch, dev)
    step, n_out, nphase = build_step(cfg, torch, mca, x, ws, dtype, dev)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3 * nphase)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        step(events[k])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = sum(e[3 * p].elapsed_time(e[3 * p + 1]) for e in events for p in range(nphase)) / steps
    bwd_ms = sum(e[3 * p + 1].elapsed_time(e[3 * p + 2]) for e in events for p in range(nphase)) / steps
    ms_per_step = wall * 1000.0 / steps
    return dict(ms_per_step=ms_per_step, fwd_ms=fwd_ms, bwd_ms=bwd_ms, n_out=n_out, x=x, ws=ws, dtype=dtype)


def step_roofline(cfg, ms_per_step, peak):
    """The whole step's algorithmic work (step_work) over the step time, against the same peak."""
    sw = step_work(cfg)
    if sw is None:
        return None
    rate = sw[0] / (ms_per_step * 1e-3)
    if sw[1] == "bytes":
        return {"bound": "hbm", "achieved": rate / 1e9, "unit": "GB/s", "frac": rate / 1e9 / PEAK_HBM_GBS, "work_per_step": sw[0]}
    return {"bound": "valu", "achieved": rate / 1e12, "unit": "TFLOP/s", "frac": rate / 1e12 / peak, "work_per_step": sw[0]}


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
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_launch": n * 4, "launches": args.steps}), flush=True)
        return
    if args.kernel_only:
        x, ws, dtype = make_inputs(cfg, torch, dev)
        launch, _, _, what = dominant(cfg, torch, _native, x, ws, dtype, dev)
        for _ in range(args.steps):
            launch()
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": what, "launches": args.steps}), flush=True)
        return
    r = run_steps(cfg, torch, mca, dev, args.steps, args.warmup)
    ms_per_step = r["ms_per_step"]

    # Roofline of the dominant kernel, timed after the step loop (outside the timed region).
    x, ws, dtype = r["x"].detach(), [w.detach() for w in r["ws"]], r["dtype"]
    launch, dwork, dunit, what = dominant(cfg, torch, _native, x, ws, dtype, dev)
    kms, kn = time_launches(torch, launch)
    executed = getattr(launch, "executed_work", None)
    del launch
    if dunit == "bytes":
        achieved = dwork / (kms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS}
    else:
        peak = PEAK_FP64_TFLOPS if cfg["dtype"] == "f64" else PEAK_FP32_TFLOPS
        achieved = dwork / (kms * 1e-3) / 1e12
        roof = {"bound": "valu", "achieved": achieved, "peak": peak, "unit": "TFLOP/s", "frac": achieved / peak}
        if executed is not None:
            # The work the kernel executes (algorithmic work less what the saved statistics spare it).
            roof["executed_work_per_launch"] = executed
            roof["frac_executed"] = executed / (kms * 1e-3) / 1e12 / peak
    roof["traffic"] = measured_traffic(args.config)
    roof.update({"kernel": what, "kernel_ms": kms, "launches_timed": kn, "work_per_launch": dwork, "work_unit": dunit})
    ceiling = instruction_ceiling(args.config, cfg, roof, dwork)
    if ceiling is not None:
        roof["instruction_ceiling"] = ceiling
        roof["ceiling_frac"] = ceiling["ceiling_frac"]
    line = {
        "metric": METRIC,
        "value": r["n_out"] / (ms_per_step * 1e-3),
        "unit": "output-elements/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "fwd_ms": r["fwd_ms"],
        "bwd_ms": r["bwd_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded torch generators), inputs resident in HBM",
        "config": {"workload": f"{config_key(args.config)}: {cfg['name']}", "x": list(cfg["x"]), "w": list(cfg["w"]),
                   "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "step_roofline": step_roofline(cfg, ms_per_step, roof.get("peak", PEAK_FP32_TFLOPS)),
        "cpu_baseline": None,
    }
    del r, x, ws
    if args.config == 5 and not args.no_extra:
        # configs[2], the smorph alpha sweep the north star's >= 60% target is stated on.
        torch.cuda.empty_cache()
        c3 = CONFIGS[3]
        s3, w3 = DEFAULT_STEPS[3]
        r3 = run_steps(c3, torch, mca, dev, s3 - 1, w3)
        line["configs2_step"] = {"workload": f"configs[2]: {c3['name']}", "steps": s3 - 1, "warmup": w3, "ms_per_step": r3["ms_per_step"],
                                 "fwd_ms": r3["fwd_ms"], "bwd_ms": r3["bwd_ms"], "value": r3["n_out"] / (r3["ms_per_step"] * 1e-3),
                                 "unit": "output-elements/s", "step_roofline": step_roofline(c3, r3["ms_per_step"], PEAK_FP32_TFLOPS)}
        del r3
        torch.cuda.empty_cache()
    if cfg["kind"] in ("pair", "sigma") and not args.no_extra:
        # The same step as the reference writes it: separate operator calls, intermediates in HBM.
        torch.cuda.empty_cache()
        comp = dict(cfg, kind=cfg["kind"] + "_composition")
        rc = run_steps(comp, torch, mca, dev, args.steps, args.warmup)
        desc = ("two operator calls (erosion, then dilation)" if cfg["kind"] == "pair"
                else "two operator calls (erosion, dilation) and torch's blend")
        line["composition_step"] = {"workload": "the same step as " + desc, "ms_per_step": rc["ms_per_step"],
                                    "fwd_ms": rc["fwd_ms"], "bwd_ms": rc["bwd_ms"], "value": rc["n_out"] / (rc["ms_per_step"] * 1e-3)}
        del rc
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
