"""Optimizer-step benchmark on one MI355X.

One step is one pass of the fused hot path over a resident parameter set:
GradScaler.unscale_ -> clip_grad_norm_(max_norm=1.0) -> GradScaler.step
(AdamW) -> GradScaler.update, exactly the call sequence of the reference's
training loop (train.py:483-491), driven through this package's drop-in API.

Default workload: the Qwen3-8B-shaped parameter set (399 tensors,
8,190,735,360 params), bf16 params and grads, fp32 master / exp_avg /
exp_avg_sq (131 GB resident), synthetic data.  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]
    python bench.py --workload uniform_262144x16 --no-cpu-baseline   # 16 fp32 tensors of 16,384 elements
    python bench.py --vs-torch [--workload NAME]   # torch's own GPU step beside this one
"""

from __future__ import annotations

import argparse
import gc
import importlib
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

importlib.import_module("__graft_entry__").ensure_built()   # builds only on a fresh checkout
PKG_DIR = "minigpt-train-infra_amd"
mg = importlib.import_module(PKG_DIR)
syn = importlib.import_module("minigpt-train-infra_amd.synthetic")

METRIC = "optimizer steps/sec + achieved HBM GB/s (% of peak) at Qwen3-8B-shaped 8.2B params"
HBM_PEAK_GBPS = 8000.0
# compulsory bytes per parameter of one executed step, by (param dtype, grad dtype):
# grad read + param (or master) read/write + exp_avg read/write + exp_avg_sq read/write
# (+ the bf16/fp16 model-copy write when a master exists)
ELEM_BYTES = {"f32": 4, "f16": 2, "bf16": 2}


def bytes_per_param(param: str, grad: str) -> int:
    """Compulsory bytes per parameter of one executed step: the gradient
    read, the fp32 param (or master), exp_avg and exp_avg_sq each read and
    written, and the bf16/fp16 model copy written when a master exists."""
    return ELEM_BYTES[grad] + 24 + (ELEM_BYTES[param] if param != "f32" else 0)
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}

WORKLOADS = {
    "qwen3_8b": dict(param="bf16", grad="bf16"),
    "gpt_1p3b": dict(param="bf16", grad="bf16"),
    "gpt2_small": dict(param="f32", grad="f16"),
    "ragged_20k": dict(param="f32", grad="f16"),
    "minigpt_tiny_cpu": dict(param="f32", grad="f32"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# Above this many tensors the synthetic values are written by one generator
# launch into a staging buffer and copied in by multi-tensor copies, instead of
# one launch per tensor: the 20,000-tensor set then takes a few hundred set-up
# dispatches instead of 40,000.  The tensors stay separate allocations.
MANY_TENSORS = 1000
#: steps shorter than 1 ms carry the per-pass HIP events at one step in this many
EVENT_SAMPLE = 16


def fill_tensors(tensors: list[torch.Tensor], seed: int, stream_of, sigma: float) -> None:
    """Synthetic values for a list of tensors: tensor i from stream
    stream_of(i), or, for long lists, all of them from stream stream_of(0)
    through one staging fill."""
    if len(tensors) > MANY_TENSORS:
        syn.fill_many_(tensors, seed, stream_of(0), sigma)
    else:
        for i, t in enumerate(tensors):
            syn.fill_(t, seed, stream_of(i), sigma)


def workload_spec(name: str) -> dict:
    """Parameter and gradient dtypes of a workload (uniform_<n>x<k> sets: fp32)."""
    if name in WORKLOADS:
        return dict(WORKLOADS[name])
    mg.paramsets.shapes_of(name)      # raises for an unknown name
    return dict(param="f32", grad="f32")


def build_workload(name: str, dev: torch.device, param_dtype: str | None = None, grad_dtype: str | None = None):
    spec = workload_spec(name)
    if param_dtype is not None:
        spec["param"] = param_dtype
    if grad_dtype is not None:
        spec["grad"] = grad_dtype
    shapes = mg.paramsets.shapes_of(name)
    decay = [(n, s) for n, s in shapes if len(s) >= 2]
    nodecay = [(n, s) for n, s in shapes if len(s) < 2]
    ordered = decay + nodecay
    raw = [torch.empty(s, dtype=DT[spec["param"]], device=dev) for _, s in ordered]
    fill_tensors(raw, syn.PARAM_SEED, syn.param_stream, 0.02)
    params = [torch.nn.Parameter(p) for p in raw]
    groups = [
        {"params": params[: len(decay)], "param_names": [n for n, _ in decay], "group_name": "decay", "weight_decay": 0.1},
        {"params": params[len(decay):], "param_names": [n for n, _ in nodecay], "group_name": "no_decay", "weight_decay": 0.0},
    ]
    return spec, ordered, params, [g for g in groups if g["params"]]


def time_cpu_baseline(name: str, budget_params: int) -> dict:
    """The reference's CPU step (torch 2.10 on the host cores) on a bounded,
    contiguous sample of the workload's tensors, extrapolated per parameter."""
    from oracle.torch_path import time_reference_step

    shapes = mg.paramsets.shapes_of(name)
    # take tensors in model order (embeddings, then whole layers with their
    # norm weights) until the budget is reached, skipping any single tensor
    # that alone would overshoot it by more than half
    sample, n = [], 0
    for _, s in shapes:
        k = math.prod(s)
        if n >= budget_params:
            break
        if n + k > 1.5 * budget_params and sample:
            continue
        sample.append(s)
        n += k
    total = sum(math.prod(s) for _, s in shapes)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    r = time_reference_step(sample, steps=5, scaler=True, threads=threads)
    ns_per_param = r["seconds"] / r["params"] * 1e9
    return {
        "value": 1.0 / (ns_per_param * 1e-9 * total),
        "unit": "steps/s",
        "cores": r["threads"],
        "kind": "reference",
        "cpu_model": cpu_model(),
        "sample": (f"torch {torch.__version__.split('+')[0]} CPU AdamW(fused=False) + clip_grad_norm_ + "
                   f"GradScaler('cpu'), the calls of train.py:485-491, on {r['tensors']} tensors / {r['params']:,} fp32 params "
                   f"of the workload; median of 5 steps = {r['seconds']*1e3:.1f} ms ({ns_per_param:.3f} ns/param: "
                   f"unscale {r['unscale_s']*1e3:.1f} ms, clip {r['clip_s']*1e3:.1f} ms, step {r['step_s']*1e3:.1f} ms, "
                   f"update {r['update_s']*1e3:.2f} ms), extrapolated to {total:,} params"),
    }


def cpu_model() -> str:
    """The host CPU's model name (first entry of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def read_traffic(name: str) -> float | None:
    """HBM bytes per pass-2 launch measured with rocprofv3 counters, when a
    profile summary for this workload is committed under profiles/."""
    f = ROOT / "profiles" / f"adamw_kernel_{name}_traffic.json"
    if f.exists():
        try:
            return float(json.loads(f.read_text())["bytes_per_launch"])
        except (KeyError, ValueError):
            return None
    return None


def time_device_copy(dev: torch.device, gib: float, stream, launches: int = 6) -> dict:
    """Two reference streams over `gib`-GiB fp32 buffers, timed with HIP
    events on `stream` (the first launch of each untimed):
      - the runtime's device-to-device copy (torch's copy_ -> hipMemcpyAsync,
        run as the runtime's own copy kernel): the buffer read once and
        written once, half reads and half writes like pass 2;
      - torch's fill kernel (fill_) over the destination: writes only.
    Returns the copy's figures, with the fill's under "fill"."""
    n = int(gib * (1 << 30)) // 4
    src = torch.empty(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1.0)

    def timed(op) -> list[float]:
        op()
        spans = []
        for _ in range(launches):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            op()
            b.record(stream)
            spans.append((a, b))
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) for a, b in spans)

    ms = timed(lambda: dst.copy_(src))
    fill_ms = timed(lambda: dst.fill_(2.0))
    moved = 2 * 4 * n
    med, fmed = ms[len(ms) // 2], fill_ms[len(fill_ms) // 2]
    out = {"bytes_per_launch": moved, "launches": launches, "ms": med, "ms_all": ms, "GBps": moved / (med * 1e-3) / 1e9,
           "fill": {"bytes_per_launch": 4 * n, "ms": fmed, "ms_all": fill_ms, "GBps": 4 * n / (fmed * 1e-3) / 1e9}}
    del src, dst
    torch.cuda.empty_cache()
    return out


def vs_torch(name: str, steps: int, warmup: int, dev: torch.device) -> dict:
    """The reference's own GPU path on this GPU, beside this package, on the
    same fp32 parameters and gradients.  On a cuda device the reference's
    loop builds torch.optim.AdamW(..., fused=True) (train.py:359-365 with
    src/minigpt/runtime.py:164) and torch.amp.GradScaler('cuda')
    (train.py:366-370) over fp32 parameters, and calls unscale_ ->
    clip_grad_norm_ -> step -> update (train.py:485-491).  Gradients are
    refilled before every step (torch's unscale_ and clip rewrite them in
    place); HIP events on the current stream bracket only the four calls.
    The two optimizers keep separate state and update the shared parameters
    in turn, each for warmup + steps iterations, twice."""
    _, ordered, params, groups = build_workload(name, dev, param_dtype="f32", grad_dtype="f32")
    n_params = sum(p.numel() for p in params)
    init_scale = 65536.0
    stream = torch.cuda.current_stream(dev)

    def refill(step: int) -> None:
        for p in params:
            if p.grad is None:
                p.grad = torch.empty_like(p)
        fill_tensors([p.grad for p in params], syn.GRAD_SEED, lambda i: syn.grad_stream(step, i), 1e-3 * init_scale)

    def torch_groups():
        return [{k: v for k, v in g.items()} for g in groups]

    runs = {
        "torch": (torch.optim.AdamW(torch_groups(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, fused=True),
                  torch.amp.GradScaler("cuda", init_scale=init_scale), torch.nn.utils.clip_grad_norm_),
        "mgopt": (mg.AdamW(torch_groups(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8),
                  mg.GradScaler("cuda", init_scale=init_scale), mg.clip_grad_norm_),
    }
    ms: dict[str, list[float]] = {k: [] for k in runs}
    for rnd in range(2):
        for key, (opt, scaler, clip) in runs.items():
            scaler.scale(torch.ones((), device=dev))
            spans = []
            for s in range(warmup + steps):
                refill(s + 1)
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                for g in opt.param_groups:
                    g["lr"] = 3e-4
                scaler.unscale_(opt)
                clip(params, 1.0)
                scaler.step(opt)
                scaler.update()
                b.record(stream)
                if s >= warmup:
                    spans.append((a, b))
            torch.cuda.synchronize()
            ms[key].append(sum(a.elapsed_time(b) for a, b in spans) / len(spans))
            log(f"round {rnd}: {key} {ms[key][-1]:.3f} ms/step")
    t, m = min(ms["torch"]), min(ms["mgopt"])
    return {
        "comparison": "the reference's GPU optimizer step (torch AdamW fused=True + torch.amp.GradScaler + "
                      "clip_grad_norm_) vs this package, same GPU, same fp32 params and fp32 grads",
        "workload": name, "tensors": len(params), "params": n_params, "steps": steps, "warmup": warmup,
        "torch_version": torch.__version__,
        "torch_ms_per_step": ms["torch"], "mgopt_ms_per_step": ms["mgopt"],
        "torch_steps_per_s": 1e3 / t, "mgopt_steps_per_s": 1e3 / m,
        "speedup": t / m,
        "compulsory_bytes_per_param": 28,
        "torch_compulsory_GBps": 28 * n_params / (t * 1e-3) / 1e9,
        "mgopt_compulsory_GBps": 28 * n_params / (m * 1e-3) / 1e9,
    }


def time_allocation_round(name: str, dev: torch.device, steps: int, warmup: int, state_layout: str = "rows",
                          chunk_elems: int | None = None, param_dtype: str | None = None) -> dict:
    """The workload built again from fresh allocations in this process (after
    the previous round's memory went back to the driver), its two passes timed
    with HIP events at every step, then released.  The same pass over the same
    sizes can run at a different speed depending on which physical memory
    backs its buffers; rounds in one process show that spread apart from the
    kernel."""
    spec, _, params, groups = build_workload(name, dev, param_dtype)
    opt = mg.AdamW(groups, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, state_layout=state_layout, chunk_elems=chunk_elems)
    scaler = mg.GradScaler("cuda", init_scale=65536.0)
    scaler.scale(torch.ones((), device=dev))
    grads = [torch.empty(p.shape, dtype=DT[spec["grad"]], device=dev) for p in params]
    fill_tensors(grads, syn.GRAD_SEED, lambda i: syn.grad_stream(1, i), 1e-3 * 65536.0)
    if spec["grad"] == spec["param"]:
        for p, g in zip(params, grads):
            p.grad = g
    else:
        opt.set_grad_source(grads)
    stream = torch.cuda.current_stream(dev)
    spans = []
    for k in range(warmup + steps):
        mg.set_optimizer_lr(opt, 3e-4)
        scaler.unscale_(opt)
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record(stream)
        mg.clip_grad_norm_(params, 1.0)
        b.record(stream)
        scaler.step(opt)
        c.record(stream)
        scaler.update()
        if k >= warmup:
            spans.append((a, b, c))
    torch.cuda.synchronize()
    norm = sorted(a.elapsed_time(b) for a, b, _ in spans)
    adamw = sorted(b.elapsed_time(c) for _, b, c in spans)
    out = {"norm_ms": norm[len(norm) // 2], "adamw_ms": adamw[len(adamw) // 2], "adamw_ms_min": adamw[0],
           "adamw_ms_max": adamw[-1]}
    del opt, scaler, grads, params, groups
    gc.collect()
    torch.cuda.empty_cache()
    return out


def _workload_name(name: str) -> str:
    try:
        workload_spec(name)
    except (KeyError, ValueError) as e:
        raise argparse.ArgumentTypeError(str(e)) from None
    return name


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=15)
    ap.add_argument("--workload", default="qwen3_8b", type=_workload_name, metavar="NAME",
                    help=f"one of {', '.join(sorted(WORKLOADS))}, or uniform_<params>x<tensors> (fp32 tensors "
                         "of equal size, to see how the step scales)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-params", type=int, default=1_000_000_000)
    ap.add_argument("--vs-torch", action="store_true",
                    help="instead of the benchmark line, time torch's own GPU path (the reference's fused AdamW + "
                         "GradScaler + clip_grad_norm_) beside this package on fp32 params and grads of the workload")
    ap.add_argument("--graph", action="store_true",
                    help="AdamW(capturable=True): capture the whole step in one HIP graph after the warm-up and "
                         "time its replays (for small sets, whose eager step is bound by the host's launches)")
    ap.add_argument("--copy-ceiling", type=float, default=0.0, metavar="GIB",
                    help="after the timed steps, also time the runtime's own device-to-device copy "
                         "(hipMemcpyAsync, torch's copy_) of a GIB-gibibyte buffer and torch's fill of it "
                         "(writes only) in this process, and report pass 2's rate against the copy")
    ap.add_argument("--state-layout", choices=("rows", "separate"), default="rows",
                    help="AdamW(state_layout=...): each parameter's master / exp_avg / exp_avg_sq rows side by side "
                         "(rows, the default) or each in its own contiguous arena (separate)")
    ap.add_argument("--param-dtype", choices=("bf16", "f16", "f32"), default=None,
                    help="the workload's parameters in this dtype instead of its own (gradients keep theirs); "
                         "bf16/fp16 parameters get fp32 masters")
    ap.add_argument("--chunk-elems", type=int, default=None, metavar="N",
                    help="AdamW(chunk_elems=N): elements per pass-2 work-group (a multiple of 512; default 1,024)")
    ap.add_argument("--alloc-rounds", type=int, default=0, metavar="R",
                    help="after the benchmark line's measurement, release the workload and build it again from "
                         "fresh allocations R times in this process, timing both passes in each round (the spread "
                         "that physical placement alone causes); reported under alloc_rounds")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB fp32 device copy (reads 1 GiB, writes 1 GiB) three times, "
                         "to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.alloc_rounds and args.graph:
        ap.error("--alloc-rounds times eager steps; it does not combine with --graph")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the optimizer step here has no multi-GPU path (use --gpus 1)", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30, "launches": 3}))
        return 0
    if args.vs_torch:
        print(json.dumps(vs_torch(args.workload, args.steps, args.warmup, dev)), flush=True)
        return 0
    spec, ordered, params, groups = build_workload(args.workload, dev, args.param_dtype)
    n_params, n_tensors = sum(p.numel() for p in params), len(params)
    log(f"workload {args.workload}: {len(params)} tensors, {n_params:,} params ({spec['param']} params, {spec['grad']} grads)")

    init_scale = 65536.0
    opt = mg.AdamW(groups, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, capturable=args.graph, state_layout=args.state_layout,
                   chunk_elems=args.chunk_elems)
    scaler = mg.GradScaler("cuda", init_scale=init_scale, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000)
    scaler.scale(torch.ones((), device=dev))
    grads = [torch.empty(p.shape, dtype=DT[spec["grad"]], device=dev) for p in params]
    fill_tensors(grads, syn.GRAD_SEED, lambda i: syn.grad_stream(1, i), 1e-3 * init_scale)
    if spec["grad"] == spec["param"]:
        for p, g in zip(params, grads):
            p.grad = g
    else:
        opt.set_grad_source(grads)
    del grads
    eng = opt._get_engine()
    torch.cuda.synchronize()
    log(f"resident: {torch.cuda.memory_allocated(dev) / 1e9:.1f} GB (parameters, gradients, optimizer state)")
    stream = torch.cuda.current_stream(dev)
    ev = {"norm": [], "adamw": []}

    def one_step(record: bool) -> None:
        mg.set_optimizer_lr(opt, 3e-4)
        scaler.unscale_(opt)
        if record:
            a = torch.cuda.Event(enable_timing=True)
            a.record(stream)
        mg.clip_grad_norm_(params, 1.0)
        if record:
            b = torch.cuda.Event(enable_timing=True)
            b.record(stream)
        scaler.step(opt)
        if record:
            c = torch.cuda.Event(enable_timing=True)
            c.record(stream)
            ev["norm"].append((a, b))
            ev["adamw"].append((b, c))
        scaler.update()

    for _ in range(args.warmup):
        one_step(False)
    torch.cuda.synchronize()
    if args.graph:
        # the whole step (unscale_, clip_grad_norm_, step, update) in one HIP
        # graph; each timed step refreshes the learning rate and replays it
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            scaler.unscale_(opt)
            mg.clip_grad_norm_(params, 1.0)
            scaler.step(opt)
            scaler.update()

        def one_step(record: bool) -> None:
            mg.set_optimizer_lr(opt, 3e-4)
            if record:
                a = torch.cuda.Event(enable_timing=True)
                a.record(stream)
            graph.replay()
            if record:
                b = torch.cuda.Event(enable_timing=True)
                b.record(stream)
                ev["adamw"].append((a, b))

        one_step(False)
        torch.cuda.synchronize()
    # Steps of a millisecond or more carry the per-pass HIP events at every
    # step.  Shorter ones (small sets, whose step is a few launches) carry them
    # at every EVENT_SAMPLE-th step only: three event records cost about as
    # much host time as the step itself there, and would be measured with it.
    probe = time.perf_counter()
    for _ in range(5):
        one_step(False)
    torch.cuda.synchronize()
    every = 1 if (time.perf_counter() - probe) / 5 >= 1e-3 else EVENT_SAMPLE
    t0 = time.perf_counter()
    for k in range(args.steps):
        one_step(k % every == 0)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    step_s = (t1 - t0) / args.steps
    taken = args.steps + args.warmup + 5 + (1 if args.graph else 0)
    skipped = int(round(taken - float(eng.steps.max())))
    if eng.device_bc_flag() != 0 or skipped != 0:
        log(f"bias corrections evaluated on the device: {eng.device_bc_flag()}, skipped {skipped}")
        return 1
    # graph mode: one replay holds both passes, so "adamw" times the whole step
    norm_ms = sum(a.elapsed_time(b) for a, b in ev["norm"]) / len(ev["norm"]) if ev["norm"] else 0.0
    adamw_ms = sum(a.elapsed_time(b) for a, b in ev["adamw"]) / len(ev["adamw"])

    bpp = bytes_per_param(spec["param"], spec["grad"])
    grad_bytes = 2 if spec["grad"] != "f32" else 4
    achieved_step = bpp * n_params / step_s / 1e9
    adamw_gbps = bpp * n_params / (adamw_ms * 1e-3) / 1e9
    norm_gbps = grad_bytes * n_params / (norm_ms * 1e-3) / 1e9 if norm_ms else 0.0
    log(f"step {step_s*1e3:.3f} ms ({1/step_s:.2f} steps/s); compulsory {bpp} B/param -> {achieved_step:.0f} GB/s "
        f"({100*achieved_step/HBM_PEAK_GBPS:.1f}% of peak); norm pass {norm_ms:.3f} ms ({norm_gbps:.0f} GB/s), "
        f"AdamW pass {adamw_ms:.3f} ms ({adamw_gbps:.0f} GB/s)")

    copy = None
    if args.copy_ceiling > 0:
        copy = time_device_copy(dev, args.copy_ceiling, stream)
        log(f"runtime copy of {args.copy_ceiling:g} GiB: {copy['ms']:.3f} ms = {copy['GBps']:.0f} GB/s "
            f"(read + write); pass 2 runs at {adamw_gbps / copy['GBps']:.3f} of it")
        log(f"fill of {args.copy_ceiling:g} GiB (writes only): {copy['fill']['ms']:.3f} ms = "
            f"{copy['fill']['GBps']:.0f} GB/s")

    rounds = None
    if args.alloc_rounds > 0:
        first = {"norm_ms": norm_ms, "adamw_ms": adamw_ms}
        del one_step, opt, scaler, eng, params, groups, ordered
        ev.clear()
        gc.collect()
        torch.cuda.empty_cache()
        rounds = [first]
        for r in range(1, args.alloc_rounds + 1):
            rounds.append(time_allocation_round(args.workload, dev, max(args.steps, 5), max(args.warmup, 2),
                                                args.state_layout, args.chunk_elems, args.param_dtype))
            log(f"allocation round {r}: norm pass {rounds[-1]['norm_ms']:.3f} ms, AdamW pass "
                f"{rounds[-1]['adamw_ms']:.3f} ms")

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the reference's CPU step on a bounded sample ...")
        try:
            cpu = time_cpu_baseline(args.workload, args.cpu_sample_params)
            log(f"cpu baseline {cpu['value']:.5f} steps/s on {cpu['cores']} threads")
        except Exception as e:  # the GPU measurement above stands without it
            log(f"cpu baseline failed: {type(e).__name__}: {e}")
            cpu = {"value": None, "unit": "steps/s", "cores": None, "kind": "reference",
                   "sample": f"not measured: {type(e).__name__}: {e}"}

    out = {
        "metric": METRIC,
        "value": 1.0 / step_s,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded counter-hash generator; random-init parameters of the named shapes)",
        "config": {
            "workload": args.workload,
            "tensors": n_tensors,
            "params": n_params,
            "param_dtype": spec["param"],
            "grad_dtype": spec["grad"],
            "state": ("fp32 master/exp_avg/exp_avg_sq" if spec["param"] != "f32" else "fp32 exp_avg/exp_avg_sq")
                     + f", layout {args.state_layout}"
                     + (f", pass-2 chunks of {args.chunk_elems}" if args.chunk_elems else ""),
            "step": "GradScaler.unscale_ + clip_grad_norm_(1.0) + AdamW + GradScaler.update"
                    + (", captured in one HIP graph and replayed (AdamW capturable=True)" if args.graph else ""),
            "parallelism": "single GPU",
        },
        "achieved_GBps": achieved_step,
        "pct_of_hbm_peak": 100.0 * achieved_step / HBM_PEAK_GBPS,
        "bytes_per_param": bpp,
        # what the two passes move: the gradients are read once more by the norm pass
        "implementation_bytes_per_param": bpp + grad_bytes,
        "implementation_GBps": (bpp + grad_bytes) * n_params / step_s / 1e9,
        "skipped_steps": skipped,
        "passes_ms": {"graph_replay": adamw_ms} if args.graph else {"norm": norm_ms, "adamw": adamw_ms},
        "pass_events_every": every,
        "roofline": {
            "bound": "hbm",
            "achieved": adamw_gbps,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": adamw_gbps / HBM_PEAK_GBPS,
            "traffic": read_traffic(args.workload),
        },
        "cpu_baseline": cpu,
    }
    if copy is not None:
        copy["adamw_frac_of_copy"] = adamw_gbps / copy["GBps"]
        out["copy_ceiling"] = copy
    if rounds is not None:
        out["alloc_rounds"] = rounds
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
