"""GPU parity on 24 seeded random configurations against the oracle: parameter
dtype (fp32, or bf16 / fp16 with an fp32 master), gradient dtype, tensor sizes
(1 element to several 131,072-element pass-1 chunks, odd sizes for the scalar
tails; the 4,096- and 65,536-element tensors as matrices whose state takes the
row layout), chunk size, one or two groups with random betas (both lerp branches),
eps, weight decay and maximize, a GradScaler with a random initial scale and
growth interval or none, clipping or none, and NaN / +inf / -inf injected at a
random position on some steps.

Bar: skip decisions, scale, growth tracker and step counts bit-exact; fp32
state (params or masters, exp_avg, exp_avg_sq) bit-exact; the bf16 / fp16
model copy equal to the round-to-nearest-even image of the master; norms
within 1e-5 relative.

Odd seeds create their plans with MGOPT_FOLD=0, so the five-kernel step is
checked on small sets as well as the three-kernel step of small plans.

MGOPT_RANDOM_CASES=N runs seeds 0..N-1 instead of the default 24.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests._compare import RTOL_NORM, rel
from tests._gpu_harness import host_grad, log, mg, syn, to_f32

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
# matrices whose optimizer state takes the row layout at chunks of up to 4,096
# (16 rows of 4,096 elements; 2 rows of 2,048 at chunks of 512 to 2,048)
SHAPE_OF = {65536: (16, 4096), 4096: (2, 2048)}


def _config(seed: int) -> dict:
    r = np.random.RandomState(5000 + seed)
    pdt = str(r.choice(["f32", "f32", "bf16", "f16"]))
    gdt = str(r.choice(["f32", "f16", "bf16"])) if pdt == "f32" else str(r.choice([pdt, "f32", pdt]))
    n_groups = int(r.randint(1, 3))
    groups = []
    for _ in range(n_groups):
        groups.append(dict(betas=(float(r.choice([0.0, 0.3, 0.5, 0.9, 0.99])), float(r.choice([0.9, 0.95, 0.999]))),
                           eps=float(10.0 ** r.uniform(-10, -3)), weight_decay=float(r.choice([0.0, 0.1, 0.3])),
                           maximize=bool(r.rand() < 0.2)))
    n_tensors = int(r.randint(2, 6))
    sizes = [int(r.choice([1, 7, 64, 1001, 4096, 4099, 65536, 70001, 131073, 300001])) for _ in range(n_tensors)]
    group_of = [k % n_groups for k in range(n_tensors)]
    scaler = None
    if r.rand() < 0.6:
        scaler = dict(init_scale=float(2.0 ** r.randint(4, 17)), growth_factor=2.0, backoff_factor=0.5,
                      growth_interval=int(r.randint(1, 4)))
    if gdt == "f16" and scaler:
        scaler["init_scale"] = min(scaler["init_scale"], 1024.0)   # keep scaled fp16 grads finite
    steps = int(r.randint(3, 7))
    bad = {int(s): float(r.choice([math.nan, math.inf, -math.inf])) for s in r.randint(1, steps + 1, size=2)} \
        if scaler and r.rand() < 0.6 else {}
    return dict(pdt=pdt, gdt=gdt, groups=groups, sizes=sizes, group_of=group_of, scaler=scaler,
                max_norm=None if r.rand() < 0.3 else float(r.choice([0.05, 1.0])), steps=steps, bad=bad,
                chunk=int(r.choice([512, 1024, 4096, 65536])), sigma=float(10.0 ** r.uniform(-3, -1)),
                lr=float(10.0 ** r.uniform(-4, -2)), bad_pos=float(r.rand()))


@pytest.mark.parametrize("seed", list(range(int(os.environ.get("MGOPT_RANDOM_CASES", "24")))))
def test_random_configuration_against_the_oracle(seed, monkeypatch):
    c = _config(seed)
    five = seed % 2 == 1
    if five:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    log(f"case: seed {seed} {c['pdt']}/{c['gdt']} sizes {c['sizes']} chunk {c['chunk']} scaler {bool(c['scaler'])} "
        f"clip {c['max_norm']} bad {sorted(c['bad'])} at {c['bad_pos']:.3f}{' MGOPT_FOLD=0' if five else ''}")
    params = []
    for i, n in enumerate(c["sizes"]):
        p = torch.empty(SHAPE_OF.get(n, (n,)), dtype=DT[c["pdt"]], device=DEV)
        syn.fill_(p, 3, 100 * seed + i, 0.05)
        params.append(torch.nn.Parameter(p))
    groups = []
    for g, h in enumerate(c["groups"]):
        groups.append(dict(params=[p for p, k in zip(params, c["group_of"]) if k == g], **h))
    opt = mg.AdamW(groups, lr=c["lr"], chunk_elems=c["chunk"])
    order = [p for grp in opt.param_groups for p in grp["params"]]          # param_groups order
    index = [next(i for i, p in enumerate(params) if p is q) for q in order]
    sc = mg.GradScaler("cuda", enabled=c["scaler"] is not None, **({} if c["scaler"] is None else c["scaler"]))
    sc.scale(torch.ones((), device=DEV))
    separate = c["gdt"] != c["pdt"]
    grads = [torch.empty(p.shape, dtype=DT[c["gdt"]], device=DEV) for p in order]
    if separate:
        opt.set_grad_source(grads)
    torch.cuda.synchronize()
    init = [p.detach().float().cpu().numpy().copy() for p in order]
    orc = O.OracleRun(init, [c["group_of"][i] for i in index], c["groups"], scaler=c["scaler"], max_norm=c["max_norm"])
    for s in range(1, c["steps"] + 1):
        lr = c["lr"] * (1.0 + 0.05 * s)
        mg.set_optimizer_lr(opt, lr)
        scale = orc.scale if c["scaler"] else 1.0
        for k, g in enumerate(grads):
            syn.fill_(g, 4, (s << 20) | (100 * seed + index[k]), c["sigma"] * scale)
        if s in c["bad"]:
            g = grads[s % len(grads)].view(-1)
            g[int(c["bad_pos"] * g.numel())] = c["bad"][s]
        if not separate:
            for p, g in zip(order, grads):
                p.grad = g
        torch.cuda.synchronize()
        out = orc.step([to_f32(*host_grad(g)) for g in grads], lr)
        sc.unscale_(opt)
        norm = mg.clip_grad_norm_(order, c["max_norm"]) if c["max_norm"] is not None else None
        sc.step(opt)
        sc.update()
        torch.cuda.synchronize()
        if c["scaler"]:
            assert sc.get_scale() == out["scale"] and sc._get_growth_tracker() == out["tracker"], (seed, s)
        if norm is not None:
            n, no = float(norm), out["norm"]
            assert (rel(n, no) <= RTOL_NORM) if math.isfinite(no) else (n == no or (math.isnan(n) and math.isnan(no))), \
                (seed, s, n, no)
    for k, p in enumerate(order):
        st = opt.state[p]
        assert float(st["step"]) == orc.steps[k], (seed, k)
        master = st["master_param"] if "master_param" in st else p
        for got, ref in ((master, orc.p[k]), (st["exp_avg"], orc.m[k]), (st["exp_avg_sq"], orc.v[k])):
            assert np.array_equal(got.detach().cpu().numpy().ravel().view(np.uint32), ref.ravel().view(np.uint32)), \
                (seed, k)
        if "master_param" in st:
            bits = p.detach().view(torch.int16).cpu().numpy().view(np.uint16).ravel()
            want = O.to_bf16(orc.p[k].ravel()) if c["pdt"] == "bf16" else O.to_f16(orc.p[k].ravel())
            assert np.array_equal(bits, want), (seed, k)
    assert opt._engine.device_bc_flag() == 0
    if five:
        assert opt._engine.folded() == 0
