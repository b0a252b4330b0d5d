"""The CPU oracle against torch 2.10's own CPU path (oracle/torch_path.py: the
calls of train.py:483-491 with AdamW(fused=False), clip_grad_norm_ and
GradScaler("cpu")) over 40 seeded random configurations, beyond the golden
cases: random tensor counts and sizes, betas on both sides of ATen's lerp
switch (1 - beta1 < 0.5 and >= 0.5, beta1 = 0 and 0.5 included), eps from
1e-10 to 1e-2, weight decay, maximize, per-group values, clipping on or off,
a GradScaler with a random initial scale and growth interval, and NaN / +inf /
-inf injected at a random position on some steps.

torch's fp32 norm is replayed into the oracle (as the golden-vector test does)
so that the update itself is compared: skip decisions, scale trajectory and
step counts bit-exact; moments bit-exact; parameters within 1e-6 relative
(torch's vectorised CPU sqrt is not always correctly rounded, the oracle's is).
The oracle's own norm is held to 1e-5 relative of torch's.

MGOPT_RANDOM_CASES=N runs seeds 0..N-1 instead of the default 40.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from oracle.torch_path import TorchReferencePath
from tests._compare import RTOL_NORM, RTOL_STATE, exact_fraction, maxrel, rel

SEEDS = list(range(int(os.environ.get("MGOPT_RANDOM_CASES", "40"))))


def _config(seed: int) -> dict:
    r = np.random.RandomState(1000 + seed)
    n_groups = int(r.randint(1, 3))
    groups = []
    for _ in range(n_groups):
        b1 = float(r.choice([0.0, 0.3, 0.5, 0.6, 0.9, 0.99, r.uniform(0.0, 0.999)]))
        b2 = float(r.choice([0.5, 0.9, 0.95, 0.999, r.uniform(0.5, 0.9999)]))
        groups.append(dict(betas=(b1, b2), eps=float(10.0 ** r.uniform(-10, -2)),
                           weight_decay=float(r.choice([0.0, 0.01, 0.1, r.uniform(0, 0.5)])),
                           maximize=bool(r.rand() < 0.2)))
    n_tensors = int(r.randint(1, 5))
    sizes = [int(r.choice([1, 3, 17, 128, 1000, 4097])) for _ in range(n_tensors)]
    group_of = [int(r.randint(n_groups)) for _ in range(n_tensors)]
    for g in range(n_groups):           # every group holds at least one tensor
        if g not in group_of:
            group_of[g % n_tensors] = g
    groups = [groups[g] for g in sorted(set(group_of))]
    remap = {g: k for k, g in enumerate(sorted(set(group_of)))}
    group_of = [remap[g] for g in group_of]
    scaler = None
    if r.rand() < 0.6:
        scaler = dict(init_scale=float(2.0 ** r.randint(-4, 17)), growth_factor=2.0, backoff_factor=0.5,
                      growth_interval=int(r.randint(1, 5)))
    max_norm = None if r.rand() < 0.3 else float(r.choice([0.1, 1.0, 5.0]))
    steps = int(r.randint(3, 9))
    bad = {int(s): float(r.choice([math.nan, math.inf, -math.inf])) for s in r.randint(1, steps + 1, size=2)} \
        if scaler and r.rand() < 0.7 else {}
    return dict(groups=groups, sizes=sizes, group_of=group_of, scaler=scaler, max_norm=max_norm, steps=steps,
                bad=bad, sigma=float(10.0 ** r.uniform(-4, -1)), lr=float(10.0 ** r.uniform(-5, -1)), seed=seed,
                bad_pos=float(r.rand()))


@pytest.mark.parametrize("seed", SEEDS)
def test_oracle_matches_torch_cpu_on_random_configurations(seed):
    c = _config(seed)
    init = [O.synth(n, 7, 100 * seed + i, O.synth_k(0.05)) for i, n in enumerate(c["sizes"])]
    ref = TorchReferencePath(init, c["group_of"], c["groups"], scaler=c["scaler"], max_norm=c["max_norm"])
    orc = O.OracleRun(init, c["group_of"], c["groups"], scaler=c["scaler"], max_norm=c["max_norm"])
    mine = O.OracleRun(init, c["group_of"], c["groups"], scaler=c["scaler"], max_norm=c["max_norm"])
    for s in range(1, c["steps"] + 1):
        scale = orc.scale if c["scaler"] else 1.0
        grads = [O.synth(n, 8, (s << 20) | (100 * seed + i), O.synth_k(c["sigma"] * scale))
                 for i, n in enumerate(c["sizes"])]
        if s in c["bad"]:
            g = grads[s % len(grads)]
            g[int(c["bad_pos"] * g.size)] = c["bad"][s]
        lr = c["lr"] * (1.0 + 0.1 * s)
        t = ref.step([g.copy() for g in grads], lr)
        o = orc.step([g.copy() for g in grads], lr,
                     norm_override=t["norm"] if c["max_norm"] is not None and t["norm"] is not None else None)
        own = mine.step([g.copy() for g in grads], lr)
        if c["scaler"]:
            assert o["skipped"] == (s in c["bad"]), (seed, s)
            assert (o["scale"], o["tracker"]) == (t["scale"], t["tracker"]), (seed, s, o, t)
        if c["max_norm"] is not None and own["norm"] is not None:
            tn = t["norm"]
            if math.isfinite(tn):
                assert rel(own["norm"], tn) <= RTOL_NORM, (seed, s, own["norm"], tn)
            else:
                assert (math.isnan(tn) and math.isnan(own["norm"])) or own["norm"] == tn, (seed, s)
    for i in range(len(c["sizes"])):
        p, m, v, step = ref.state(i)
        assert orc.steps[i] == step, (seed, i)
        assert exact_fraction(orc.m[i], m.ravel()) == 1.0, (seed, i, "m")
        assert exact_fraction(orc.v[i], v.ravel()) == 1.0, (seed, i, "v")
        assert maxrel(orc.p[i], p.ravel()) <= RTOL_STATE, (seed, i, maxrel(orc.p[i], p.ravel()))
