"""The reference's optimizer step run with torch 2.10 on the CPU.
TEST INFRASTRUCTURE ONLY (pinning the C oracle, and bench.py's cpu_baseline).

It performs exactly the calls of train.py:483-491 on CPU tensors:

    scaler.unscale_(optimizer)                        # GradScaler("cpu")
    torch.nn.utils.clip_grad_norm_(params, max_norm)
    scaler.step(optimizer)
    scaler.update()

with torch.optim.AdamW(groups, lr, betas, eps, fused=False) as built at
train.py:359-365 (on CPU the reference passes fused=False: runtime.py:164).
"""

from __future__ import annotations

import time

import numpy as np
import torch


class TorchReferencePath:
    def __init__(self, params, group_of, hparams, scaler=None, max_norm=None):
        self.params = [torch.nn.Parameter(torch.from_numpy(np.array(p, np.float32, copy=True))) for p in params]
        groups = []
        for gi, h in enumerate(hparams):
            groups.append({
                "params": [p for p, g in zip(self.params, group_of) if g == gi],
                "weight_decay": h["weight_decay"],
                "betas": tuple(h["betas"]),
                "eps": h["eps"],
                "maximize": h.get("maximize", False),
            })
        self.order = [p for g in groups for p in g["params"]]
        self.opt = torch.optim.AdamW(groups, lr=1e-3, fused=False)
        self.max_norm = max_norm
        if scaler:
            self.scaler = torch.amp.GradScaler(
                "cpu", init_scale=scaler["init_scale"], growth_factor=scaler["growth_factor"],
                backoff_factor=scaler["backoff_factor"], growth_interval=scaler["growth_interval"])
            self.scaler.scale(torch.ones(()))  # creates the scale and growth-tracker tensors
        else:
            self.scaler = torch.amp.GradScaler("cpu", enabled=False)

    def set_grads(self, grads) -> None:
        for p, g in zip(self.params, grads):
            p.grad = None if g is None else torch.from_numpy(np.array(g, np.float32, copy=True))

    def step(self, grads, lr) -> dict:
        """One iteration; grads are fp32 numpy arrays (scaled when the scaler is on)."""
        for g in self.opt.param_groups:
            g["lr"] = lr
        self.set_grads(grads)
        return self.step_prepared()

    def step_prepared(self) -> dict:
        self.scaler.unscale_(self.opt)
        norm = None
        if self.max_norm is not None:
            norm = torch.nn.utils.clip_grad_norm_(self.params, self.max_norm)
        scale_before = self.scaler.get_scale()
        self.scaler.step(self.opt)
        self.scaler.update()
        out = {"norm": None if norm is None else float(norm), "scale_before": scale_before}
        if self.scaler.is_enabled():
            out["scale"] = self.scaler.get_scale()
            out["tracker"] = self.scaler._get_growth_tracker()
        return out

    def state(self, i: int) -> tuple[np.ndarray, np.ndarray, np.ndarray, float]:
        p = self.params[i]
        st = self.opt.state.get(p, {})
        m = st.get("exp_avg", torch.zeros_like(p)).numpy().copy()
        v = st.get("exp_avg_sq", torch.zeros_like(p)).numpy().copy()
        step = float(st["step"]) if "step" in st else 0.0
        return p.detach().numpy().copy(), m, v, step


def time_reference_step(shapes, seed: int = 0, steps: int = 5, scaler: bool = True, threads: int | None = None) -> dict:
    """Median wall time of the reference's CPU step over a parameter set of
    the given shapes (fp32 params, N(0, 1e-2)-like grads), after one warm-up
    step, with a per-stage breakdown (unscale_, clip, step, update)."""
    import os

    torch.set_num_threads(threads or os.cpu_count() or 1)
    gen = torch.Generator().manual_seed(seed)
    params = [torch.nn.Parameter(torch.randn(s, generator=gen) * 0.02) for s in shapes]
    decay = [p for p in params if p.ndim >= 2]
    no_decay = [p for p in params if p.ndim < 2]
    groups = [g for g in ({"params": decay, "weight_decay": 0.1}, {"params": no_decay, "weight_decay": 0.0}) if g["params"]]
    opt = torch.optim.AdamW(groups, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, fused=False)
    sc = torch.amp.GradScaler("cpu", init_scale=65536.0, enabled=scaler)
    sc.scale(torch.ones(()))
    grads = [torch.randn(p.shape, generator=gen) * (1e-2 * 65536.0 if scaler else 1e-2) for p in params]
    rows = []
    for it in range(steps + 1):
        for p, g in zip(params, grads):
            p.grad = g.clone()
        t0 = time.perf_counter()
        sc.unscale_(opt)
        t1 = time.perf_counter()
        torch.nn.utils.clip_grad_norm_(params, 1.0)
        t2 = time.perf_counter()
        sc.step(opt)
        t3 = time.perf_counter()
        sc.update()
        t4 = time.perf_counter()
        if it > 0:
            rows.append((t4 - t0, t1 - t0, t2 - t1, t3 - t2, t4 - t3))
    rows.sort(key=lambda r: r[0])
    med = rows[len(rows) // 2]
    n = sum(p.numel() for p in params)
    return {
        "seconds": med[0], "unscale_s": med[1], "clip_s": med[2], "step_s": med[3], "update_s": med[4],
        "params": n, "tensors": len(params), "threads": torch.get_num_threads(),
    }
