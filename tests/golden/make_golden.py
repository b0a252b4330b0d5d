"""Writes the golden vectors under tests/golden/ from torch 2.10.0 on the CPU.

torch is the reference's pinned third-party dependency for every arithmetic
step of the optimizer path (.github/workflows/v06-frozen-review.yml:51-53),
and the reference's own tests hold no numeric vectors for it.  This script
runs the exact torch calls of train.py:483-491 (GradScaler("cpu").unscale_,
clip_grad_norm_, AdamW(fused=False).step, GradScaler.update) and the element
kernels behind them on small seeded inputs, and stores inputs and outputs.

Inputs come from the oracle's synthetic generator (seed/stream recorded, plus
a checksum so a test can confirm the generator still reproduces them).

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402
from oracle.torch_path import TorchReferencePath  # noqa: E402

OUT = Path(__file__).resolve().parent
SIZES = [1, 7, 64, 1000, 4099]


def grads_for(step: int, sizes, sigma: float, seed: int = 2) -> list[np.ndarray]:
    return [O.synth(n, seed, (step << 20) | i, O.synth_k(sigma)) for i, n in enumerate(sizes)]


def digest(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def run_case(name: str, *, steps: int, sigma: float, hparams, scaler=None, max_norm=1.0, inf_at=(), nan_at=(),
             lr_sched=(3e-4, 3e-5, 10, 100)) -> None:
    params = [O.synth(n, 1, i, O.synth_k(0.02)) for i, n in enumerate(SIZES)]
    group_of = [0 if i % 2 == 0 else 1 for i in range(len(SIZES))]
    ref = TorchReferencePath(params, group_of, hparams, scaler=scaler, max_norm=max_norm)
    norms, scales, trackers, lrs, gdig = [], [], [], [], []
    for s in range(1, steps + 1):
        scale = ref.scaler.get_scale() if scaler else 1.0
        grads = grads_for(s, SIZES, sigma * scale)
        if s in inf_at:
            grads[3][17] = np.inf
        if s in nan_at:
            grads[4][4098] = np.nan
        gdig.append(digest(grads))
        lr = O.cosine_lr(s - 1, *lr_sched)
        out = ref.step(grads, lr)
        lrs.append(lr)
        norms.append(np.nan if out["norm"] is None else out["norm"])
        if scaler:
            scales.append(out["scale"])
            trackers.append(out["tracker"])
    meta = dict(steps=steps, sigma=sigma, hparams=hparams, scaler=scaler, max_norm=max_norm, inf_at=list(inf_at),
                nan_at=list(nan_at), lr_sched=list(lr_sched), param_seed=1, param_sigma=0.02, grad_seed=2)
    arrays = {
        "meta": np.array(json.dumps(meta)),
        "sizes": np.array(SIZES, np.int64),
        "group_of": np.array(group_of, np.int64),
        "norms": np.array(norms, np.float32),
        "lrs": np.array(lrs, np.float64),
        "grad_sha256": np.array(gdig),
        "scales": np.array(scales, np.float32),
        "trackers": np.array(trackers, np.int32),
    }
    for i in range(len(SIZES)):
        p, m, v, st = ref.state(i)
        arrays[f"p0_{i}"] = params[i]
        arrays[f"p_{i}"] = p
        arrays[f"m_{i}"] = m
        arrays[f"v_{i}"] = v
        arrays[f"step_{i}"] = np.array(st, np.float64)
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(name, "written")


HP = [dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1), dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)]
SCALER = dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=3)


def elementwise_vectors() -> None:
    """Element kernels: dtype rounding, unscale with non-finite detection,
    clip coefficient, scaler update state machine."""
    rng = np.random.RandomState(7)
    f32 = np.float32
    special = np.array([
        0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 65536.0, 1e-8, 5.96e-8, 2.98e-8,
        2.9802322387695312e-08, 8.940696716308594e-08, 6.103515625e-05, 6.1035e-05, 1.0009765625, 1.00048828125,
        1.0014648437500, 1.00390625, 1.001953125, 1.005859375, 3.4028235e38, 1.1754944e-38, 1e-40, -1e-45,
        0.1, 0.2, 0.3, 1.0 / 3.0,
    ], dtype=f32)
    x = np.concatenate([special, (rng.randn(4000) * np.exp(rng.uniform(-30, 30, 4000))).astype(f32),
                        rng.randn(1000).astype(f32) * f32(1e-5)])
    t = torch.from_numpy(x)
    bf16 = t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    f16 = t.to(torch.float16).view(torch.int16).numpy().view(np.uint16)

    # unscale with a non-finite check (torch._amp_foreach_non_finite_check_and_unscale_)
    g = (rng.randn(3000) * 1000).astype(f32)
    g[[5, 900]] = [np.inf, -np.inf]
    g2 = (rng.randn(3000) * 1000).astype(f32)
    g2[77] = np.nan
    g3 = (rng.randn(3000) * 1000).astype(f32)
    unscale_out = []
    found = []
    inv_list = [2.0**-16, 1.0, 1.0 / 3.0, 0.7, 2.0**-140]
    for inv in inv_list:
        row, frow = [], []
        for arr in (g, g2, g3):
            tt = torch.from_numpy(arr.copy())
            fi = torch.zeros(())
            torch._amp_foreach_non_finite_check_and_unscale_([tt], fi, torch.tensor(f32(inv)))
            row.append(tt.numpy())
            frow.append(float(fi))
        unscale_out.append(np.stack(row))
        found.append(frow)

    # clip coefficient (clip_grad.py:165-174): torch's clip_grads_with_norm_
    # multiplies a unit gradient by exactly the coefficient it computes
    norms = np.array([0.0, 1e-7, 0.5, 0.999999, 1.0, 1.000001, 3.0, 111.6, 1e30, np.inf, np.nan], f32)
    coefs = []
    for max_norm in (1.0, 0.25, 7.5):
        row = []
        for n in norms:
            p = torch.nn.Parameter(torch.zeros(1))
            p.grad = torch.ones(1)
            torch.nn.utils.clip_grads_with_norm_([p], max_norm, torch.tensor(n))
            row.append(float(p.grad[0]))
        coefs.append(row)

    # scaler update state machine (torch._amp_update_scale_)
    cases = []
    for scale0, growth, backoff, interval in [(65536.0, 2.0, 0.5, 3), (1000.0, 1.5, 0.7, 2), (3.0e38, 2.0, 0.5, 1),
                                              (1.0, 3.0, 0.125, 4)]:
        seq = [0, 0, 1, 0, 0, 0, 0, np.nan, 0, 0, 2, 0, 0, 0, 0, 0]
        scale = torch.tensor(f32(scale0))
        tracker = torch.tensor(0, dtype=torch.int32)
        traj = []
        for fi in seq:
            torch._amp_update_scale_(scale, tracker, torch.tensor(f32(fi)), growth, backoff, interval)
            traj.append((float(scale), int(tracker)))
        cases.append((scale0, growth, backoff, interval, seq, traj))
    np.savez_compressed(
        OUT / "elementwise.npz",
        x=x, bf16=bf16, f16=f16,
        unscale_in=np.stack([g, g2, g3]), unscale_inv=np.array(inv_list, np.float32),
        unscale_out=np.stack(unscale_out), unscale_found=np.array(found, np.float32),
        clip_norms=norms, clip_max=np.array([1.0, 0.25, 7.5]), clip_coefs=np.array(coefs, np.float32),
        scaler_params=np.array([c[:4] for c in cases], np.float64),
        scaler_found=np.array([c[4] for c in cases], np.float32),
        scaler_traj_scale=np.array([[s for s, _ in c[5]] for c in cases], np.float32),
        scaler_traj_tracker=np.array([[t for _, t in c[5]] for c in cases], np.int32),
    )
    print("elementwise written")


def main() -> None:
    torch.set_num_threads(1)
    run_case("adamw_noclip", steps=30, sigma=1e-3, hparams=HP)
    run_case("adamw_clip", steps=30, sigma=1e-1, hparams=HP)
    run_case("adamw_noclipcall", steps=12, sigma=1e-3, hparams=HP, max_norm=None)
    run_case("scaler_inf", steps=24, sigma=1e-2, hparams=HP, scaler=SCALER, inf_at=(5, 11), nan_at=(8,))
    hp_odd = [dict(betas=(0.3, 0.5), eps=1e-3, weight_decay=0.5, maximize=True),
              dict(betas=(0.5, 0.999), eps=1e-6, weight_decay=0.0)]
    run_case("adamw_branches", steps=15, sigma=1e-3, hparams=hp_odd, lr_sched=(1e-2, 1e-3, 3, 15))
    elementwise_vectors()


if __name__ == "__main__":
    main()
