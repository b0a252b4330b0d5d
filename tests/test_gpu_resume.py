"""Continuous-vs-resumed training through a checkpoint, as the reference's
resume acceptance test does (tests/test_resume_consistency.py:76-147): one run
trains 8 iterations straight; another trains 4, saves a checkpoint, and a
fresh process-state (new model, optimizer and scaler) loads it and trains the
remaining 4 on the same batches.  The two final model, optimizer and scaler
states must be equal bit for bit.

The loop is train.py:457-491 (set_optimizer_lr, zero_grad(set_to_none=True),
two micro-batches of scaler.scale(loss).backward(), unscale_,
clip_grad_norm_, step, update) on a model with MiniGPT's parameter structure
(tests/_minigpt.py), with an inf gradient at one step on each side of the
checkpoint so the loss scale backs off in both halves.  The checkpoint is the
dict of src/minigpt/checkpoint.py:28-52 (build_checkpoint_payload), written
with torch.save and read back with torch.load(weights_only=True); the
optimizer and scaler states go back in through this package's
load_optimizer_state and load_grad_scaler_state, the calls of
train.py:376-377 (a native checkpoint: load_state_dict with this run's
execution options kept, src/minigpt/optim.py:161-177).
"""

from __future__ import annotations

import math

import pytest
import torch
from torch import nn

from tests._gpu_harness import log, mg
from tests._minigpt import MiniGPT, batches

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
STEPS, SAVE_AT, INF_AT = 8, 4, (3, 6)


@pytest.fixture(autouse=True, params=[True, False], ids=["three_kernels", "five_kernels"])
def step_form(request, monkeypatch):
    """Every test here runs with the step of a small plan in its three-kernel
    form and again in the five-kernel form of larger plans (MGOPT_FOLD=0 when
    the plans are made)."""
    if not request.param:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    return request.param


def _build(dtype, seed):
    torch.manual_seed(seed)
    model = MiniGPT(dtype=dtype).to(DEV)
    opt = mg.AdamW(mg.build_adamw_param_groups(model, 0.1), lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    scaler = mg.GradScaler("cuda", init_scale=2.0**12, growth_interval=3)
    return model, opt, scaler


def _iterate(model, opt, scaler, data, start, stop):
    for s in range(start, stop + 1):
        mg.set_optimizer_lr(opt, mg.cosine_lr(s - 1, 3e-3, 3e-4, 2, STEPS))
        opt.zero_grad(set_to_none=True)
        x, y = data[s - 1]
        for xm, ym in zip(x.chunk(2), y.chunk(2)):
            loss = nn.functional.cross_entropy(model(xm).flatten(0, 1), ym.flatten()) / 2
            scaler.scale(loss).backward()
        if s in INF_AT:
            model.blocks[0].mlp.fc.weight.grad.view(-1)[5] = float("inf")
        scaler.unscale_(opt)
        mg.clip_grad_norm_(model.parameters(), 1.0)
        scaler.step(opt)
        scaler.update()


def _payload(model, opt, scaler, step):
    """src/minigpt/checkpoint.py:28-52."""
    out = {
        "model_state": model.state_dict(),
        "optimizer_state": opt.state_dict(),
        "scaler_state": scaler.state_dict(),
        "step": step,
        "config": {"model": {"n_layer": 2, "n_head": 4, "n_embd": 64}},
        "best_val_loss": None,
        "rng_state": torch.get_rng_state(),
    }
    out["cuda_rng_state_all"] = torch.cuda.get_rng_state_all()
    return out


def _assert_equal(a, b, path):
    """Nested bitwise equality (tests/test_resume_consistency.py's assert_nested_equal)."""
    if isinstance(a, torch.Tensor):
        assert isinstance(b, torch.Tensor) and a.dtype == b.dtype and a.shape == b.shape, path
        x, y = a.detach().cpu().reshape(-1), b.detach().cpu().reshape(-1)
        if x.dtype.is_floating_point:
            x, y = x.view(torch.uint8), y.view(torch.uint8)     # bit patterns (NaN == NaN)
        assert torch.equal(x, y), path
    elif isinstance(a, dict):
        assert set(a) == set(b), (path, set(a) ^ set(b))
        for k in a:
            _assert_equal(a[k], b[k], f"{path}.{k}")
    elif isinstance(a, (list, tuple)):
        assert len(a) == len(b), path
        for i, (x, y) in enumerate(zip(a, b)):
            _assert_equal(x, y, f"{path}[{i}]")
    elif isinstance(a, float) and math.isnan(a):
        assert isinstance(b, float) and math.isnan(b), path
    else:
        assert a == b, (path, a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_resume_from_checkpoint_is_bit_exact(dtype, tmp_path):
    data = batches(STEPS)
    log(f"case: resume {dtype}, {STEPS} steps, checkpoint after {SAVE_AT}, inf at {INF_AT}")

    model, opt, scaler = _build(dtype, seed=0)
    _iterate(model, opt, scaler, data, 1, STEPS)
    continuous = _payload(model, opt, scaler, STEPS)

    model, opt, scaler = _build(dtype, seed=0)
    _iterate(model, opt, scaler, data, 1, SAVE_AT)
    path = tmp_path / "step_000004.pt"
    torch.save(_payload(model, opt, scaler, SAVE_AT), path)
    del model, opt, scaler

    ckpt = torch.load(path, map_location=DEV, weights_only=True)
    model, opt, scaler = _build(dtype, seed=123)          # different initial weights: everything comes from the file
    model.load_state_dict(ckpt["model_state"])
    # the resume calls of train.py:376-377
    mg.load_optimizer_state(opt, ckpt["optimizer_state"], model)
    mg.load_grad_scaler_state(scaler, ckpt["scaler_state"])
    assert mg.optimizer_completed_steps(opt) == SAVE_AT - 1
    _iterate(model, opt, scaler, data, SAVE_AT + 1, STEPS)
    resumed = _payload(model, opt, scaler, STEPS)
    torch.cuda.synchronize()

    for key in ("model_state", "optimizer_state", "scaler_state", "step"):
        _assert_equal(continuous[key], resumed[key], key)
    assert mg.optimizer_completed_steps(opt) == STEPS - len(INF_AT)
    assert continuous["scaler_state"]["scale"] < 2.0**12
    if dtype == torch.bfloat16:
        assert all("master_param" in e for e in continuous["optimizer_state"]["state"].values())
    log(f"[resume {dtype}] model, optimizer ({len(continuous['optimizer_state']['state'])} entries) and scaler "
        f"states equal bit for bit; scale {continuous['scaler_state']['scale']}")
