"""Host-side helpers the reference's training loop calls around the optimizer
step: parameter grouping and the learning-rate schedule.

Same names, arguments and error behaviour as src/minigpt/optim.py of the
reference, so a training loop can import them from here unchanged.
"""

from __future__ import annotations

import math
from typing import Any

import torch


def build_adamw_param_groups(model: torch.nn.Module, weight_decay: float) -> list[dict[str, Any]]:
    """Two AdamW groups: "decay" (parameters with ndim >= 2: Linear and
    Embedding weights) and "no_decay" (biases and norm weights), each with the
    parameter names attached.  Follows src/minigpt/optim.py:15-64: negative
    weight decay is rejected, frozen parameters are left out, a parameter
    reached twice raises, and the groups must cover every trainable parameter
    exactly once.  Tied weights appear once (named_parameters deduplicates).
    """
    if weight_decay < 0:
        raise ValueError("weight_decay must be non-negative")
    split: dict[str, tuple[list[torch.nn.Parameter], list[str]]] = {"decay": ([], []), "no_decay": ([], [])}
    visited: set[int] = set()
    for name, param in model.named_parameters():
        if not param.requires_grad:
            continue
        if id(param) in visited:
            raise ValueError(f"Model parameter appears more than once: {name}")
        visited.add(id(param))
        params, names = split["decay" if param.ndim >= 2 else "no_decay"]
        params.append(param)
        names.append(name)
    trainable = {id(p) for p in model.parameters() if p.requires_grad}
    if visited != trainable:
        raise ValueError("Optimizer parameter grouping did not cover every trainable model parameter exactly once")
    groups = []
    for group_name, wd in (("decay", weight_decay), ("no_decay", 0.0)):
        params, names = split[group_name]
        groups.append({"params": params, "param_names": names, "group_name": group_name, "weight_decay": wd})
    return groups


def set_optimizer_lr(optimizer: torch.optim.Optimizer, lr: float) -> None:
    """Writes one learning rate into every group (src/minigpt/optim.py:67-71).
    A capturable AdamW of this package also gets the value into the device
    records a captured step reads (an asynchronous copy)."""
    for group in optimizer.param_groups:
        group["lr"] = lr
    refresh = getattr(optimizer, "refresh_hparams", None)
    if refresh is not None:
        refresh()


def cosine_lr(step: int, base_lr: float, min_lr: float, warmup_steps: int, max_steps: int) -> float:
    """Linear warm-up to base_lr over warmup_steps, then a half cosine down to
    min_lr at max_steps, min_lr afterwards (src/minigpt/optim.py:276-289).
    The loop step, not the optimizer step, drives it (train.py:457-463)."""
    if warmup_steps > 0 and step < warmup_steps:
        return base_lr * float(step + 1) / float(warmup_steps)
    if step >= max_steps:
        return min_lr
    span = max(1, max_steps - warmup_steps)
    progress = min(1.0, max(0.0, float(step - warmup_steps) / float(span)))
    return min_lr + 0.5 * (1.0 + math.cos(math.pi * progress)) * (base_lr - min_lr)


def optimizer_completed_steps(optimizer: torch.optim.Optimizer) -> int:
    """Completed AdamW updates, read from the first parameter that has state
    (train.py:162-176).  One device read; call it at log-window boundaries."""
    for group in optimizer.param_groups:
        for param in group["params"]:
            state = optimizer.state.get(param)
            if not state or "step" not in state:
                continue
            step = state["step"]
            return int(step.item()) if isinstance(step, torch.Tensor) else int(step)
    return 0
