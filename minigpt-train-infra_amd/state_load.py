"""Loading checkpointed optimizer and GradScaler state.

The two loaders the reference's training loop calls on resume
(train.py:376-377), with the behaviour of src/minigpt/optim.py:74-273, so
that a loop can import them from this package with the rest of its helpers.

load_optimizer_state accepts the three checkpoint forms the reference accepts:
  - torch's state_dict whose groups match the optimizer's (same group sizes,
    and the same param_names or a single group on both sides): loaded with
    optimizer.load_state_dict, after which the execution flags of this run's
    groups (fused, foreach, capturable, differentiable) are put back
    (optim.py:147-177);
  - torch's state_dict of another grouping, such as a single group over
    model.parameters(), or one saved before the q/k/v projections were fused
    into qkv_proj: states are matched to parameters by name, the hyper-
    parameters are taken from the saved groups, and the q/k/v states of a
    fused projection are concatenated (optim.py:179-216, 229-251);
  - the teaching version's format: a list with one state per parameter in
    model order, a global step_num and scalar hyper-parameters
    (optim.py:217-240).

One difference, on purpose.  The reference moves every migrated state tensor
to the parameter's dtype (optim.py:124-133).  This package's AdamW keeps
exp_avg, exp_avg_sq and master_param in fp32 whatever the parameter dtype, so
for bf16/fp16 parameters those three are moved to the device in fp32 rather
than rounded to the parameter's dtype first.  For fp32 parameters, and for
optimizers other than this package's AdamW, the two agree.
"""

from __future__ import annotations

from typing import Any

import torch

from .adamw import AdamW

#: group options that select an execution path, kept from the current run
_EXEC_FLAGS = ("fused", "foreach", "capturable", "differentiable")
#: group hyper-parameters a migration takes from the checkpoint
_HPARAMS = ("lr", "betas", "eps", "amsgrad", "maximize")
_PROJECTIONS = ("q_proj", "k_proj", "v_proj")
#: state tensors this package's AdamW keeps in fp32
_FP32_STATE = frozenset(("exp_avg", "exp_avg_sq", "master_param"))


def _optimizer_parameter_names(optimizer: torch.optim.Optimizer, model: torch.nn.Module) -> list[tuple[str, Any]]:
    """(name, parameter) for every parameter of the optimizer, in its group
    order, named as model.named_parameters() names it."""
    name_of = {id(p): n for n, p in model.named_parameters()}
    out = []
    for group in optimizer.param_groups:
        for p in group["params"]:
            if id(p) not in name_of:
                raise ValueError("Optimizer contains a parameter that is not present in the model")
            out.append((name_of[id(p)], p))
    return out


def _unfused_names(names: list[str]) -> list[str]:
    """The parameter names of the same model before the q/k/v projections were
    fused: each attn.qkv_proj.weight stands for q_proj, k_proj and v_proj,
    weight and bias each, in that order; attn.qkv_proj.bias stands for
    nothing more."""
    out: list[str] = []
    for name in names:
        if name.endswith(".attn.qkv_proj.bias"):
            continue
        if name.endswith(".attn.qkv_proj.weight"):
            stem = name[: -len("qkv_proj.weight")]
            out.extend(f"{stem}{proj}.{kind}" for proj in _PROJECTIONS for kind in ("weight", "bias"))
        else:
            out.append(name)
    return out


def _names_for_model_order(model: torch.nn.Module, count: int) -> list[str]:
    """Names of `count` states saved in model order: the model's trainable
    parameters as they are, or as they were before the QKV fusion."""
    current = [n for n, p in model.named_parameters() if p.requires_grad]
    if count == len(current):
        return current
    unfused = _unfused_names(current)
    if count == len(unfused):
        return unfused
    raise ValueError("Optimizer state does not match current or separate-QKV model parameters")


def _fused_projection_state(name: str, states: dict[str, dict[str, Any]]) -> dict[str, Any]:
    """State of a fused qkv_proj weight or bias from the saved q/k/v states:
    tensors with dimensions are concatenated along dim 0, anything else (the
    step) is taken from q_proj.  Empty when any of the three is empty."""
    kind = "weight" if name.endswith("qkv_proj.weight") else "bias"
    stem = name[: -len(f"qkv_proj.{kind}")]
    parts = [states[f"{stem}{proj}.{kind}"] for proj in _PROJECTIONS]
    if not all(parts):
        return {}
    fused: dict[str, Any] = {}
    for key, first in parts[0].items():
        values = [part[key] for part in parts]
        fused[key] = torch.cat(values, dim=0) if isinstance(first, torch.Tensor) and first.ndim > 0 else first
    return fused


def _on_parameter_device(state: dict[str, Any], param: torch.Tensor, keep_fp32: bool) -> dict[str, Any]:
    """The state moved to the parameter's device: the step count in fp32,
    other tensors in the parameter's dtype, except the fp32 state of this
    package's AdamW when keep_fp32."""
    out: dict[str, Any] = {}
    for key, value in state.items():
        if not isinstance(value, torch.Tensor):
            out[key] = value
        elif key == "step" or (keep_fp32 and key in _FP32_STATE):
            out[key] = value.to(device=param.device, dtype=torch.float32)
        else:
            out[key] = value.to(device=param.device, dtype=param.dtype)
    return out


def load_optimizer_state(optimizer: torch.optim.Optimizer, payload: dict[str, Any], model: torch.nn.Module) -> None:
    """Loads a checkpointed optimizer state into `optimizer`, whose parameters
    belong to `model` (src/minigpt/optim.py:136-251; the three accepted forms
    are listed in the module docstring).  Raises ValueError for a parameter
    the model does not own, for param_names that do not match the saved
    parameter ids, for a state list that fits neither the current nor the
    pre-fusion parameter list, and for an unknown format."""
    named = _optimizer_parameter_names(optimizer, model)
    if "param_groups" in payload:
        saved_groups = payload["param_groups"]
        current_groups = optimizer.state_dict()["param_groups"]
        saved_ids = [pid for group in saved_groups for pid in group["params"]]
        saved_names = [n for group in saved_groups for n in group.get("param_names", [])]
        current_names = [n for group in current_groups for n in group.get("param_names", [])]
        same_sizes = len(saved_groups) == len(current_groups) and all(
            len(s["params"]) == len(c["params"]) for s, c in zip(saved_groups, current_groups))
        same_layout = (bool(saved_names) and saved_names == current_names) or (
            len(saved_groups) == 1 and len(current_groups) == 1)
        if len(saved_ids) == len(named) and same_sizes and same_layout:
            flags = [{k: group[k] for k in _EXEC_FLAGS if k in group} for group in optimizer.param_groups]
            optimizer.load_state_dict(payload)
            for group, kept in zip(optimizer.param_groups, flags):
                group.update(kept)
            return
        if saved_names:
            if len(saved_names) != len(saved_ids):
                raise ValueError("Optimizer checkpoint param_names do not match saved parameter IDs")
            source_names = saved_names
        else:
            # saved before the decay / no_decay split: model registration order
            source_names = _names_for_model_order(model, len(saved_ids))
        states = {name: payload["state"].get(pid, {}) for name, pid in zip(source_names, saved_ids)}
        hparams = saved_groups[0]
        saved_by_group = {g["group_name"]: g for g in saved_groups if isinstance(g.get("group_name"), str)}
    else:
        entries = payload.get("state")
        if not isinstance(entries, list):
            raise ValueError("Unsupported optimizer checkpoint format")
        source_names = _names_for_model_order(model, len(entries))
        step = torch.tensor(float(payload["step_num"]), dtype=torch.float32)
        states = {name: {"step": step, **entry} for name, entry in zip(source_names, entries)}
        hparams = {
            "lr": float(payload["lr"]),
            "betas": (float(payload["beta1"]), float(payload["beta2"])),
            "eps": float(payload["eps"]),
            "weight_decay": float(payload["weight_decay"]),
        }
        saved_by_group = {}

    for group in optimizer.param_groups:
        group.update({k: hparams[k] for k in _HPARAMS if k in hparams})
        name = group.get("group_name")
        if name in saved_by_group:
            group["weight_decay"] = saved_by_group[name]["weight_decay"]
        elif name == "no_decay":
            group["weight_decay"] = 0.0
        elif "weight_decay" in hparams:
            group["weight_decay"] = hparams["weight_decay"]

    keep_fp32 = isinstance(optimizer, AdamW)
    optimizer.state.clear()
    for name, param in named:
        if name in states:
            state = states[name]
        elif name.endswith(("qkv_proj.weight", "qkv_proj.bias")):
            state = _fused_projection_state(name, states)
        else:
            state = {}
        if state:
            optimizer.state[param] = _on_parameter_device(state, param, keep_fp32)


def load_grad_scaler_state(scaler, payload: dict[str, Any]) -> None:
    """Loads a checkpointed GradScaler state (src/minigpt/optim.py:254-273):
    torch's five-key state dict as it is, or the teaching version's form
    (enabled, scale, growth factors, growth_interval, growth_tracker).
    Nothing happens for a disabled scaler, an empty payload, or a payload
    saved from a disabled scaler."""
    if not scaler.is_enabled() or not payload:
        return
    if "_growth_tracker" in payload:
        scaler.load_state_dict(payload)
        return
    if not payload.get("enabled", False):
        return
    scaler.load_state_dict({
        "scale": float(payload["scale"]),
        "growth_factor": float(payload["growth_factor"]),
        "backoff_factor": float(payload["backoff_factor"]),
        "growth_interval": int(payload["growth_interval"]),
        "_growth_tracker": int(payload["growth_tracker"]),
    })
