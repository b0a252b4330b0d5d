"""Loading checkpointed optimizer and GradScaler state on resume.

The reference's training loop restores its optimizer and scaler through two
loaders (train.py:376-377; behaviour at src/minigpt/optim.py:136-273).  This
module gives a loop the same two calls with the same accepted inputs, built as
three stages:

  1. classify the payload once (`_classify`): torch's state_dict laid out as
     this optimizer's groups ("native"), torch's state_dict of another
     grouping ("by_name"), or the teaching version's per-parameter list
     ("list");
  2. resolve a non-native payload into a `_Resolved` record: every saved state
     keyed by parameter name, plus the hyper-parameters and per-group weight
     decays the groups take on (`_resolve_by_name`, `_resolve_list`);
  3. install the record into the optimizer (`_install`): each parameter takes
     the state saved under its name; a fused q/k/v projection saved as three
     separate projections takes their states joined along dim 0; a parameter
     with neither starts from fresh state.

Saved states without a param_names list are in model registration order,
either of the current model or of the same model before its q/k/v
projections were fused (`_QkvLayout`).

One difference, on purpose: the reference moves every migrated state tensor to
the parameter's dtype (optim.py:124-133).  This package's AdamW keeps
exp_avg, exp_avg_sq and master_param in fp32 whatever the parameter dtype, so
for its bf16/fp16 parameters those three stay fp32.  For fp32 parameters, and
for optimizers other than this package's AdamW, the two agree.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Any, Callable

import torch

from .adamw import AdamW

#: group options that pick an execution path on this machine: the current
#: run's values survive a native load
_RUNTIME_OPTIONS = ("fused", "foreach", "capturable", "differentiable")
#: hyper-parameters every group takes from a migrated checkpoint
_SHARED_HPARAMS = ("lr", "betas", "eps", "amsgrad", "maximize")
#: state entries this package's AdamW holds in fp32 for any parameter dtype
_FP32_ENTRIES = frozenset(("exp_avg", "exp_avg_sq", "master_param"))

#: a fused attention projection: stem, then weight or bias
_FUSED_QKV = re.compile(r"^(?P<stem>.*\.attn\.)qkv_proj\.(?P<kind>weight|bias)$")
_SEPARATE_PROJECTIONS = ("q_proj", "k_proj", "v_proj")

#: the teaching version's scaler keys -> torch's state_dict keys and types
_TEACHING_SCALER = {
    "scale": ("scale", float),
    "growth_factor": ("growth_factor", float),
    "backoff_factor": ("backoff_factor", float),
    "growth_interval": ("growth_interval", int),
    "_growth_tracker": ("growth_tracker", int),
}


class _QkvLayout:
    """A model's trainable parameter names in registration order, as they are
    and as they were before each attention's q/k/v projections were fused
    into one qkv_proj (weight and bias of q_proj, k_proj and v_proj, in that
    order, in place of qkv_proj.weight; nothing in place of qkv_proj.bias)."""

    def __init__(self, model: torch.nn.Module):
        self.current = [n for n, p in model.named_parameters() if p.requires_grad]
        self.separate: list[str] = []
        #: fused name -> the three separate names its state is joined from
        self.parts: dict[str, list[str]] = {}
        for name in self.current:
            hit = _FUSED_QKV.match(name)
            if hit is None:
                self.separate.append(name)
                continue
            stem, kind = hit["stem"], hit["kind"]
            self.parts[name] = [f"{stem}{proj}.{kind}" for proj in _SEPARATE_PROJECTIONS]
            if kind == "weight":
                self.separate += [f"{stem}{proj}.{k}" for proj in _SEPARATE_PROJECTIONS for k in ("weight", "bias")]

    def names_for(self, count: int) -> list[str]:
        """The layout that `count` saved states were written in."""
        for layout in (self.current, self.separate):
            if len(layout) == count:
                return layout
        raise ValueError(f"load_optimizer_state: {count} saved states fit neither the model's "
                         f"{len(self.current)} trainable parameters nor the {len(self.separate)} of its layout "
                         f"before the q/k/v fusion")


@dataclass
class _Resolved:
    """A migrated checkpoint: saved states by parameter name, the
    hyper-parameters every group takes on, and the weight decay of a group
    given its group_name."""

    by_name: dict[str, dict[str, Any]]
    hparams: dict[str, Any]
    decay_of: Callable[[Any, float], float]


def _named_optimizer_params(optimizer: torch.optim.Optimizer, model: torch.nn.Module) -> list[tuple[str, Any]]:
    """(model name, parameter) for each parameter of the optimizer, in its
    param_groups order."""
    names = {id(p): n for n, p in model.named_parameters()}
    out = []
    for p in (p for group in optimizer.param_groups for p in group["params"]):
        if id(p) not in names:
            raise ValueError("load_optimizer_state: the optimizer holds a parameter that model.named_parameters() "
                             "does not yield")
        out.append((names[id(p)], p))
    return out


def _group_sizes(groups: list[dict[str, Any]]) -> list[int]:
    return [len(g["params"]) for g in groups]


def _group_names(groups: list[dict[str, Any]]) -> list[str]:
    return [n for g in groups for n in g.get("param_names", ())]


def _classify(payload: dict[str, Any], optimizer: torch.optim.Optimizer, n_params: int) -> str:
    """'native' (load as it is), 'by_name' (torch format, other grouping) or
    'list' (teaching format)."""
    if "param_groups" not in payload:
        if isinstance(payload.get("state"), list):
            return "list"
        raise ValueError("load_optimizer_state: unrecognised checkpoint; expected torch's optimizer state_dict or "
                         "a list of per-parameter states with step_num and scalar hyper-parameters")
    saved, mine = payload["param_groups"], optimizer.param_groups
    sizes = _group_sizes(saved)
    if sum(sizes) != n_params or sizes != _group_sizes(mine):
        return "by_name"
    saved_names = _group_names(saved)
    if saved_names and saved_names == _group_names(mine):
        return "native"
    return "native" if len(saved) == 1 and len(mine) == 1 else "by_name"


def _load_native(optimizer: torch.optim.Optimizer, payload: dict[str, Any]) -> None:
    """load_state_dict, then this run's execution options back on every group
    (a checkpoint written on a CPU must not switch off the fused path here)."""
    runtime = [{k: g[k] for k in _RUNTIME_OPTIONS if k in g} for g in optimizer.param_groups]
    optimizer.load_state_dict(payload)
    for group, options in zip(optimizer.param_groups, runtime):
        group.update(options)


def _resolve_by_name(payload: dict[str, Any], layout: _QkvLayout) -> _Resolved:
    """torch's state_dict of another grouping: saved states named by the saved
    param_names, else by model order (the checkpoint predates the grouping);
    the first saved group's hyper-parameters; weight decay per group_name."""
    saved = payload["param_groups"]
    ids = [pid for g in saved for pid in g["params"]]
    names = _group_names(saved)
    if names and len(names) != len(ids):
        raise ValueError(f"load_optimizer_state: the checkpoint lists {len(names)} param_names for "
                         f"{len(ids)} saved parameter ids")
    if not names:
        names = layout.names_for(len(ids))
    stored = payload["state"]
    by_name = {name: stored.get(pid, {}) for name, pid in zip(names, ids)}
    named_decay = {g["group_name"]: g["weight_decay"] for g in saved if isinstance(g.get("group_name"), str)}
    first = saved[0]

    def decay_of(group_name, current):
        if group_name in named_decay:
            return named_decay[group_name]
        if group_name == "no_decay":
            return 0.0
        return first.get("weight_decay", current)

    return _Resolved(by_name, {k: first[k] for k in _SHARED_HPARAMS if k in first}, decay_of)


def _resolve_list(payload: dict[str, Any], layout: _QkvLayout) -> _Resolved:
    """The teaching format: one state per parameter in model order, one global
    step_num, scalar lr / beta1 / beta2 / eps / weight_decay."""
    entries = payload["state"]
    names = layout.names_for(len(entries))
    step = torch.tensor(float(payload["step_num"]), dtype=torch.float32)
    hparams = {"lr": float(payload["lr"]), "betas": (float(payload["beta1"]), float(payload["beta2"])),
               "eps": float(payload["eps"])}
    decay = float(payload["weight_decay"])

    def decay_of(group_name, current):
        return 0.0 if group_name == "no_decay" else decay

    return _Resolved({name: dict(entry, step=step) for name, entry in zip(names, entries)}, hparams, decay_of)


def _joined(parts: list[dict[str, Any]]) -> dict[str, Any]:
    """One fused projection's state from its three separate states: tensors
    with dimensions joined along dim 0, anything else (the step count) from
    the first.  Empty when a part has no state."""
    if not all(parts):
        return {}
    head = parts[0]
    out = {}
    for key in head:
        values = [part[key] for part in parts]
        joinable = isinstance(head[key], torch.Tensor) and head[key].dim() > 0
        out[key] = torch.cat(values) if joinable else head[key]
    return out


def _placed(entry: dict[str, Any], param: torch.Tensor, keep_fp32: bool) -> dict[str, Any]:
    """Entry tensors copied to the parameter's device: the step count and (for
    this package's AdamW) its fp32 entries in fp32, others in the parameter's
    dtype."""
    def place(key: str, value: Any) -> Any:
        if not isinstance(value, torch.Tensor):
            return value
        fp32 = key == "step" or (keep_fp32 and key in _FP32_ENTRIES)
        return value.to(device=param.device, dtype=torch.float32 if fp32 else param.dtype)

    return {key: place(key, value) for key, value in entry.items()}


def _install(optimizer: torch.optim.Optimizer, record: _Resolved, named: list[tuple[str, Any]],
             layout: _QkvLayout) -> None:
    for group in optimizer.param_groups:
        group.update(record.hparams)
        group["weight_decay"] = record.decay_of(group.get("group_name"), group["weight_decay"])
    keep_fp32 = isinstance(optimizer, AdamW)
    optimizer.state.clear()
    for name, param in named:
        entry = record.by_name.get(name)
        if entry is None and name in layout.parts:
            entry = _joined([record.by_name.get(part, {}) for part in layout.parts[name]])
        if entry:
            optimizer.state[param] = _placed(entry, param, keep_fp32)


def load_optimizer_state(optimizer: torch.optim.Optimizer, payload: dict[str, Any], model: torch.nn.Module) -> None:
    """Restores a checkpointed optimizer state into `optimizer`, whose
    parameters belong to `model` (the call of train.py:376; accepted forms in
    the module docstring).  Raises ValueError for an optimizer parameter the
    model does not own, for a checkpoint whose param_names and saved ids
    disagree in number, for saved states that fit neither of the model's
    layouts, and for an unrecognised payload."""
    named = _named_optimizer_params(optimizer, model)
    form = _classify(payload, optimizer, len(named))
    if form == "native":
        _load_native(optimizer, payload)
        return
    layout = _QkvLayout(model)
    record = _resolve_list(payload, layout) if form == "list" else _resolve_by_name(payload, layout)
    _install(optimizer, record, named, layout)


def load_grad_scaler_state(scaler, payload: dict[str, Any]) -> None:
    """Restores a checkpointed GradScaler state (the call of train.py:377):
    torch's state_dict, or the teaching version's form (enabled, scale,
    growth_factor, backoff_factor, growth_interval, growth_tracker), which is
    translated to torch's keys first.  A disabled scaler, an empty payload and
    a teaching payload saved with the scaler off leave the scaler as it is."""
    if not scaler.is_enabled() or not payload:
        return
    if "_growth_tracker" not in payload:
        if not payload.get("enabled", False):
            return
        payload = {key: cast(payload[old]) for key, (old, cast) in _TEACHING_SCALER.items()}
    scaler.load_state_dict(payload)
