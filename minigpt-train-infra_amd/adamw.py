"""AdamW with the torch.optim.AdamW surface, stepped by libmgopt on one GPU.

Drop-in for the optimizer the reference builds at train.py:359-365: same
constructor arguments, param_groups (any extra keys such as param_names and
group_name are kept), step/zero_grad, and torch-format state_dict
({"state": {i: {"step", "exp_avg", "exp_avg_sq"}}, "param_groups": [...]},
torch/optim/optimizer.py:677-767).

Differences a caller can observe, all by design:
  - optimizer state lives in flat device arenas; optimizer.state[p] holds
    views into them.  Assigning new entries into optimizer.state (as
    src/minigpt/optim.py:242-251 does when migrating checkpoints) or new
    tensors into an entry is picked up and copied into the arenas before the
    next step.  state_dict() entries are fresh dicts holding those views.
  - bf16/fp16 parameters are updated through an fp32 master copy (state key
    "master_param"); exp_avg/exp_avg_sq are always fp32.
  - amsgrad and differentiable are not supported (the reference uses neither).
"""

from __future__ import annotations

import copy
import functools
import weakref
from collections import defaultdict
from itertools import chain
from typing import Any, Iterable

import numpy as np
import torch
from torch.optim import optimizer as _torch_optimizer
from torch.utils.weak import WeakIdKeyDictionary

from .engine import _Engine

#: parameter -> weak reference to the AdamW that owns it, registered when the
#: parameter is added to the optimizer (used by clip_grad_norm_)
_OWNER: WeakIdKeyDictionary = WeakIdKeyDictionary()


def engine_of(param: torch.Tensor) -> _Engine | None:
    """The engine of the AdamW that owns `param` (created on first use), or None."""
    ref = _OWNER.get(param)
    opt = ref() if ref is not None else None
    return None if opt is None else opt._get_engine()


def _step_hooks(func):
    """What torch.optim.Optimizer wraps around a subclass's step()
    (torch/optim/optimizer.py:503-536): global then per-optimizer pre hooks
    (which may replace the arguments), the step, _optimizer_step_code (the
    profiler's Python-tracer anchor), per-optimizer then global post hooks,
    all inside a record_function range named Optimizer.step#<class>.step.
    Here the range is opened only while the autograd profiler runs: outside a
    profile torch's record_function costs ~15 us per call, a third of a small
    model's whole optimizer step.  The `hooked` mark keeps
    Optimizer._patch_step_function (optimizer.py:557-564) from wrapping step()
    again."""

    @functools.wraps(func)
    def wrapper(*args, **kwargs):
        self = args[0]
        if torch.autograd._profiler_enabled():
            with torch.autograd.profiler.record_function(f"Optimizer.step#{type(self).__name__}.step"):
                return _call_with_hooks(func, self, args, kwargs)
        return _call_with_hooks(func, self, args, kwargs)

    wrapper.hooked = True
    return wrapper


def _call_with_hooks(func, self, args, kwargs):
    pre = _torch_optimizer._global_optimizer_pre_hooks
    if pre or self._optimizer_step_pre_hooks:
        for hook in chain(pre.values(), self._optimizer_step_pre_hooks.values()):
            result = hook(self, args, kwargs)
            if result is not None:
                if not (isinstance(result, tuple) and len(result) == 2):
                    raise RuntimeError(f"{func} must return None or a tuple of (new_args, new_kwargs), but got {result}.")
                args, kwargs = result
    out = func(*args, **kwargs)
    self._optimizer_step_code()
    post = _torch_optimizer._global_optimizer_post_hooks
    if post or self._optimizer_step_post_hooks:
        for hook in chain(self._optimizer_step_post_hooks.values(), post.values()):
            hook(self, args, kwargs)
    return out


class _GradMark:
    """Post-accumulate-grad hook of a parameter backed by the gradient arena:
    records that its gradient exists.  Holds only the record, not the
    optimizer."""

    __slots__ = ("present", "i")

    def __init__(self, present: np.ndarray, i: int):
        self.present, self.i = present, i

    def __call__(self, param) -> None:
        self.present[self.i] = 1


class _TrackedEntry(dict):
    """One parameter's optimizer.state entry.  A write into it
    (state[p]["step"] = ..., state[p]["exp_avg"] = ...) changes what torch's
    next step reads; here it marks the optimizer so that the next step copies
    the new value into the arenas."""

    def __init__(self, owner: "weakref.ref[AdamW]", *args):
        super().__init__(*args)
        self._owner = owner

    def _dirty(self) -> None:
        opt = self._owner()
        if opt is not None:
            opt._state_dirty = True

    def __setitem__(self, key, value):
        super().__setitem__(key, value)
        self._dirty()

    def __delitem__(self, key):
        super().__delitem__(key)
        self._dirty()

    def clear(self):
        super().clear()
        self._dirty()

    def update(self, *args, **kwargs):
        super().update(*args, **kwargs)
        self._dirty()

    def pop(self, *args):
        r = super().pop(*args)
        self._dirty()
        return r

    def popitem(self):
        r = super().popitem()
        self._dirty()
        return r

    def setdefault(self, key, default=None):
        r = super().setdefault(key, default)
        self._dirty()
        return r

    def __reduce__(self):
        return (dict, (dict(self),))


class _TrackedState(defaultdict):
    """optimizer.state that notices when entries are replaced or written into."""

    def __init__(self, owner: "AdamW"):
        super().__init__()
        # a weak reference: the optimizer owns this dict, and a cycle would keep
        # its device arenas alive until the cyclic collector runs
        self._owner = weakref.ref(owner)

    def __missing__(self, key):
        # torch's _init_group reads state[p] for a parameter without state.  An
        # empty entry means no state, so creating one needs no copy; a later
        # write into it marks the optimizer.
        entry = _TrackedEntry(self._owner)
        dict.__setitem__(self, key, entry)
        return entry

    def entry(self, values: dict) -> _TrackedEntry:
        return _TrackedEntry(self._owner, values)

    def _dirty(self) -> None:
        owner = self._owner()
        if owner is not None:
            owner._state_dirty = True

    def __setitem__(self, key, value):
        super().__setitem__(key, value)
        self._dirty()

    def __delitem__(self, key):
        super().__delitem__(key)
        self._dirty()

    def clear(self):
        super().clear()
        self._dirty()

    def update(self, *args, **kwargs):
        super().update(*args, **kwargs)
        self._dirty()

    def pop(self, *args):
        r = super().pop(*args)
        self._dirty()
        return r

    def popitem(self):
        r = super().popitem()
        self._dirty()
        return r

    def setdefault(self, key, default=None):
        r = super().setdefault(key, default)
        self._dirty()
        return r

    def __reduce__(self):
        return (dict, (dict(self),))


class AdamW(torch.optim.Optimizer):
    """torch.optim.AdamW (decoupled weight decay), executed by the fused
    unscale + clip + AdamW kernels.  Extra keyword arguments:

    master_weights: None (auto: on for bf16/fp16 params) or True.
    writeback_grads: also store the unscaled, clipped gradient into each
        .grad during the step (the reference leaves them in .grad;
        train.py never reads them after the step, so this is off by default).
    chunk_elems: elements per pass-2 work-group (a multiple of 512); by
        default 2,048 for a set small enough for the three-kernel step at that
        chunk (at most 2,097,152 elements, no tensor of more than 256 chunks),
        1,024 otherwise.
    state_layout: "rows" (default) keeps each parameter's fp32 master,
        exp_avg and exp_avg_sq rows side by side in memory when its row
        length (the smallest product of trailing dimensions that is a
        multiple of chunk_elems, at most 16,384 elements) exists, which the
        update streams measurably faster; optimizer.state[p] then holds
        strided views of p's shape (non-contiguous).  "separate" keeps every
        state tensor contiguous in its own arena.

    capturable=True (torch/optim/adam.py:163-176, 343-346): step() may be
    captured in a HIP graph (torch.cuda.graph) together with the scaler's
    unscale_/step/update and clip_grad_norm_, and replayed.  The kernels then
    read the groups' hyper-parameters from device memory (refresh_hparams, or
    set_optimizer_lr, brings them up to date before a replay) and the step
    counts and bias corrections from device memory; gradients must stay in
    the same buffers as at capture.  Run one step outside capture first.
    """

    # GradScaler.step hands found_inf/grad_scale to the optimizer instead of
    # syncing on the host (torch/amp/grad_scaler.py:403-454).
    _step_supports_amp_scaling = True

    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
        amsgrad: bool = False,
        *,
        maximize: bool = False,
        foreach: bool | None = None,
        capturable: bool = False,
        differentiable: bool = False,
        fused: bool | None = None,
        master_weights: bool | None = None,
        writeback_grads: bool = False,
        chunk_elems: int | None = None,
        state_layout: str = "rows",
    ):
        if isinstance(lr, torch.Tensor) and lr.numel() != 1:
            raise ValueError("Tensor lr must be 1-element")
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if amsgrad:
            raise NotImplementedError("amsgrad is not supported by this AdamW")
        if differentiable:
            raise NotImplementedError("differentiable=True is not supported by this AdamW")
        defaults = dict(
            lr=lr,
            betas=betas,
            eps=eps,
            weight_decay=weight_decay,
            amsgrad=amsgrad,
            maximize=maximize,
            foreach=foreach,
            capturable=capturable,
            differentiable=differentiable,
            fused=fused,
            decoupled_weight_decay=True,
        )
        super().__init__(params, defaults)
        self._master_weights = master_weights
        self._writeback = bool(writeback_grads)
        self._chunk_elems = chunk_elems
        if state_layout not in ("rows", "separate"):
            raise ValueError(f"state_layout must be 'rows' or 'separate', got {state_layout!r}")
        self._state_layout = state_layout
        self._engine: _Engine | None = None
        self._state_dirty = False
        self._installed: set[int] = set()
        self.state = _TrackedState(self)
        self._state_dirty = False

    # ----------------------------------------------------------- internals
    def _get_engine(self) -> _Engine:
        if self._engine is None:
            if torch.cuda.is_current_stream_capturing():
                # creating the engine allocates device and pinned host memory
                # and uploads its tables, none of which a graph can record
                raise RuntimeError("this optimizer has not stepped yet: run one step outside graph capture "
                                   "before capturing")
            capturable = bool(self.defaults.get("capturable")) or any(g.get("capturable") for g in self.param_groups)
            self._engine = _Engine(self, self._master_weights, self._chunk_elems, capturable=capturable,
                                   state_layout=self._state_layout)
        return self._engine

    def _reconcile_state(self) -> None:
        """Copies state entries a caller assigned directly into the arenas."""
        eng = self._get_engine()
        self._sync_all_masters()
        changed = []
        for i, p in enumerate(eng.params):
            entry = dict.get(self.state, p)
            views = eng.views[i]
            if not entry:
                if i in self._installed:
                    # entry removed: the parameter starts from fresh state
                    views["exp_avg"].zero_()
                    views["exp_avg_sq"].zero_()
                    views["step"].zero_()
                    self._installed.discard(i)
                continue
            if all(entry.get(k) is v for k, v in views.items()):
                continue
            changed.append((i, entry))
        self._copy_in_many(changed)
        self._install_views(only_existing=True)
        eng.t_bound = max(eng.t_bound, int(eng.steps.max().item()) if len(eng.params) else 0)
        self._state_dirty = False

    def _copy_in_many(self, items: list[tuple[int, dict[str, Any]]]) -> None:
        """Copies saved per-parameter state into the arenas: every step count
        in one indexed write (no per-parameter .item(), which would wait for
        the GPU when the saved steps live there) and the moments and masters
        in multi-tensor copies (a few launches instead of two or three per
        parameter).  Missing moments start from zero."""
        if not items:
            return
        eng = self._get_engine()
        host_idx: list[int] = []
        host_val: list[float] = []
        dev_idx: list[int] = []
        dev_val: list[torch.Tensor] = []
        dst: list[torch.Tensor] = []
        src: list[torch.Tensor] = []
        zero: list[torch.Tensor] = []
        for i, entry in items:
            views = eng.views[i]
            step = entry.get("step", 0.0)
            if isinstance(step, torch.Tensor) and step.device.type != "cpu":
                dev_idx.append(i)
                dev_val.append(step.reshape(()).to(torch.float32))
            else:
                host_idx.append(i)
                host_val.append(float(step))
            keys = ["exp_avg", "exp_avg_sq"] + (["master_param"] if "master_param" in views else [])
            for key in keys:
                t = entry.get(key)
                if t is None:
                    if key != "master_param":
                        zero.append(views[key])
                    continue
                if t.numel() != views[key].numel():
                    raise ValueError(f"state {key} of parameter {i} has {t.numel()} elements, expected {views[key].numel()}")
                dst.append(views[key])
                src.append(t.reshape(views[key].shape))
        if host_idx:
            eng.steps[torch.tensor(host_idx, device=eng.device)] = torch.tensor(host_val, dtype=torch.float32).to(eng.device)
        if dev_idx:
            eng.steps[torch.tensor(dev_idx, device=eng.device)] = torch.stack(dev_val).to(eng.device)
        if zero:
            torch._foreach_zero_(zero)
        if dst:
            torch._foreach_copy_(dst, src)
        self._installed.update(i for i, _ in items)

    def _sync_all_masters(self, keep: frozenset[int] | set[int] = frozenset()) -> None:
        """Master copies start from the current bf16/fp16 parameters (one
        multi-tensor copy, exact widening); the masters of the tensors in
        `keep` are left alone because a loaded state supplies them."""
        eng = self._get_engine()
        if not eng.has_master or eng.master_synced:
            return
        dst, src = [], []
        for i, p in enumerate(eng.params):
            if "master_param" in eng.views[i] and i not in keep:
                dst.append(eng.views[i]["master_param"])
                src.append(p.detach())
        if dst:
            torch._foreach_copy_(dst, src)
        eng.master_synced = True

    def _install_views(self, only_existing: bool = False) -> None:
        eng = self._get_engine()
        for i, p in enumerate(eng.params):
            if only_existing and i not in self._installed:
                continue
            dict.__setitem__(self.state, p, self.state.entry(eng.views[i]))
            self._installed.add(i)

    # ------------------------------------------------------------ surface
    @_step_hooks
    def step(self, closure=None):
        # No autograd-visible tensor op runs on this path (the kernels write
        # through raw pointers), so grad mode is switched off only around the
        # state copies that need it, not for every call as torch's step does.
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        eng = self._get_engine()
        if torch.cuda.is_current_stream_capturing():
            if not eng.capturable:
                # as torch's non-capturable optimizers refuse (optimizer.py:451-478):
                # a replay would reuse this step's learning rate and host-side state
                raise RuntimeError("Attempting graph capture of step() for an instance of this AdamW, which runs "
                                   "with capturable=False: the learning rate and step bookkeeping are host-side")
            if self._state_dirty:
                raise RuntimeError("optimizer state was written since the last step; run one step outside graph "
                                   "capture first")
        if self._state_dirty:
            with torch.no_grad():
                self._reconcile_state()
        grads = eng.current_grads() if len(self._installed) < len(eng.params) else None
        eng.step(
            found_inf=getattr(self, "found_inf", None),
            grad_scale=getattr(self, "grad_scale", None),
            writeback=self._writeback,
        )
        # torch creates state on a parameter's first step with a grad (adam.py:153-184)
        if grads is not None:
            for i, (p, g) in enumerate(zip(eng.params, grads)):
                if g is not None and i not in self._installed:
                    dict.__setitem__(self.state, p, self.state.entry(eng.views[i]))
                    self._installed.add(i)
        return loss

    def zero_grad(self, set_to_none: bool = True) -> None:
        arena = getattr(self, "_grad_arena", None)
        if arena is not None:
            # the arena persists: one fill, and every p.grad is (again) its view;
            # set_to_none=True forgets which gradients exist, as torch's None does
            arena.zero_()
            eng = self._get_engine()
            for p, g in zip(eng.params, self._grad_views):
                if p.grad is not g:
                    p.grad = g
            if set_to_none and eng.present is not None:
                eng.present[:] = 0
        elif set_to_none and self._engine is not None and self._engine.grad_source is None:
            # the per-parameter `p.grad = None` loop of Optimizer.zero_grad, done natively
            # (3.4 ms of Python at 20,000 parameters)
            self._engine.clear_grads()
        else:
            super().zero_grad(set_to_none=set_to_none)
        if self._engine is not None:
            self._engine.reset_iteration()

    def use_grad_arena(self, dtype: torch.dtype | None = None, track_unused: bool = True) -> torch.Tensor:
        """Backs every parameter's .grad with a view of one flat device buffer
        (segments on 256-byte boundaries, the layout of the moment arenas), so
        gradients are contiguous across the whole parameter set and
        zero_grad() is a single fill whatever set_to_none says; autograd then
        accumulates into the views in place.  dtype: gradient dtype when it
        differs from the parameters' (fp16 gradients for fp32 parameters, for
        instance; sets each parameter's grad_dtype).  Returns the buffer.

        track_unused (default): a post-accumulate-grad hook on each parameter
        records which gradients exist in torch's sense, so a parameter that
        received no gradient since zero_grad(set_to_none=True) is left alone
        by the step (no update, no state), as torch leaves a parameter whose
        .grad is None (torch/optim/adam.py:153); zero_grad(set_to_none=False)
        keeps the record, as torch keeps the zeroed tensors.  The hooks cost
        about a microsecond per parameter and backward.  track_unused=False:
        no hooks, and every arena gradient takes part in every step (torch's
        behaviour when every .grad exists, as after one backward through a
        model that uses all its parameters with set_to_none=False)."""
        eng = self._get_engine()
        dts = {p.dtype for p in eng.params}
        if dtype is None:
            if len(dts) != 1:
                raise ValueError("parameters of several dtypes: pass the gradient dtype explicitly")
            dtype = next(iter(dts))
        if dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise TypeError(f"unsupported gradient dtype {dtype}")
        arena = torch.zeros(max(eng.total, 1), dtype=dtype, device=eng.device)
        views = []
        for p, off in zip(eng.params, eng.offsets):
            if dtype != p.dtype:
                p.grad_dtype = dtype
            views.append(arena[off : off + p.numel()].view(p.shape))
        present = np.array([p.grad is not None for p in eng.params], np.uint8)
        with torch.no_grad():
            for p, g in zip(eng.params, views):
                if p.grad is not None:
                    g.copy_(p.grad)
                p.grad = g
        for h in getattr(self, "_arena_hooks", ()):
            h.remove()
        self._arena_hooks = []
        if track_unused:
            for i, p in enumerate(eng.params):
                self._arena_hooks.append(p.register_post_accumulate_grad_hook(_GradMark(present, i)))
            eng.set_present(present)
        else:
            eng.set_present(None)
        self._grad_arena = arena
        self._grad_views = views
        eng.reset_iteration()
        return arena

    def set_grad_source(self, grads: Iterable[torch.Tensor | None] | None) -> None:
        """Reads gradients from these tensors (one per parameter, in
        param_groups order; fp32, fp16 or bf16) instead of p.grad.  None
        restores p.grad."""
        self._get_engine().set_grad_source(None if grads is None else list(grads))

    def window_metrics(self, reset: bool = True) -> dict:
        """Statistics accumulated on the GPU since the last reset, read with one
        copy: last and maximum clip_grad_norm_ result (maximum with
        torch.maximum's NaN rule, from 0), optimizer steps skipped on inf/NaN and
        taken.  Replaces the per-step window bookkeeping of train.py:487-489 and
        the optimizer-step difference of train.py:501-507."""
        return self._get_engine().window_metrics(reset)

    def refresh_hparams(self) -> None:
        """capturable=True: copies the current param_groups values (lr, weight
        decay, betas, eps) into the device records the kernels read, so that a
        replay of a captured step uses them.  set_optimizer_lr calls it; call it
        after any other change to param_groups before a replay.  Asynchronous;
        a no-op for a non-capturable optimizer or unchanged values."""
        if self._engine is not None and self._engine.capturable:
            self._engine.refresh_hparams()

    def sync_master_from_params(self) -> None:
        """Re-reads bf16/fp16 parameters into the fp32 master copy (after the
        parameters were overwritten outside the optimizer)."""
        self._get_engine().sync_master()

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        old = getattr(self, "_engine", None)
        if old is not None and (getattr(self, "_grad_arena", None) is not None or old.grad_source is not None):
            raise RuntimeError("add_param_group after use_grad_arena or set_grad_source is not supported: "
                               "those gradient buffers are laid out for the current parameters")
        if old is not None and old.captured:
            raise RuntimeError("add_param_group after a step of this optimizer was captured in a HIP graph is not "
                               "supported: the graph reads the current state arenas, which a new group replaces")
        super().add_param_group(param_group)
        me = weakref.ref(self)
        for p in self.param_groups[-1]["params"]:
            _OWNER[p] = me
        if old is not None:
            self._rebuild_engine(old)

    @torch.no_grad()
    def _rebuild_engine(self, old: _Engine) -> None:
        """A new engine over the enlarged parameter list (arenas are laid out
        per parameter list).  The new group comes last, so every existing
        parameter keeps its position; its moments, master copy and step count,
        and the window record, are copied over exactly."""
        self._engine = old                       # state assigned since the last step lands in the old arenas first
        if self._state_dirty:
            self._reconcile_state()
        self._engine = None
        new = self._get_engine()
        self._sync_all_masters()                 # the new parameters' masters from their values
        self._copy_in_many([(i, old.views[i]) for i in sorted(self._installed)])
        new.window.copy_(old.window)
        new.t_bound = old.t_bound
        self._install_views(only_existing=True)
        old.close()

    def state_dict(self) -> dict[str, Any]:
        if self._state_dirty:
            with torch.no_grad():
                self._reconcile_state()
        sd = super().state_dict()
        # plain dicts, as torch's are: torch.load(weights_only=True) refuses
        # any other class, and checkpoints are read that way
        sd["state"] = {k: dict(v) for k, v in sd["state"].items()}
        return sd

    @torch.no_grad()
    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        # torch's order (torch/optim/optimizer.py:877-1017): a shallow copy that
        # the load-state-dict pre hooks may replace, saved groups deep-copied,
        # post hooks after the load
        state_dict = state_dict.copy()
        for pre_hook in self._optimizer_load_state_dict_pre_hooks.values():
            hook_result = pre_hook(self, state_dict)
            if hook_result is not None:
                state_dict = hook_result
        groups = self.param_groups
        saved_groups = copy.deepcopy(state_dict["param_groups"])
        if len(groups) != len(saved_groups):
            raise ValueError("loaded state dict has a different number of parameter groups")
        if any(len(g["params"]) != len(s["params"]) for g, s in zip(groups, saved_groups)):
            raise ValueError("loaded state dict contains a parameter group that doesn't match the size of optimizer's group")
        eng = self._get_engine()
        id_to_param = {}
        for g, s in zip(groups, saved_groups):
            for pid, p in zip(s["params"], g["params"]):
                id_to_param[pid] = p
        index = {id(p): i for i, p in enumerate(eng.params)}
        new_groups = []
        for g, s in zip(groups, saved_groups):
            ng = {k: v for k, v in s.items() if k != "params"}
            ng["params"] = g["params"]
            if "param_names" in g and "param_names" not in ng:
                ng["param_names"] = g["param_names"]
            new_groups.append(ng)
        self.param_groups = new_groups
        # Loading replaces all state: parameters absent from the saved state
        # start fresh.  Nothing a present entry supplies is cleared or
        # re-synced first: the entries may be views of these very arenas (a
        # state_dict() of this optimizer, loaded back), as torch's
        # state_dict() hands out its live tensors.
        items = [(index[id(id_to_param[pid])], entry) for pid, entry in state_dict["state"].items() if pid in id_to_param]
        present = {i for i, _ in items}
        absent = [i for i in range(len(eng.params)) if i not in present]
        fresh = [eng.views[i][k] for i in absent for k in ("exp_avg", "exp_avg_sq")]
        if fresh:
            torch._foreach_zero_(fresh)
        if absent:
            eng.steps[torch.tensor(absent, device=eng.device)] = 0.0
        self._installed.clear()
        eng.master_synced = False
        self._sync_all_masters(keep={i for i, e in items if e.get("master_param") is not None})
        self._copy_in_many(items)
        dict.clear(self.state)
        self._install_views(only_existing=True)
        eng.t_bound = int(eng.steps.max().item())
        eng.reset_iteration()
        self._state_dirty = False
        for post_hook in self._optimizer_load_state_dict_post_hooks.values():
            post_hook(self)

    def __getstate__(self) -> dict[str, Any]:
        # torch pickles defaults, state and param_groups
        # (torch/optim/optimizer.py:415-420); this optimizer's own settings
        # travel with them, the device engine does not
        st = super().__getstate__()
        st["state"] = {k: dict(v) for k, v in self.state.items()}
        st.update(_master_weights=self._master_weights, _writeback=self._writeback, _chunk_elems=self._chunk_elems,
                  _state_layout=self._state_layout)
        return st

    def __setstate__(self, state: dict[str, Any]) -> None:
        super().__setstate__(state)
        self.__dict__.setdefault("_master_weights", None)
        self.__dict__.setdefault("_writeback", False)
        self.__dict__.setdefault("_chunk_elems", None)
        self.__dict__.setdefault("_state_layout", "rows")
        self._engine = None
        self._installed = set()
        tracked = _TrackedState(self)
        dict.update(tracked, self.state)
        self.state = tracked
        # the unpickled state tensors are copied into a new engine's arenas
        # at the first step, as directly assigned state is
        self._state_dirty = bool(tracked)
        me = weakref.ref(self)
        for group in self.param_groups:
            for p in group["params"]:
                _OWNER[p] = me
