"""clip_grad_norm_ with torch.nn.utils.clip_grad_norm_'s signature and result.

Called by the reference's loop at train.py:486 on model.parameters().  When
those parameters are exactly the ones (with grads) of one of this package's
AdamW optimizers, the norm pass runs on the optimizer's plan and the clip
coefficient stays on the GPU for the AdamW pass to apply in registers: the
gradients are read once here and once in the step, never rewritten.  Any other
parameter list goes through a grads-only plan and is scaled in place, as
torch/nn/utils/clip_grad.py:120-182 does.
"""

from __future__ import annotations

import ctypes
import types
import warnings
import weakref
from typing import Iterable

import torch

from . import _native as N
from .adamw import engine_of

_GRAD_PLANS: dict[tuple, tuple[int, list[int]]] = {}
_last_fast: tuple[tuple, weakref.ref] | None = None   # (id tuple, engine) of the last fused-path call


def _norm_only(grads: list[torch.Tensor], max_norm: float, error_if_nonfinite: bool) -> torch.Tensor:
    dev = grads[0].device
    if dev.type != "cuda":
        raise RuntimeError("clip_grad_norm_ runs on the GPU only; there is no CPU path")
    for g in grads:
        if g.device != dev:
            raise RuntimeError("clip_grad_norm_ needs all gradients on one GPU")
        if not g.is_contiguous():
            raise RuntimeError("clip_grad_norm_ needs contiguous gradients")
    lib = N.lib()
    key = (dev.index, tuple((N.dtype_code(g.dtype), g.numel()) for g in grads))
    entry = _GRAD_PLANS.get(key)
    if entry is None:
        descs = (N.TensorDesc * len(grads))()
        for i, g in enumerate(grads):
            descs[i].numel = g.numel()
            descs[i].group = 0
            descs[i].grad_dtype = N.dtype_code(g.dtype)
            descs[i].lowp_dtype = N.NONE
        plan = ctypes.c_void_p()
        with torch.cuda.device(dev):
            N.check(lib.mgopt_plan_create(descs, len(grads), 1, None, 65536, ctypes.byref(plan)), "mgopt_plan_create")
        if len(_GRAD_PLANS) > 16:
            old_key = next(iter(_GRAD_PLANS))
            lib.mgopt_plan_destroy(ctypes.c_void_p(_GRAD_PLANS.pop(old_key)[0]))
        entry = (plan.value, [])
        _GRAD_PLANS[key] = entry
    plan = ctypes.c_void_p(entry[0])
    stream = ctypes.c_void_p(N.stream_handle(dev))
    arr = (ctypes.c_void_p * len(grads))(*[g.data_ptr() for g in grads])
    N.check(lib.mgopt_plan_set_grads(plan, arr, stream), "mgopt_plan_set_grads")
    norm = torch.empty((), dtype=torch.float32, device=dev)
    coef = torch.empty((), dtype=torch.float32, device=dev)
    N.check(
        lib.mgopt_grad_norm(plan, None, ctypes.c_double(max_norm), ctypes.c_void_p(norm.data_ptr()),
                            ctypes.c_void_p(coef.data_ptr()), None, stream),
        "mgopt_grad_norm",
    )
    # torch checks finiteness (clip_grad.py:110-116) before it scales (:232)
    _check_finite(norm, error_if_nonfinite)
    N.check(lib.mgopt_scale_grads(plan, ctypes.c_void_p(coef.data_ptr()), stream), "mgopt_scale_grads")
    return norm


# (no no_grad wrapper: nothing here records autograd history, the kernels
# write through raw pointers, and the decorator costs ~2.5 us per call)
def clip_grad_norm_(
    parameters: torch.Tensor | Iterable[torch.Tensor],
    max_norm: float,
    norm_type: float = 2.0,
    error_if_nonfinite: bool = False,
    foreach: bool | None = None,
) -> torch.Tensor:
    """Total L2 norm of the gradients (as one vector), clipping them to
    max_norm: coefficient min(1, max_norm / (norm + 1e-6)), applied with no
    host branch (clip_grad.py:185-233).  Returns the pre-clip norm as a 0-dim
    float32 tensor on the GPU."""
    if float(norm_type) != 2.0:
        raise NotImplementedError("only norm_type=2.0 is implemented")
    if isinstance(parameters, torch.Tensor):
        parameters = [parameters]
    else:
        is_generator = isinstance(parameters, types.GeneratorType)
        parameters = list(parameters)
        if is_generator and len(parameters) == 0:
            warnings.warn("`parameters` is an empty generator, no gradient clipping will occur.", stacklevel=3)
    max_norm = float(max_norm)

    # Fast path: this exact parameter list was seen before and is the whole
    # parameter set of one optimizer (the train.py:486 call, every step).  The
    # last such list is remembered with its engine, which holds the
    # parameters (so their ids cannot be reused while it lives).
    global _last_fast
    key = tuple(map(id, parameters))
    if _last_fast is not None and _last_fast[0] == key and (eng := _last_fast[1]()) is not None:
        total = eng.norm(max_norm)
        _check_finite(total, error_if_nonfinite, eng)
        return total
    eng = engine_of(parameters[0]) if parameters else None
    if eng is not None and key in eng.complete_keys:
        _last_fast = (key, weakref.ref(eng))
        total = eng.norm(max_norm)
        _check_finite(total, error_if_nonfinite, eng)
        return total

    engines = {id(e): e for p in parameters if (e := engine_of(p)) is not None}
    if len(engines) == 1:
        eng = next(iter(engines.values()))
        grads = eng.current_grads()
        mine = {id(p) for p, g in zip(eng.params, grads) if g is not None}
        given = {id(p) for p in parameters if engine_of(p) is eng}
        given_with_grad = {i for i in given if i in mine}
        if len(given) == len(parameters) and given_with_grad == mine:
            if not mine:
                return torch.tensor(0.0)
            if given == {id(p) for p in eng.params} and len(eng.complete_keys) < 8:
                eng.complete_keys.add(key)
            total = eng.norm(max_norm)
            _check_finite(total, error_if_nonfinite, eng)
            return total
    for e in engines.values():
        if e.scale_src is not None:
            raise RuntimeError(
                "clip_grad_norm_ on a parameter list that is not exactly an optimizer's parameters "
                "cannot follow GradScaler.unscale_ of that optimizer"
            )
    grads = [p.grad for p in parameters if p.grad is not None]
    if not grads:
        return torch.tensor(0.0)
    return _norm_only(grads, max_norm, error_if_nonfinite)


def _check_finite(total: torch.Tensor, error_if_nonfinite: bool, eng=None) -> None:
    if error_if_nonfinite and not bool(torch.isfinite(total)):
        if eng is not None:
            # torch raises before clipping, so a step taken anyway uses the
            # unclipped gradients: withdraw the pending coefficient
            eng.clip_pending = False
        raise RuntimeError(
            "The total norm of order 2.0 for gradients from `parameters` is non-finite, so it cannot be "
            "clipped. To disable this error and scale the gradients by the non-finite norm anyway, "
            "set `error_if_nonfinite=False`"
        )
