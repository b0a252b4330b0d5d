"""GradScaler with the torch.amp.GradScaler surface for this package's AdamW.

Drop-in for the scaler the reference builds at train.py:366-370 and drives at
train.py:479-491: scale / unscale_ / step / update, get_scale, the growth and
backoff setters, is_enabled, state_dict / load_state_dict (same five keys,
torch/amp/grad_scaler.py:607-632), and the same stage errors.

What differs is where the work happens:
  - unscale_ touches no gradient: it records the scale on the optimizer's
    engine, and the unscale is applied in registers by the norm pass (when
    clip_grad_norm_ follows) and by the AdamW pass;
  - step never reads found_inf on the host: the skip is decided on the GPU;
  - update runs torch._amp_update_scale_'s state machine in one GPU thread.
"""

from __future__ import annotations

import ctypes
from collections import abc
from typing import Any

import torch

from . import _native as N

#: the keys of a GradScaler state dict, in torch's order (the checkpoint
#: format of src/minigpt/checkpoint.py:40-42 and src/minigpt/optim.py:254-273)
_STATE_KEYS = ("scale", "growth_factor", "backoff_factor", "growth_interval", "_growth_tracker")


class _Iteration:
    """What this scaler has done to one optimizer since the last update():
    whether unscale_ and step ran, and the device flag the norm pass fills."""

    __slots__ = ("unscaled", "stepped", "found_inf")

    def __init__(self) -> None:
        self.unscaled = False
        self.stepped = False
        self.found_inf: torch.Tensor | None = None


class GradScaler:
    def __init__(
        self,
        device: str = "cuda",
        init_scale: float = 2.0**16,
        growth_factor: float = 2.0,
        backoff_factor: float = 0.5,
        growth_interval: int = 2000,
        enabled: bool = True,
    ) -> None:
        self._device = device
        self._enabled = enabled
        self._iters: dict[int, _Iteration] = {}
        if not enabled:
            return
        if device != "cuda":
            raise RuntimeError("this GradScaler runs on the GPU only (device='cuda'); there is no CPU path")
        if not torch.cuda.is_available():
            raise RuntimeError("GradScaler is enabled but no ROCm GPU is visible")
        if not growth_factor > 1.0:
            raise AssertionError("The growth factor must be > 1.0.")
        if not backoff_factor < 1.0:
            raise AssertionError("The backoff factor must be < 1.0.")
        self._growth_factor = growth_factor
        self._backoff_factor = backoff_factor
        self._growth_interval = growth_interval
        # values the device scalars start from when scale() first creates them
        self._init_scale = init_scale
        self._init_growth_tracker = 0
        self._scale: torch.Tensor | None = None
        self._growth_tracker: torch.Tensor | None = None

    def _iteration(self, optimizer) -> _Iteration:
        rec = self._iters.get(id(optimizer))
        if rec is None:
            rec = self._iters[id(optimizer)] = _Iteration()
        return rec

    # --------------------------------------------------------------- scale
    def _check_scale_growth_tracker(self, funcname: str) -> tuple[torch.Tensor, torch.Tensor]:
        fix = "This may indicate your script did not use scaler.scale(loss or outputs) earlier in the iteration."
        if self._scale is None:
            raise AssertionError(f"Attempted {funcname} but _scale is None.  " + fix)
        if self._growth_tracker is None:
            raise AssertionError(f"Attempted {funcname} but _growth_tracker is None.  " + fix)
        return self._scale, self._growth_tracker

    def _lazy_init_scale_growth_tracker(self, dev: torch.device) -> None:
        self._scale = torch.full((), self._init_scale, dtype=torch.float32, device=dev)
        self._growth_tracker = torch.full((), self._init_growth_tracker, dtype=torch.int32, device=dev)

    def scale(self, outputs):
        """outputs * scale, for a tensor or a (nested) list/tuple/iterable of
        them (grad_scaler.py:190-233); the scale and growth tracker are created
        on the first tensor's device."""
        if not self._enabled:
            return outputs
        return self._scaled(outputs)

    def _scaled(self, x):
        if isinstance(x, torch.Tensor):
            if self._scale is None:
                self._lazy_init_scale_growth_tracker(x.device)
            s = self._scale if self._scale.device == x.device else self._scale.to(x.device, non_blocking=True)
            return x * s
        if isinstance(x, (list, tuple)):
            return type(x)(self._scaled(v) for v in x)
        if isinstance(x, abc.Iterable):
            return map(self._scaled, x)
        raise ValueError("outputs must be a Tensor or an iterable of Tensors")

    def _engine_of(self, optimizer) -> Any:
        get = getattr(optimizer, "_get_engine", None)
        if get is None:
            raise TypeError(
                "this GradScaler drives the package's AdamW; use torch.amp.GradScaler for other optimizers"
            )
        return get()

    # ------------------------------------------------------------ unscale_
    def unscale_(self, optimizer) -> None:
        """Records the unscale on the optimizer's engine (grad_scaler.py:288-346)."""
        if not self._enabled:
            return
        self._check_scale_growth_tracker("unscale_")
        rec = self._iteration(optimizer)
        if rec.unscaled and not rec.stepped:
            raise RuntimeError("unscale_() has already been called on this optimizer since the last update().")
        if rec.stepped:
            raise RuntimeError("unscale_() is being called after step().")
        rec.found_inf = self._engine_of(optimizer).request_unscale(self._scale)
        rec.unscaled = True

    # ---------------------------------------------------------------- step
    def step(self, optimizer, *args: Any, **kwargs: Any):
        """Unscale if not done, then the optimizer step with the skip decided
        on the GPU (grad_scaler.py:360-467)."""
        if not self._enabled:
            return optimizer.step(*args, **kwargs)
        if "closure" in kwargs:
            raise RuntimeError("Closure use is not currently supported if GradScaler is enabled.")
        self._check_scale_growth_tracker("step")
        rec = self._iteration(optimizer)
        if rec.stepped:
            raise RuntimeError("step() has already been called since the last update().")
        if not rec.unscaled:
            self.unscale_(optimizer)
        retval = optimizer.step(*args, **kwargs)
        rec.stepped = True
        return retval

    # -------------------------------------------------------------- update
    def update(self, new_scale: float | torch.Tensor | None = None) -> None:
        """torch._amp_update_scale_ on the GPU (grad_scaler.py:469-539)."""
        if not self._enabled:
            return
        _scale, _tracker = self._check_scale_growth_tracker("update")
        if new_scale is not None:
            if isinstance(new_scale, float):
                _scale.fill_(new_scale)
            else:
                reason = (
                    "new_scale should be a float or a 1-element torch.cuda.FloatTensor or "
                    "torch.FloatTensor with requires_grad=False."
                )
                assert new_scale.device.type == self._device, reason
                assert new_scale.numel() == 1, reason
                assert new_scale.requires_grad is False, reason
                _scale.copy_(new_scale)
        else:
            found = [rec.found_inf for rec in self._iters.values() if rec.found_inf is not None]
            if not found:
                raise AssertionError("No inf checks were recorded prior to update.")
            if len(found) > 8:
                raise RuntimeError("at most 8 optimizers per scaler")
            ptrs = tuple(f.data_ptr() for f in found)
            if getattr(self, "_found_ptrs", None) != ptrs:
                # the optimizers' found_inf tensors persist: the pointer array is rebuilt only when they change
                self._found_ptrs, self._found_arr = ptrs, (ctypes.c_void_p * len(ptrs))(*ptrs)
                self._found_addr = ctypes.addressof(self._found_arr)
            # one native call: the launch through the entry point's address
            rc = N.host().scaler_update(
                N.entry_address("mgopt_scaler_update"), _scale.data_ptr(), _tracker.data_ptr(), self._found_addr,
                len(ptrs), float(self._growth_factor), float(self._backoff_factor), int(self._growth_interval),
                N.stream_handle(_scale.device))
            if rc:
                N.check(rc, "mgopt_scaler_update")
        self._iters = {}

    # ------------------------------------------------------------ accessors
    def _get_scale_async(self) -> torch.Tensor | None:
        return self._scale

    def _found_inf_per_device(self, optimizer) -> dict:
        """{device: found_inf} recorded by unscale_ for this optimizer
        (grad_scaler.py:465-467): a device tensor that the coming norm pass
        fills, 1.0 when a scaled gradient is inf or NaN."""
        rec = self._iters.get(id(optimizer))
        return {} if rec is None or rec.found_inf is None else {rec.found_inf.device: rec.found_inf}

    def get_scale(self) -> float:
        if self._enabled:
            return self._init_scale if self._scale is None else float(self._scale.item())
        return 1.0

    def get_growth_factor(self) -> float:
        return self._growth_factor

    def set_growth_factor(self, new_factor: float) -> None:
        self._growth_factor = new_factor

    def get_backoff_factor(self) -> float:
        return self._backoff_factor

    def set_backoff_factor(self, new_factor: float) -> None:
        self._backoff_factor = new_factor

    def get_growth_interval(self) -> int:
        return self._growth_interval

    def set_growth_interval(self, new_interval: int) -> None:
        self._growth_interval = new_interval

    def _get_growth_tracker(self) -> int:
        if self._enabled:
            return self._init_growth_tracker if self._growth_tracker is None else int(self._growth_tracker.item())
        return 0

    def is_enabled(self) -> bool:
        return self._enabled

    def state_dict(self) -> dict[str, Any]:
        """The five values of torch's GradScaler state dict (plain Python
        numbers, so torch.load(weights_only=True) reads them back); {} when
        disabled."""
        if not self._enabled:
            return {}
        values = (self.get_scale(), self._growth_factor, self._backoff_factor, self._growth_interval,
                  self._get_growth_tracker())
        return dict(zip(_STATE_KEYS, values))

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        if not self._enabled:
            return
        if not state_dict:
            raise RuntimeError(
                "The source state dict is empty, possibly because it was saved "
                "from a disabled instance of GradScaler."
            )
        scale, growth, backoff, interval, tracker = (state_dict[k] for k in _STATE_KEYS)
        self._growth_factor, self._backoff_factor = float(growth), float(backoff)
        self._growth_interval = int(interval)
        self._init_scale, self._init_growth_tracker = float(scale), int(tracker)
        # device scalars that already exist take the values in place (a
        # captured or recorded pointer to them stays valid)
        if self._scale is not None:
            self._scale.fill_(self._init_scale)
        if self._growth_tracker is not None:
            self._growth_tracker.fill_(self._init_growth_tracker)

    def __getstate__(self) -> dict[str, Any]:
        # Device scalars and pointer caches stay behind: the unpickled scaler
        # recreates its scalars from the current values at its next scale().
        if self._enabled and self._iters:
            raise AssertionError(
                "A GradScaler instance may only be pickled at the beginning "
                "of an iteration, or at the end after scaler.update()."
            )
        transient = ("_found_ptrs", "_found_arr", "_found_addr")
        state = {k: v for k, v in self.__dict__.items() if k not in transient}
        if self._enabled:
            state.update(_init_scale=self.get_scale(), _init_growth_tracker=self._get_growth_tracker(),
                         _scale=None, _growth_tracker=None)
        return state

    def __setstate__(self, state: dict[str, Any]) -> None:
        self.__dict__.update(state)
