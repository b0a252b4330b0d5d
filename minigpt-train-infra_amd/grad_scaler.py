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
from collections import abc, defaultdict
from enum import Enum
from typing import Any, Iterable

import torch

from . import _native as N


class OptState(Enum):
    READY = 0
    UNSCALED = 1
    STEPPED = 2


def _refresh_per_optimizer_state() -> dict[str, Any]:
    return {"stage": OptState.READY, "found_inf_per_device": {}}


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
        if self._enabled:
            if device != "cuda":
                raise RuntimeError("this GradScaler runs on the GPU only (device='cuda'); there is no CPU path")
            if not torch.cuda.is_available():
                raise RuntimeError("GradScaler is enabled but no ROCm GPU is visible")
            if not growth_factor > 1.0:
                raise AssertionError("The growth factor must be > 1.0.")
            if not backoff_factor < 1.0:
                raise AssertionError("The backoff factor must be < 1.0.")
            self._init_scale = init_scale
            self._scale: torch.Tensor | None = None
            self._growth_factor = growth_factor
            self._backoff_factor = backoff_factor
            self._growth_interval = growth_interval
            self._init_growth_tracker = 0
            self._growth_tracker: torch.Tensor | None = None
            self._per_optimizer_states: dict[int, dict[str, Any]] = defaultdict(_refresh_per_optimizer_state)

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
        """outputs * scale (grad_scaler.py:190-233)."""
        if not self._enabled:
            return outputs
        if isinstance(outputs, torch.Tensor):
            if self._scale is None:
                self._lazy_init_scale_growth_tracker(outputs.device)
            return outputs * self._scale.to(device=outputs.device, non_blocking=True)

        def apply(val):
            if isinstance(val, torch.Tensor):
                if self._scale is None:
                    self._lazy_init_scale_growth_tracker(val.device)
                return val * self._scale.to(device=val.device, non_blocking=True)
            if isinstance(val, abc.Iterable):
                mapped = map(apply, val)
                if isinstance(val, (list, tuple)):
                    return type(val)(mapped)
                return mapped
            raise ValueError("outputs must be a Tensor or an iterable of Tensors")

        return apply(outputs)

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
        state = self._per_optimizer_states[id(optimizer)]
        if state["stage"] is OptState.UNSCALED:
            raise RuntimeError("unscale_() has already been called on this optimizer since the last update().")
        if state["stage"] is OptState.STEPPED:
            raise RuntimeError("unscale_() is being called after step().")
        engine = self._engine_of(optimizer)
        found_inf = engine.request_unscale(self._scale)
        state["found_inf_per_device"] = {found_inf.device: found_inf}
        state["stage"] = OptState.UNSCALED

    # ---------------------------------------------------------------- step
    def step(self, optimizer, *args: Any, **kwargs: Any):
        """Unscale if not done, then the optimizer step with the skip decided
        on the GPU (grad_scaler.py:360-467)."""
        if not self._enabled:
            return optimizer.step(*args, **kwargs)
        if "closure" in kwargs:
            raise RuntimeError("Closure use is not currently supported if GradScaler is enabled.")
        self._check_scale_growth_tracker("step")
        state = self._per_optimizer_states[id(optimizer)]
        if state["stage"] is OptState.STEPPED:
            raise RuntimeError("step() has already been called since the last update().")
        if state["stage"] is OptState.READY:
            self.unscale_(optimizer)
        retval = optimizer.step(*args, **kwargs)
        state["stage"] = OptState.STEPPED
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
            found = [
                f for s in self._per_optimizer_states.values() for f in s["found_inf_per_device"].values()
            ]
            if not found:
                raise AssertionError("No inf checks were recorded prior to update.")
            if len(found) > 8:
                raise RuntimeError("at most 8 optimizers per scaler")
            ptrs = tuple(f.data_ptr() for f in found)
            if getattr(self, "_found_ptrs", None) != ptrs:
                # the optimizers' found_inf tensors persist: the pointer array is rebuilt only when they change
                self._found_ptrs, self._found_arr = ptrs, (ctypes.c_void_p * len(ptrs))(*ptrs)
            N.check(
                N.lib().mgopt_scaler_update(
                    _scale.data_ptr(), _tracker.data_ptr(), self._found_arr, len(ptrs),
                    float(self._growth_factor), float(self._backoff_factor), int(self._growth_interval),
                    N.stream_handle(_scale.device),
                ),
                "mgopt_scaler_update",
            )
        self._per_optimizer_states = defaultdict(_refresh_per_optimizer_state)

    # ------------------------------------------------------------ accessors
    def _get_scale_async(self) -> torch.Tensor | None:
        return self._scale

    def _found_inf_per_device(self, optimizer) -> dict:
        """{device: found_inf} recorded by unscale_ for this optimizer
        (grad_scaler.py:465-467): a device tensor that the coming norm pass
        fills, 1.0 when a scaled gradient is inf or NaN."""
        return self._per_optimizer_states[id(optimizer)]["found_inf_per_device"]

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
        if self._enabled:
            return {
                "scale": self.get_scale(),
                "growth_factor": self._growth_factor,
                "backoff_factor": self._backoff_factor,
                "growth_interval": self._growth_interval,
                "_growth_tracker": self._get_growth_tracker(),
            }
        return {}

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        if not self._enabled:
            return
        if len(state_dict) == 0:
            raise RuntimeError(
                "The source state dict is empty, possibly because it was saved "
                "from a disabled instance of GradScaler."
            )
        self._init_scale = float(state_dict["scale"])
        if self._scale is not None:
            self._scale.fill_(state_dict["scale"])
        self._growth_factor = float(state_dict["growth_factor"])
        self._backoff_factor = float(state_dict["backoff_factor"])
        self._growth_interval = int(state_dict["growth_interval"])
        self._init_growth_tracker = int(state_dict["_growth_tracker"])
        if self._growth_tracker is not None:
            self._growth_tracker.fill_(state_dict["_growth_tracker"])

    def __getstate__(self) -> dict[str, Any]:
        state = self.__dict__.copy()
        if self._enabled:
            if len(self._per_optimizer_states) != 0:
                raise AssertionError(
                    "A GradScaler instance may only be pickled at the beginning "
                    "of an iteration, or at the end after scaler.update()."
                )
            state["_init_scale"] = self.get_scale()
            state["_init_growth_tracker"] = self._get_growth_tracker()
            state["_scale"] = None
            state["_growth_tracker"] = None
        state.pop("_found_ptrs", None)   # device addresses and a ctypes array: not part of the state
        state.pop("_found_arr", None)
        return state

    def __setstate__(self, state: dict[str, Any]) -> None:
        self.__dict__.update(state)
