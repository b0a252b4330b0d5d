"""Deterministic synthetic parameters and gradients on the GPU.

Values come from mgopt_synth_fill: element i of stream (seed, stream_id) is a
sum of four 16-bit uniforms from a 64-bit counter hash, centred and scaled
(Irwin-Hall n=4, standard deviation sigma), optionally with a heavy tail.  The
CPU oracle implements the same generator, so both sides see identical bits.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native as N

PARAM_SEED = 1
GRAD_SEED = 2


def k_for(sigma: float) -> float:
    """Generator multiplier for standard deviation sigma."""
    return sigma * math.sqrt(3.0) / 65536.0


def param_stream(i: int) -> int:
    return i


def grad_stream(step: int, i: int) -> int:
    """Stream of tensor i's gradient at (1-based) iteration `step`."""
    return (step << 20) | i


def fill_(t: torch.Tensor, seed: int, stream: int, sigma: float, tail_every: int = 0, tail_mult: float = 1.0) -> torch.Tensor:
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("fill_ needs a contiguous GPU tensor")
    N.check(
        N.lib().mgopt_synth_fill(
            ctypes.c_void_p(t.data_ptr()), N.dtype_code(t.dtype), t.numel(), seed, stream, k_for(sigma), tail_every,
            tail_mult, ctypes.c_void_p(N.stream_handle(t.device)),
        ),
        "mgopt_synth_fill",
    )
    return t


def fill_many_(tensors: list[torch.Tensor], seed: int, stream: int, sigma: float) -> list[torch.Tensor]:
    """Fills many tensors of one dtype and device from one generator launch:
    stream `stream` over a flat staging buffer, tensor k taking the elements
    from the sum of the earlier tensors' sizes onward, then copied in with
    multi-tensor copies (a few hundred launches for 20,000 tensors instead of
    one launch each).  The staging buffer is freed before returning."""
    if not tensors:
        return tensors
    total = sum(t.numel() for t in tensors)
    staging = torch.empty(total, dtype=tensors[0].dtype, device=tensors[0].device)
    fill_(staging, seed, stream, sigma)
    views, off = [], 0
    for t in tensors:
        views.append(staging[off : off + t.numel()].view(t.shape))
        off += t.numel()
    torch._foreach_copy_(tensors, views)
    del views, staging
    return tensors
