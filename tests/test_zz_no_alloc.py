"""mgopt_grad_norm_noalloc through the C ABI: the allocation-free gradient norm
of one flat gradient buffer against mgopt_grad_norm on a plan that holds the
same buffer as its one tensor.  Both sum the same 131,072-element chunks into
partials and finalize them in the same fixed order, so norm, clip
coefficient and found_inf must agree bit for bit.  Two calls in a row, the
second over a smaller buffer, show that the static partials array keeps no
state a later call depends on; sizes above its maximum are refused.  Calls
on either side of 256 MiB cover both of its load forms."""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import pytest
import torch

from oracle import oracle as O
from tests._gpu_harness import log

pytestmark = pytest.mark.gpu

LIB_PATH = Path(__file__).resolve().parents[1] / "minigpt-train-infra_amd" / "_build" / "libmgopt.so"
F32, F16, BF16, NONE = 0, 1, 2, -1
E_INVALID, E_LIMIT = 10001, 10003
MAX_ELEMS = 65536 * 131072          # 65,536 partials of 131,072-element chunks
DEV = "cuda:0"
CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


class TensorDesc(ctypes.Structure):            # mgopt_tensor_desc
    _fields_ = [("param_dev", ctypes.c_void_p), ("lowp_dev", ctypes.c_void_p),
                ("exp_avg_dev", ctypes.c_void_p), ("exp_avg_sq_dev", ctypes.c_void_p),
                ("numel", ctypes.c_int64), ("group", ctypes.c_int32), ("grad_dtype", ctypes.c_int32),
                ("lowp_dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("row_elems", ctypes.c_int64), ("param_pitch", ctypes.c_int64), ("state_pitch", ctypes.c_int64)]


def _lib():
    lib = ctypes.CDLL(str(LIB_PATH))
    vp = ctypes.c_void_p
    lib.mgopt_plan_create.argtypes = [ctypes.POINTER(TensorDesc), ctypes.c_int32, ctypes.c_int32, vp, ctypes.c_int64,
                                      ctypes.POINTER(vp)]
    lib.mgopt_plan_destroy.argtypes = [vp]
    lib.mgopt_plan_set_grads.argtypes = [vp, ctypes.POINTER(vp), vp]
    lib.mgopt_grad_norm.argtypes = [vp, vp, ctypes.c_double, vp, vp, vp, vp]
    lib.mgopt_grad_norm_noalloc.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, vp, ctypes.c_double, vp, vp, vp, vp]
    lib.mgopt_synth_fill.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64,
                                     ctypes.c_double, ctypes.c_uint64, ctypes.c_double, vp]
    lib.mgopt_last_error.restype = ctypes.c_char_p
    return lib


def _ok(rc, lib, what):
    assert rc == 0, (what, rc, lib.mgopt_last_error())


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _plan_norm(lib, g, scale, max_norm):
    """mgopt_grad_norm over a grads-only plan with `g` as its one tensor, in
    the five-kernel form (MGOPT_FOLD=0), whose pass 1 sums the same
    131,072-element chunks as the allocation-free norm."""
    d = (TensorDesc * 1)()
    d[0].numel, d[0].group, d[0].grad_dtype, d[0].lowp_dtype = g.numel(), 0, CODES[g.dtype], NONE
    plan = ctypes.c_void_p()
    saved = os.environ.get("MGOPT_FOLD")
    os.environ["MGOPT_FOLD"] = "0"
    try:
        _ok(lib.mgopt_plan_create(d, 1, 1, None, 65536, ctypes.byref(plan)), lib, "create")
    finally:
        if saved is None:
            del os.environ["MGOPT_FOLD"]
        else:
            os.environ["MGOPT_FOLD"] = saved
    out = [torch.full((), -1.0, dtype=torch.float32, device=DEV) for _ in range(3)]
    try:
        _ok(lib.mgopt_plan_set_grads(plan, (ctypes.c_void_p * 1)(g.data_ptr()), _stream()), lib, "set_grads")
        _ok(lib.mgopt_grad_norm(plan, None if scale is None else scale.data_ptr(), max_norm, out[0].data_ptr(),
                                out[1].data_ptr(), None if scale is None else out[2].data_ptr(), _stream()), lib, "norm")
        torch.cuda.synchronize()
    finally:
        lib.mgopt_plan_destroy(plan)
    return [float(t) for t in out]


def _noalloc_norm(lib, g, n, scale, max_norm):
    out = [torch.full((), -1.0, dtype=torch.float32, device=DEV) for _ in range(3)]
    _ok(lib.mgopt_grad_norm_noalloc(g.data_ptr(), CODES[g.dtype], n, None if scale is None else scale.data_ptr(),
                                    max_norm, out[0].data_ptr(), out[1].data_ptr(),
                                    None if scale is None else out[2].data_ptr(), _stream()), lib, "noalloc")
    torch.cuda.synchronize()
    return [float(t) for t in out]


def _same(a, b):
    return all(x == y or (math.isnan(x) and math.isnan(y)) for x, y in zip(a, b))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_noalloc_norm_matches_the_plan_norm(dtype):
    """Two calls in a row, the second over a smaller buffer (a prefix of a
    fresh fill), each against a one-tensor plan over the same elements: with a
    GradScaler scale, then without one, then with an inf in the second call's
    last chunk."""
    lib = _lib()
    big, small = 131072 * 37 + 999, 131072 * 3 + 5
    buf = torch.empty(big, dtype=dtype, device=DEV)
    scale = torch.full((), 1024.0, dtype=torch.float32, device=DEV)
    code = CODES[dtype]
    for call, (n, seed, inf_at, use_scale) in enumerate([(big, 1, None, True), (small, 2, None, False),
                                                         (small, 3, small - 2, True)]):
        log(f"case: noalloc {dtype} call {call} n={n}")
        _ok(lib.mgopt_synth_fill(buf.data_ptr(), code, big, seed, 7, O.synth_k(1e-2 * 1024.0), 0, 1.0, _stream()),
            lib, "fill")
        if inf_at is not None:
            buf[inf_at] = float("inf")
        view = buf[:n]
        sc = scale if use_scale else None
        got = _noalloc_norm(lib, buf, n, sc, 1.0)
        ref = _plan_norm(lib, view, sc, 1.0)
        assert _same(got, ref), (call, got, ref)
        if use_scale:
            assert got[2] == (1.0 if inf_at is not None else 0.0)
        log(f"[noalloc {dtype}] call {call}: n {n}, norm {got[0]!r}, coef {got[1]!r}, found_inf {got[2]!r}")


def test_noalloc_norm_on_both_sides_of_the_cache_size():
    """Buffers of more than 256 MiB are read with nontemporal loads, smaller
    ones with loads that leave them in the Infinity Cache: one call just above
    that size and one just below, each against the plan norm (whose plan picks
    its loads by the same rule) and, for the sum of squares, against the
    oracle's compensated sum of the same elements."""
    lib = _lib()
    above, below = (256 << 20) // 4 + 1, (256 << 20) // 4 - 131072 - 7
    buf = torch.empty(above, dtype=torch.float32, device=DEV)
    for call, (n, seed) in enumerate([(above, 11), (below, 12)]):
        log(f"case: noalloc fp32 n={n} ({'above' if n * 4 > (256 << 20) else 'below'} 256 MiB)")
        _ok(lib.mgopt_synth_fill(buf.data_ptr(), F32, n, seed, 5, O.synth_k(1e-3), 0, 1.0, _stream()), lib, "fill")
        got = _noalloc_norm(lib, buf, n, None, 1.0)
        ref = _plan_norm(lib, buf[:n], None, 1.0)
        assert _same(got, ref), (call, got, ref)
        want = O.norm_from_sumsq(O.sumsq(buf[:n].cpu().numpy()))
        assert got[0] == want, (call, got[0], want)
        log(f"[noalloc cache sizes] n {n}: norm {got[0]!r} = oracle")


def test_noalloc_norm_refuses_what_it_cannot_hold():
    lib = _lib()
    buf = torch.zeros(16, dtype=torch.float32, device=DEV)
    norm = torch.empty((), dtype=torch.float32, device=DEV)
    assert lib.mgopt_grad_norm_noalloc(buf.data_ptr(), F32, MAX_ELEMS + 1, None, 1.0, norm.data_ptr(), None, None,
                                       _stream()) == E_LIMIT
    assert b"maximum" in lib.mgopt_last_error()
    assert lib.mgopt_grad_norm_noalloc(buf.data_ptr(), F32, 0, None, 1.0, norm.data_ptr(), None, None,
                                       _stream()) == E_INVALID
    assert lib.mgopt_grad_norm_noalloc(None, F32, 16, None, 1.0, norm.data_ptr(), None, None, _stream()) == E_INVALID
    assert lib.mgopt_grad_norm_noalloc(buf.data_ptr(), 9, 16, None, 1.0, norm.data_ptr(), None, None,
                                       _stream()) == E_INVALID
    # a valid call still works after the refusals
    _ok(lib.mgopt_grad_norm_noalloc(buf.data_ptr(), F32, 16, None, 1.0, norm.data_ptr(), None, None, _stream()), lib,
        "zeros")
    torch.cuda.synchronize()
    assert float(norm) == 0.0
