"""The library driven through its C ABI alone (include/mgopt.h), with the
ctypes declarations a caller outside this package would write, no package
objects in the loop: a plan over three kernel classes (fp32 params with fp32
and fp16 grads, bf16 params with an fp32 master), set_grads, grad_norm,
adamw_step and scaler_update for several steps against the oracle bit for
bit; the error returns a GPU process can see; step counts outside the
bias-correction table (forced from the host with a short table, and a
non-integer count written into the step array), which pass 2 evaluates on the
device; and hyper-parameters read from device memory."""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests._gpu_harness import host_grad, log, to_f32

pytestmark = pytest.mark.gpu

LIB_PATH = Path(__file__).resolve().parents[1] / "minigpt-train-infra_amd" / "_build" / "libmgopt.so"
F32, F16, BF16, NONE = 0, 1, 2, -1
DEV = "cuda:0"


class TensorDesc(ctypes.Structure):            # mgopt_tensor_desc
    _fields_ = [("param_dev", ctypes.c_void_p), ("lowp_dev", ctypes.c_void_p),
                ("exp_avg_dev", ctypes.c_void_p), ("exp_avg_sq_dev", ctypes.c_void_p),
                ("numel", ctypes.c_int64), ("group", ctypes.c_int32), ("grad_dtype", ctypes.c_int32),
                ("lowp_dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("row_elems", ctypes.c_int64), ("param_pitch", ctypes.c_int64), ("state_pitch", ctypes.c_int64)]


class GroupHparams(ctypes.Structure):          # mgopt_group_hparams
    _fields_ = [("lr", ctypes.c_double), ("weight_decay", ctypes.c_double), ("beta1", ctypes.c_double),
                ("beta2", ctypes.c_double), ("eps", ctypes.c_double), ("maximize", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


def _lib():
    lib = ctypes.CDLL(str(LIB_PATH))
    vp = ctypes.c_void_p
    lib.mgopt_plan_create.argtypes = [ctypes.POINTER(TensorDesc), ctypes.c_int32, ctypes.c_int32, vp, ctypes.c_int64,
                                      ctypes.POINTER(vp)]
    lib.mgopt_plan_destroy.argtypes = [vp]
    lib.mgopt_plan_set_grads.argtypes = [vp, ctypes.POINTER(vp), vp]
    lib.mgopt_grad_norm.argtypes = [vp, vp, ctypes.c_double, vp, vp, vp, vp]
    lib.mgopt_adamw_step.argtypes = [vp, vp, vp, ctypes.c_int64, vp, vp, vp, ctypes.c_int32, vp]
    lib.mgopt_scaler_update.argtypes = [vp, vp, ctypes.POINTER(vp), ctypes.c_int32, ctypes.c_double, ctypes.c_double,
                                        ctypes.c_int32, vp]
    lib.mgopt_sync_master.argtypes = [vp, vp]
    lib.mgopt_plan_set_window.argtypes = [vp, vp]
    lib.mgopt_plan_flags.argtypes = [vp, ctypes.POINTER(ctypes.c_int)]
    lib.mgopt_synth_fill.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64,
                                     ctypes.c_double, ctypes.c_uint64, ctypes.c_double, vp]
    lib.mgopt_last_error.restype = ctypes.c_char_p
    return lib


def _ok(rc, lib, what):
    assert rc == 0, (what, rc, lib.mgopt_last_error())


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _fill(lib, t, seed, stream_id, sigma):
    code = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]
    _ok(lib.mgopt_synth_fill(t.data_ptr(), code, t.numel(), seed, stream_id, O.synth_k(sigma), 0, 1.0, _stream()), lib,
        "synth")


def _bc_table(betas, cap):
    """(1 - beta1**t, (1 - beta2**t) ** 0.5) for 1 <= t < cap, as torch/optim/adam.py:529-536
    forms them, after the row's betas at t = 0."""
    out = []
    for b1, b2 in betas:
        out += [b1, b2]
        for t in range(1, cap):
            out += [1 - b1 ** float(t), (1 - b2 ** float(t)) ** 0.5]
    return torch.tensor(out, dtype=torch.float64, device=DEV)


@pytest.mark.parametrize("fold", [True, False], ids=["three_kernels", "five_kernels"])
def test_three_kernel_classes_through_the_raw_abi(fold, monkeypatch):
    """In the three-kernel form this small plan runs, and in the five-kernel
    form (MGOPT_FOLD=0 when the plan is made; mgopt_plan_folded reports it)."""
    if not fold:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    lib = _lib()
    lib.mgopt_plan_folded.argtypes = [ctypes.c_void_p]
    specs = [  # (numel, param dtype, grad dtype, group)
        (5000, torch.float32, torch.float32, 0),
        (70000, torch.bfloat16, torch.bfloat16, 0),     # two chunks, bf16 model copy + fp32 master
        (129, torch.float32, torch.float16, 1),
    ]
    params, grads, masters, ms, vs = [], [], [], [], []
    for i, (n, pdt, gdt, _) in enumerate(specs):
        p = torch.empty(n, dtype=pdt, device=DEV)
        _fill(lib, p, 1, i, 0.02)
        params.append(p)
        grads.append(torch.empty(n, dtype=gdt, device=DEV))
        masters.append(torch.zeros(n, dtype=torch.float32, device=DEV) if pdt != torch.float32 else None)
        ms.append(torch.zeros(n, dtype=torch.float32, device=DEV))
        vs.append(torch.zeros(n, dtype=torch.float32, device=DEV))
    steps = torch.zeros(len(specs), dtype=torch.float32, device=DEV)
    descs = (TensorDesc * len(specs))()
    for i, (n, pdt, gdt, grp) in enumerate(specs):
        d = descs[i]
        if masters[i] is None:
            d.param_dev, d.lowp_dev, d.lowp_dtype = params[i].data_ptr(), None, NONE
        else:
            d.param_dev, d.lowp_dev, d.lowp_dtype = masters[i].data_ptr(), params[i].data_ptr(), BF16
        d.exp_avg_dev, d.exp_avg_sq_dev = ms[i].data_ptr(), vs[i].data_ptr()
        d.numel, d.group = n, grp
        d.grad_dtype = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[gdt]
    plan = ctypes.c_void_p()
    _ok(lib.mgopt_plan_create(descs, len(specs), 2, steps.data_ptr(), 65536, ctypes.byref(plan)), lib, "create")
    try:
        assert lib.mgopt_plan_folded(plan) == (1 if fold else 0)
        _ok(lib.mgopt_sync_master(plan, _stream()), lib, "sync_master")
        scale = torch.full((), 1024.0, dtype=torch.float32, device=DEV)
        tracker = torch.zeros((), dtype=torch.int32, device=DEV)
        norm = torch.empty((), dtype=torch.float32, device=DEV)
        coef = torch.empty((), dtype=torch.float32, device=DEV)
        found = torch.empty((), dtype=torch.float32, device=DEV)
        hp = (GroupHparams * 2)()
        for g, wd in enumerate((0.1, 0.0)):
            hp[g].weight_decay, hp[g].beta1, hp[g].beta2, hp[g].eps = wd, 0.9, 0.95, 1e-8
        bc = _bc_table([(0.9, 0.95), (0.9, 0.95)], 64)
        torch.cuda.synchronize()
        init = [(m if m is not None else p).float().cpu().numpy().copy() for p, m in zip(params, masters)]
        orc = O.OracleRun(init, [s[3] for s in specs],
                          [dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1),
                           dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)],
                          scaler=dict(init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2),
                          max_norm=1.0, lowp=None)
        gptrs = (ctypes.c_void_p * len(specs))(*[g.data_ptr() for g in grads])
        found_list = (ctypes.c_void_p * 1)(found.data_ptr())
        norms = []
        for s in range(1, 7):
            lr = 1e-3 * (0.5 + 0.1 * s)
            for h in hp:
                h.lr = lr
            for i, g in enumerate(grads):
                _fill(lib, g, 2, (s << 20) | i, 1e-2 * orc.scale)
            if s == 4:
                grads[2].view(-1)[-1] = float("nan")
            torch.cuda.synchronize()
            out = orc.step([to_f32(*host_grad(g)) for g in grads], lr)
            _ok(lib.mgopt_plan_set_grads(plan, gptrs, _stream()), lib, "set_grads")
            _ok(lib.mgopt_grad_norm(plan, scale.data_ptr(), 1.0, norm.data_ptr(), coef.data_ptr(), found.data_ptr(),
                                    _stream()), lib, "grad_norm")
            _ok(lib.mgopt_adamw_step(plan, hp, bc.data_ptr(), 64, scale.data_ptr(), coef.data_ptr(), found.data_ptr(),
                                     0, _stream()), lib, "adamw_step")
            _ok(lib.mgopt_scaler_update(scale.data_ptr(), tracker.data_ptr(), found_list, 1, 2.0, 0.5, 2, _stream()),
                lib, "scaler_update")
            torch.cuda.synchronize()
            norms.append(float(norm))
            assert float(scale) == out["scale"] and int(tracker) == out["tracker"], (s, float(scale), out)
            assert (float(found) != 0.0) == out["found_inf"]
            if math.isfinite(out["norm"]):
                assert abs(norms[-1] - out["norm"]) <= 1e-5 * out["norm"]
        assert [float(x) for x in steps.cpu()] == orc.steps == [5.0] * 3
        for i in range(len(specs)):
            got_p = (masters[i] if masters[i] is not None else params[i]).cpu().numpy()
            for got, ref in ((got_p, orc.p[i]), (ms[i].cpu().numpy(), orc.m[i]), (vs[i].cpu().numpy(), orc.v[i])):
                assert np.array_equal(got.view(np.uint32), ref.ravel().view(np.uint32)), i
        bf = params[1].view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(bf, O.to_bf16(orc.p[1].ravel()))
        flag = ctypes.c_int(-1)
        _ok(lib.mgopt_plan_flags(plan, ctypes.byref(flag)), lib, "flags")
        assert flag.value == 0
        log(f"[raw abi] 6 steps, one skipped; scale {float(scale)}, tracker {int(tracker)}")
    finally:
        lib.mgopt_plan_destroy(plan)


def test_error_returns_seen_by_a_gpu_caller():
    lib = _lib()
    p = torch.zeros(4096, dtype=torch.float32, device=DEV)
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    steps = torch.zeros(1, dtype=torch.float32, device=DEV)
    d = (TensorDesc * 1)()
    d[0].param_dev, d[0].exp_avg_dev, d[0].exp_avg_sq_dev = p.data_ptr(), m.data_ptr(), v.data_ptr()
    d[0].numel, d[0].group, d[0].grad_dtype, d[0].lowp_dtype = 4096, 0, F32, NONE
    plan = ctypes.c_void_p()
    assert lib.mgopt_plan_create(d, 1, 1, None, 65536, ctypes.byref(plan)) == 10001   # state without steps_dev
    assert b"steps_dev" in lib.mgopt_last_error()
    _ok(lib.mgopt_plan_create(d, 1, 1, steps.data_ptr(), 65536, ctypes.byref(plan)), lib, "create")
    try:
        norm = torch.empty((), dtype=torch.float32, device=DEV)
        assert lib.mgopt_grad_norm(plan, None, 1.0, norm.data_ptr(), None, None, _stream()) == 10001
        assert b"set_grads" in lib.mgopt_last_error()
        win = torch.zeros(8, dtype=torch.uint8, device=DEV)
        assert lib.mgopt_plan_set_window(plan, win.data_ptr() + 1) == 10002
        _ok(lib.mgopt_plan_set_window(plan, None), lib, "window off")
    finally:
        lib.mgopt_plan_destroy(plan)


def _one_tensor_plan(lib, n, chunk=65536):
    p = torch.empty(n, dtype=torch.float32, device=DEV)
    _fill(lib, p, 1, 0, 0.02)
    g = torch.empty(n, dtype=torch.float32, device=DEV)
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    steps = torch.zeros(1, dtype=torch.float32, device=DEV)
    d = (TensorDesc * 1)()
    d[0].param_dev, d[0].exp_avg_dev, d[0].exp_avg_sq_dev = p.data_ptr(), m.data_ptr(), v.data_ptr()
    d[0].numel, d[0].group, d[0].grad_dtype, d[0].lowp_dtype = n, 0, F32, NONE
    plan = ctypes.c_void_p()
    _ok(lib.mgopt_plan_create(d, 1, 1, steps.data_ptr(), chunk, ctypes.byref(plan)), lib, "create")
    return plan, p, g, m, v, steps


def test_step_counts_outside_the_bias_correction_table():
    """Steps 1-6 with a table covering only t < 3, then a count of 2.5 written
    into the step array: every step updates the tensor, with the bias
    corrections of the counts beyond the table evaluated on the device, and the
    plan's flag reports it.  Checked against the oracle (host pow) at the fp32
    tolerance, with the bit-exact fraction logged."""
    lib = _lib()
    n = 10000
    plan, p, g, m, v, steps = _one_tensor_plan(lib, n)
    try:
        hp = (GroupHparams * 1)()
        hp[0].lr, hp[0].weight_decay, hp[0].beta1, hp[0].beta2, hp[0].eps = 1e-3, 0.1, 0.9, 0.95, 1e-8
        bc = _bc_table([(0.9, 0.95)], 3)
        torch.cuda.synchronize()
        pr, mr, vr = p.cpu().numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
        _ok(lib.mgopt_plan_set_grads(plan, (ctypes.c_void_p * 1)(g.data_ptr()), _stream()), lib, "set_grads")
        flag = ctypes.c_int(-1)
        count = 0.0
        for s in range(1, 9):
            if s == 7:
                steps.fill_(2.5)      # a non-integer count written in place: the next step runs at 3.5
                count = 2.5
            _fill(lib, g, 2, s, 1e-3)
            torch.cuda.synchronize()
            gh = g.cpu().numpy()
            count += 1.0
            O.adamw(pr, gh, mr, vr, 1e-3, 0.9, 0.95, 1e-8, 0.1, count)
            _ok(lib.mgopt_adamw_step(plan, hp, bc.data_ptr(), 3, None, None, None, 0, _stream()), lib, "step")
            torch.cuda.synchronize()
            _ok(lib.mgopt_plan_flags(plan, ctypes.byref(flag)), lib, "flags")
            assert flag.value == (1 if s >= 3 else 0), s
            assert float(steps) == count
            exact = []
            for got, ref in ((p, pr), (m, mr), (v, vr)):
                a = got.cpu().numpy()
                assert np.max(np.abs(a.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)) <= 1e-6, s
                exact.append(float(np.mean(a.view(np.uint32) == ref.view(np.uint32))))
            log(f"[short table] step {s} (count {count}): bit-exact fractions p/m/v {exact}")
    finally:
        lib.mgopt_plan_destroy(plan)


def test_hyperparameters_from_device_memory_match_by_value():
    """MGOPT_GROUPS_ON_DEVICE: the same step with the group record in device
    memory (rewritten between steps, as a caller refreshes the learning rate
    before a graph replay) gives the bits of the by-value record."""
    lib = _lib()
    n = 70000
    a = _one_tensor_plan(lib, n, chunk=1024)
    b = _one_tensor_plan(lib, n, chunk=1024)
    try:
        bc = _bc_table([(0.9, 0.95)], 16)
        hp = (GroupHparams * 1)()
        hp[0].weight_decay, hp[0].beta1, hp[0].beta2, hp[0].eps = 0.1, 0.9, 0.95, 1e-8
        hp_dev = torch.zeros(6, dtype=torch.float64, device=DEV)   # 48 bytes: one mgopt_group_hparams
        for plan, _, g, *_ in (a, b):
            _ok(lib.mgopt_plan_set_grads(plan, (ctypes.c_void_p * 1)(g.data_ptr()), _stream()), lib, "set_grads")
        for s in range(1, 6):
            lr = 1e-3 * s
            hp[0].lr = lr
            hp_dev.copy_(torch.frombuffer(bytearray(bytes(hp)), dtype=torch.float64))
            for _, _, g, *_ in (a, b):
                _fill(lib, g, 3, s, 1e-3)
            _ok(lib.mgopt_adamw_step(a[0], hp, bc.data_ptr(), 16, None, None, None, 0, _stream()), lib, "by value")
            _ok(lib.mgopt_adamw_step(b[0], hp_dev.data_ptr(), bc.data_ptr(), 16, None, None, None, 2, _stream()), lib,
                "on device")
        torch.cuda.synchronize()
        for x, y in zip(a[1:], b[1:]):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32))
        assert float(a[5]) == float(b[5]) == 5.0
    finally:
        lib.mgopt_plan_destroy(a[0])
        lib.mgopt_plan_destroy(b[0])
