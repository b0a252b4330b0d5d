"""The three-kernel step of small plans against the five-kernel step.

A plan of at most 2,097,152 elements (no empty tensor, no tensor of more than
256 pass-2 chunks) runs pass 1 with the finalize in the work-group that takes
its last ticket, and pass 2 with each tensor's step count and constants
formed inside it, the tensor's last work-group advancing the count.  MGOPT_FOLD=0 in the environment when the
plan is created keeps the five-kernel form (pass 1, finalize, prologue, pass
2, scaler).  The same training sequence through both forms must give the same
norms, loss scales, step counts, parameters, moments, masters, low-precision
copies and window record bit for bit: fp32, fp16 and bf16 gradients, fp16 and
bf16 parameters with masters, tensors of one and of several chunks, an inf
step, a parameter without a gradient for one step, a learning-rate schedule,
a step count written in place beyond the bias-correction table, and written-
back gradients.  The pass-1 chunkings differ (16,384 against 131,072
elements), so the fp64 partial sums differ in rounding far below the fp32
norm's; every norm is also checked against the oracle.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests._gpu_harness import host_grad, log, mg, syn, to_f32

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SPECS = [  # (shape, param dtype, grad dtype): one-chunk and several-chunk tensors of every class
    ((300, 5), torch.float32, torch.float32),
    ((1001,), torch.float32, torch.float16),
    ((64, 33), torch.float32, torch.bfloat16),
    ((5000,), torch.float16, torch.float16),
    ((77, 13), torch.bfloat16, torch.bfloat16),
    ((4099,), torch.float16, torch.float32),
    ((7,), torch.float32, torch.float32),
    ((3, 1024), torch.bfloat16, torch.bfloat16),
]


def _build(fold: bool, writeback: bool):
    params = []
    for i, (s, pdt, _) in enumerate(SPECS):
        p = torch.empty(s, dtype=pdt, device=DEV)
        syn.fill_(p, syn.PARAM_SEED, syn.param_stream(i), 0.02)
        params.append(torch.nn.Parameter(p))
    opt = mg.AdamW([{"params": params[:4], "weight_decay": 0.1}, {"params": params[4:], "weight_decay": 0.0}],
                   lr=1e-3, betas=(0.9, 0.95), writeback_grads=writeback)
    grads = [torch.empty(s, dtype=gdt, device=DEV) for s, _, gdt in SPECS]
    opt.set_grad_source(grads)
    sc = mg.GradScaler("cuda", init_scale=1024.0, growth_interval=3)
    sc.scale(torch.ones((), device=DEV))
    return params, opt, grads, sc


def _run(fold: bool, writeback: bool, steps: int = 12):
    saved = os.environ.get("MGOPT_FOLD")
    if fold:
        os.environ.pop("MGOPT_FOLD", None)
    else:
        os.environ["MGOPT_FOLD"] = "0"
    try:
        params, opt, grads, sc = _build(fold, writeback)
        norms, scales = [], []
        for s in range(1, steps + 1):
            mg.set_optimizer_lr(opt, mg.cosine_lr(s - 1, 3e-3, 3e-4, 3, steps))
            scale = sc.get_scale()
            for i, g in enumerate(grads):
                syn.fill_(g, syn.GRAD_SEED, syn.grad_stream(s, i), 1e-2 * scale)
            if s == 4:
                grads[3].view(-1)[4321] = float("inf")
            if s == 6:      # parameter 1 has no gradient this step
                opt.set_grad_source([None if i == 1 else g for i, g in enumerate(grads)])
            if s == 7:
                opt.set_grad_source(grads)
            if s == 9:      # a count written in place, beyond the bias-correction table
                opt.state[params[5]]["step"].fill_(70000.0)
            sc.unscale_(opt)
            norms.append(mg.clip_grad_norm_(params, 1.0).item() if s != 6 else
                         mg.clip_grad_norm_([p for i, p in enumerate(params) if i != 1], 1.0).item())
            sc.step(opt)
            sc.update()
            scales.append(sc.get_scale())
            if s == 1:
                assert opt._engine.folded() == fold
        torch.cuda.synchronize()
        state = []
        for p, g in zip(params, grads):
            st = opt.state[p]
            entry = [p.detach().clone(), st["exp_avg"].clone(), st["exp_avg_sq"].clone(), st["step"].clone()]
            if "master_param" in st:
                entry.append(st["master_param"].clone())
            if writeback:
                entry.append(g.clone())
            state.append(entry)
        return norms, scales, state, opt.window_metrics(), opt._engine.device_bc_flag()
    finally:
        if saved is None:
            os.environ.pop("MGOPT_FOLD", None)
        else:
            os.environ["MGOPT_FOLD"] = saved


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16).numpy()


@pytest.mark.parametrize("writeback", [False, True])
def test_three_kernel_step_equals_five_kernel_step(writeback):
    log(f"case: folded vs five-kernel step, writeback={writeback}")
    a = _run(True, writeback)
    b = _run(False, writeback)
    assert a[0] == b[0], (a[0], b[0])                 # norms (the inf step's is inf in both)
    assert a[1] == b[1]                               # loss scales
    for i, (ea, eb) in enumerate(zip(a[2], b[2])):
        for k, (x, y) in enumerate(zip(ea, eb)):
            assert np.array_equal(_bits(x), _bits(y)), (i, k)
    assert a[3] == b[3], (a[3], b[3])                 # window record
    assert a[4] == b[4] == 1                          # the written count took the device evaluation
    assert a[3]["skipped_steps"] == 1 and a[3]["optimizer_steps"] == 11
    log(f"[fold] 12 steps equal bit for bit; window {a[3]}")


def test_three_kernel_norms_match_the_oracle():
    """The folded pass 1 (16,384-element chunks, finalize in the last
    work-group) against the oracle's compensated sum, on sets of one to many
    chunks per tensor and with an inf."""
    for n_tensors, size, inf_at in [(1, 5, None), (3, 16384, None), (5, 100003, None), (40, 20011, (7, 19999))]:
        grads = []
        for i in range(n_tensors):
            g = torch.empty(size, dtype=torch.float32, device=DEV)
            syn.fill_(g, syn.GRAD_SEED, 1000 + i, 1e-2)
            grads.append(g)
        if inf_at is not None:
            grads[inf_at[0]][inf_at[1]] = float("inf")
        params = [torch.nn.Parameter(torch.zeros(size, device=DEV)) for _ in range(n_tensors)]
        opt = mg.AdamW(params, lr=1e-3)
        opt.set_grad_source(grads)
        norm = mg.clip_grad_norm_(params, 1.0).item()
        assert opt._engine.folded()
        want = O.norm_from_sumsq(O.total_sumsq([to_f32(*host_grad(g)) for g in grads]))
        assert norm == want or (np.isinf(norm) and np.isinf(want)), (n_tensors, size, norm, want)
        log(f"[fold norm] {n_tensors} x {size}: {norm!r} = oracle")


def _forced_run(env: str, shapes, steps: int = 4):
    saved = os.environ.get("MGOPT_FOLD")
    os.environ["MGOPT_FOLD"] = env
    try:
        params = []
        for i, s in enumerate(shapes):
            p = torch.empty(s, dtype=torch.float32, device=DEV)
            syn.fill_(p, syn.PARAM_SEED, syn.param_stream(i), 0.02)
            params.append(torch.nn.Parameter(p))
        opt = mg.AdamW(params, lr=1e-3, weight_decay=0.1)
        grads = [torch.empty(s, dtype=torch.float16, device=DEV) for s in shapes]
        opt.set_grad_source(grads)
        sc = mg.GradScaler("cuda", init_scale=1024.0, growth_interval=2)
        sc.scale(torch.ones((), device=DEV))
        norms = []
        for s in range(1, steps + 1):
            for i, g in enumerate(grads):
                syn.fill_(g, syn.GRAD_SEED, syn.grad_stream(s, i), 1e-2 * sc.get_scale())
            if s == 2:
                grads[0].view(-1)[-1] = float("nan")
            sc.unscale_(opt)
            norms.append(mg.clip_grad_norm_(params, 1.0).item())
            sc.step(opt)
            sc.update()
        folded = opt._engine.folded()
        torch.cuda.synchronize()
        state = [[p.detach().clone(), opt.state[p]["exp_avg"].clone(), opt.state[p]["exp_avg_sq"].clone(),
                  opt.state[p]["step"].clone()] for p in params]
        return folded, norms, sc.get_scale(), state, opt._engine.chunk_elems
    finally:
        if saved is None:
            os.environ.pop("MGOPT_FOLD", None)
        else:
            os.environ["MGOPT_FOLD"] = saved


@pytest.mark.parametrize("shapes", [[(2048, 300), (4099,)], [(1 << 20,), (1 << 20,), (70000,)]],
                         ids=["600-chunk tensor", "2.16M elements"])
def test_forced_three_kernel_step_beyond_the_limits(shapes):
    """MGOPT_FOLD=1 takes the three-kernel form on plans the limits keep in the
    five-kernel form (a tensor of more than 256 pass-2 chunks, more than
    2,097,152 elements); 4 steps with a NaN step equal the five-kernel form's
    bit for bit, norms included."""
    log(f"case: forced three-kernel step, shapes {shapes}")
    a = _forced_run("1", shapes)
    b = _forced_run("0", shapes)
    assert a[0] and not b[0]
    assert a[4] == b[4] == 1024      # beyond the limits the default chunk is 1,024 elements
    assert a[1][1] != a[1][1] and b[1][1] != b[1][1]     # the NaN step's norm
    assert a[1][0] == b[1][0] and a[1][2:] == b[1][2:] and a[2] == b[2]
    for i, (ea, eb) in enumerate(zip(a[3], b[3])):
        for k, (x, y) in enumerate(zip(ea, eb)):
            assert np.array_equal(_bits(x), _bits(y)), (i, k)
    assert float(a[3][0][3]) == 3.0
    log(f"[forced fold] {shapes}: 4 steps equal bit for bit, norms {a[1]}")
