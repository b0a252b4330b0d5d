"""The step of a capturable AdamW (capturable=True) captured in one HIP graph
with the scaler's unscale_/step/update and clip_grad_norm_, and replayed.

Each replay is compared with an eager twin (capturable=False) stepped on the
same gradients and learning rates: parameters, moments, step counts, the
norm, the loss scale and the growth tracker must agree bit for bit after
every replay.  Between replays the program does its own eager work -- the
gradients are rewritten in place, the learning rate changes (a cosine
schedule, brought to the device by set_optimizer_lr), an inf is planted at
one replay -- and synchronizes before comparing.  A few eager steps of the
capturable optimizer after the replays continue from the replayed state.
"""

from __future__ import annotations

import math

import pytest
import torch

from tests._gpu_harness import log, mg, syn

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
# (4, 2048) keeps its state in the row layout (rows of 2,048 elements)
SHAPES = [(64, 33), (1000,), (7,), (300, 5), (2, 131072), (4, 2048)]


def _setup(capturable: bool, dtype=torch.float32):
    params = []
    for i, s in enumerate(SHAPES):
        p = torch.empty(s, dtype=dtype, device=DEV)
        syn.fill_(p, syn.PARAM_SEED, syn.param_stream(i), 0.02)
        params.append(torch.nn.Parameter(p))
        params[-1].grad = torch.empty_like(p)          # fixed gradient buffers, rewritten in place
    decay = [p for p in params if p.ndim >= 2]
    nodecay = [p for p in params if p.ndim < 2]
    opt = mg.AdamW([{"params": decay, "weight_decay": 0.1}, {"params": nodecay, "weight_decay": 0.0}],
                   lr=1e-3, betas=(0.9, 0.95), eps=1e-8, capturable=capturable)
    scaler = mg.GradScaler("cuda", init_scale=1024.0, growth_interval=3)
    scaler.scale(torch.ones((), device=DEV))
    return params, opt, scaler


def _fill(params, step, scale, inf=False):
    for i, p in enumerate(params):
        syn.fill_(p.grad, syn.GRAD_SEED, syn.grad_stream(step, i), 1e-2 * scale)
    if inf:
        params[3].grad.view(-1)[17] = float("inf")


def _eager_step(params, opt, scaler):
    scaler.unscale_(opt)
    norm = mg.clip_grad_norm_(params, 1.0)
    scaler.step(opt)
    scaler.update()
    return norm


def _same(a, b):
    x, y = a.detach().reshape(-1), b.detach().reshape(-1)
    bits = torch.int32 if x.element_size() == 4 else torch.int16
    return torch.equal(x.view(bits), y.view(bits))


def _compare(pe, oe, se, pg, og, sg, norm_e, norm_g, label):
    torch.cuda.synchronize()
    assert float(norm_e) == float(norm_g) or (math.isnan(float(norm_e)) and math.isnan(float(norm_g))), label
    assert se.get_scale() == sg.get_scale() and se._get_growth_tracker() == sg._get_growth_tracker(), label
    for a, b in zip(pe, pg):
        assert _same(a, b), label
        for k in ("exp_avg", "exp_avg_sq", "step") + (("master_param",) if "master_param" in oe.state[a] else ()):
            assert _same(oe.state[a][k], og.state[b][k]), (label, k)


@pytest.mark.parametrize("fold", [True, False], ids=["three_kernels", "five_kernels"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_captured_step_replays_match_eager(dtype, fold, monkeypatch):
    """fp32 parameters, and bf16 parameters with fp32 masters (the bf16 copy
    rewritten from the master by every replay); the step of a small plan in
    its three-kernel form, and in the five-kernel form of larger plans
    (MGOPT_FOLD=0 when the plans are made)."""
    if not fold:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    pe, oe, se = _setup(False, dtype)
    pg, og, sg = _setup(True, dtype)
    n_steps = 24
    lr_at = lambda s: mg.cosine_lr(s - 1, 3e-3, 3e-4, 4, n_steps)
    # two eager steps on both (the capturable one builds its plan, tables and device records)
    for s in (1, 2):
        for params, opt in ((pe, oe), (pg, og)):
            mg.set_optimizer_lr(opt, lr_at(s))
        scale = se.get_scale()
        _fill(pe, s, scale)
        _fill(pg, s, scale)
        norm_e = _eager_step(pe, oe, se)
        norm_g = _eager_step(pg, og, sg)
        _compare(pe, oe, se, pg, og, sg, norm_e, norm_g, f"eager step {s}")

    assert og._engine.folded() == oe._engine.folded() == fold
    assert og._engine.rows == oe._engine.rows == [0, 0, 0, 2048, 0, 0]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        norm_g = _eager_step(pg, og, sg)          # recorded, not run
    log("case: captured step, 20 replays with eager work between them, inf at replay 9")
    for s in range(3, 23):
        lr = lr_at(s)
        mg.set_optimizer_lr(oe, lr)
        mg.set_optimizer_lr(og, lr)                # refreshes the device records the graph reads
        scale = se.get_scale()
        _fill(pe, s, scale, inf=(s == 11))
        _fill(pg, s, scale, inf=(s == 11))
        norm_e = _eager_step(pe, oe, se)
        graph.replay()
        _compare(pe, oe, se, pg, og, sg, norm_e, norm_g, f"replay at step {s}")
    assert mg.optimizer_completed_steps(og) == mg.optimizer_completed_steps(oe) == 21
    # eager steps after the replays continue from the replayed state
    for s in (23, 24):
        for opt in (oe, og):
            mg.set_optimizer_lr(opt, lr_at(s))
        scale = se.get_scale()
        _fill(pe, s, scale)
        _fill(pg, s, scale)
        norm_e = _eager_step(pe, oe, se)
        norm_g2 = _eager_step(pg, og, sg)
        _compare(pe, oe, se, pg, og, sg, norm_e, norm_g2, f"eager step {s} after replays")
    assert og._engine.device_bc_flag() == 0 and og._engine.captured
    with pytest.raises(RuntimeError, match="captured"):
        og.add_param_group({"params": [torch.nn.Parameter(torch.zeros(3, device=DEV))]})
    log(f"[graph {dtype} fold={fold}] 20 replays + 4 eager steps bit-exact against the eager twin; "
        f"scale {sg.get_scale()}")


# every refused capture ends with nothing recorded, which torch reports as an empty graph
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_capture_refuses_what_a_replay_cannot_honour():
    """Capturing before any eager step, or after the gradient buffers moved,
    raises instead of recording host-side copies; a non-capturable optimizer
    refuses capture as torch's does."""
    params, opt, scaler = _setup(True)
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="outside graph capture"):
        with torch.cuda.graph(graph):
            _eager_step(params, opt, scaler)
    params, opt, scaler = _setup(True)
    _fill(params, 1, scaler.get_scale())
    _eager_step(params, opt, scaler)
    params[0].grad = torch.zeros_like(params[0])   # a new gradient buffer
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="gradient tensors changed"):
        with torch.cuda.graph(graph):
            _eager_step(params, opt, scaler)
    params, opt, scaler = _setup(False)
    _fill(params, 1, scaler.get_scale())
    _eager_step(params, opt, scaler)
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="capturable=False"):
        with torch.cuda.graph(graph):
            _eager_step(params, opt, scaler)
