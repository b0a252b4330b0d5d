"""GPU parity at the full sizes of the workloads the step is specified on.

At these sizes the oracle rebuilds on the host, from the generator the GPU
fill uses (bit-identical), the gradients of a subset of tensors -- the
largest ones always among them -- and steps those tensors in its own
arithmetic every iteration; their master, exp_avg and exp_avg_sq are compared
with the GPU's bit for bit at the check steps.  The total norm over every
gradient is rebuilt on the host at the verify steps (to 1e-5, exact count
logged); at the others the oracle's clip coefficient is formed from the GPU's
norm.  The rest of the state is checked through size-independent properties
on the device: the bf16 model copy is the round-to-nearest-even image of the
master everywhere, a skipped step leaves every arena bit for bit unchanged
(integer checksums of the bit patterns), and every step count equals the
number of steps taken.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from tests._compare import ULP_LOWP, exact_fraction, rel, ulp16, RTOL_NORM
from tests._gpu_harness import Case, Pair, log, mg

pytestmark = pytest.mark.gpu


def _checksums(pair: Pair) -> list[int]:
    eng = pair.opt._engine
    arenas = [eng.exp_avg, eng.exp_avg_sq] + ([eng.master] if eng.master is not None else [])
    if eng.master is None:
        arenas += [p.detach() for p in pair.params]
    return [int(a.reshape(-1).view(torch.int32).sum()) for a in arenas]


def _check_subset(pair: Pair, label: str, step: int) -> None:
    """The oracle's tensors against the GPU's, bit for bit, after `step`."""
    torch.cuda.synchronize()
    for i in pair.case.subset:
        st = pair.gpu_state(i)
        assert st["step"] == pair.orc.steps[i], (label, step, i, st["step"], pair.orc.steps[i])
        for k, ref in (("p", pair.orc.p[i]), ("m", pair.orc.m[i]), ("v", pair.orc.v[i])):
            assert exact_fraction(st[k], ref.ravel()) == 1.0, (label, step, k, i)
        if "lowp_bits" in st:
            assert ulp16(st["lowp_bits"], pair.oracle_lowp_bits(i)) <= ULP_LOWP, (label, step, i)
    sizes = sorted((pair.orc.p[i].size for i in pair.case.subset), reverse=True)
    log(f"[{label}] step {step}: {len(pair.case.subset)} tensors bit-exact (largest {sizes[:2]} elements)")


def _run_full(pair: Pair, label: str, check_at: set, skip_step: int | None = None) -> None:
    """Steps 1..case.steps: GPU step, then the oracle's step from host-rebuilt
    gradients; the subset compared at the steps in check_at; at skip_step the
    whole state is checksummed before and after the (skipped) step."""
    c = pair.case
    assert c.host_grads
    for s in range(1, c.steps + 1):
        lr = mg.cosine_lr(s - 1, *c.lr_sched)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        before = _checksums(pair) if s == skip_step else None
        pair.gpu_step()
        out = pair.oracle_step_host(s, lr)
        if before is not None:
            torch.cuda.synchronize()
            assert out["skipped"]
            assert _checksums(pair) == before, "a skipped step changed the optimizer state"
        if out["verified"] and out["norm"] is not None:
            ng, no = float(pair.norms_gpu[-1]), out["norm"]
            if math.isfinite(no):
                assert rel(ng, no) <= RTOL_NORM, (label, s, ng, no)
            else:
                assert (math.isnan(no) and math.isnan(ng)) or ng == no, (label, s, ng, no)
            log(f"[{label}] step {s}: norm {ng!r} (oracle {no!r}){' skipped' if out['skipped'] else ''}")
        if s in check_at:
            _check_subset(pair, label, s)
    torch.cuda.synchronize()


def _check_full(pair: Pair, label: str, expect_steps: int) -> None:
    """After the run: the scale trajectory, every step count, the bf16 copies."""
    verified = [(float(t), o["norm"]) for t, o in zip(pair.norms_gpu, pair.outs) if o.get("norm") is not None]
    exact_norms = sum(1 for ng, no in verified if ng == no or not math.isfinite(no))
    if pair.case.scaler:
        assert [float(t) for t in pair.scale_gpu] == [o["scale"] for o in pair.outs]
    eng = pair.opt._engine
    assert bool((eng.steps == float(expect_steps)).all())
    if eng.master is not None:
        for i, p in enumerate(pair.params):
            m = pair.opt.state[p]["master_param"]
            assert torch.equal(m.to(p.dtype).view(torch.int16), p.detach().view(torch.int16)), (label, i)
    assert eng.device_bc_flag() == 0
    log(f"[{label}] {len(pair.outs)} steps, {len(verified)} norms verified ({exact_norms} exact), "
        f"subset of {len(pair.case.subset)} tensors bit-exact at every check step")


def _tensor_at_chunk(shapes_in_plan_order, chunk_elems: int, chunk: int) -> int:
    """Position of the tensor that holds pass-2 chunk number `chunk`."""
    seen = 0
    for k, s in enumerate(shapes_in_plan_order):
        seen += -(-math.prod(s) // chunk_elems)
        if seen > chunk:
            return k
    raise ValueError("the set has fewer chunks")


def test_gpt2_small_200_steps():
    """GPT-2-small shapes, 124,475,904 fp32 params, fp16 grads N(0,1e-2) x scale,
    GradScaler 65536 / x2 per 2000 / x0.5, +inf at one seeded element at steps
    17 and 53, 200 steps.  The oracle steps the tied token embedding (38.6M
    elements), three more matrices and every no-decay tensor; the norm is
    verified at every step."""
    shapes = mg.paramsets.WORKLOADS["gpt2_small"]()
    rng = np.random.RandomState(17)
    inject = {s: [(int(rng.randint(len(shapes))), 0, float("inf"))] for s in (17, 53)}
    decay_n = sum(1 for _, s in shapes if len(s) >= 2)
    subset = [0, 1, 4, 5] + list(range(decay_n, len(shapes)))
    log("case: gpt2_small 200 steps")
    pair = Pair(Case(shapes=shapes, grad_dtype="f16", steps=200, sigma=1e-2,
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000),
                     inject=inject, subset=subset, lr_sched=(6e-4, 6e-5, 10, 200), host_grads=True))
    _run_full(pair, "gpt2_small_200", check_at={1, 17, 53, 100, 200})
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [17, 53]
    assert pair.outs[-1]["scale"] == 16384.0 and pair.outs[-1]["tracker"] == 200 - 53
    _check_full(pair, "gpt2_small_200", 198)


def test_gpt_1p3b_full_size_bf16_master():
    """1.3B GPT (24 layers, width 2048, vocab 50304): bf16 params and grads,
    fp32 master/m/v, grads N(0,1e-3) with 0.1% x100 so clipping acts every
    step; 100 steps.  The oracle steps the token embedding (103M elements),
    four more matrices and every no-decay tensor."""
    shapes = mg.paramsets.WORKLOADS["gpt_1p3b"]()
    log("case: gpt_1p3b full size, 100 steps")
    decay = [s for _, s in shapes if len(s) >= 2]
    nodecay_idx = list(range(len(decay), len(shapes)))
    subset = [0, 1, 2, 3, len(decay) - 1] + nodecay_idx
    pair = Pair(Case(shapes=shapes, param_dtype="bf16", grad_dtype="bf16", steps=100, sigma=1e-3,
                     tail=(1000, 100.0), subset=subset, host_grads=True,
                     verify_norm={1, 2, 3, 4, 5, 10, 25, 50, 75, 100}))
    _run_full(pair, "gpt_1p3b", check_at={1, 10, 50, 100})
    assert all(o["norm"] > 1.0 for o in pair.outs if o["norm"] is not None)
    assert all(float(t) > 1.0 for t in pair.norms_gpu)
    _check_full(pair, "gpt_1p3b", 100)


def test_qwen3_8b_full_size():
    """Qwen3-8B-shaped set, 8,190,735,360 params (131 GB resident): bf16 params
    and grads, fp32 master/m/v, GradScaler, clip 1.0; 50 steps with +inf at
    step 2 (a skipped step over the whole set).  The oracle steps
    model.embed_tokens and lm_head (622M elements each, the only tensors whose
    fp32 master exceeds 2 GiB), four layer matrices and every RMSNorm weight.
    MGOPT_QWEN3_STEPS=N runs N steps instead (a multiple of 25), checked every
    25 steps."""
    steps = int(os.environ.get("MGOPT_QWEN3_STEPS", "50"))
    assert steps >= 25 and steps % 25 == 0
    shapes = mg.paramsets.WORKLOADS["qwen3_8b"]()
    decay_n = sum(1 for _, s in shapes if len(s) >= 2)
    assert shapes[0][0] == "model.embed_tokens.weight" and shapes[-1][0] == "lm_head.weight"
    subset = [0, 1, 2, 5, decay_n - 2, decay_n - 1] + list(range(decay_n, len(shapes)))
    log(f"case: qwen3_8b full size, {steps} steps, inf at step 2")
    every25 = set(range(25, steps + 1, 25))
    pair = Pair(Case(shapes=shapes, param_dtype="bf16", grad_dtype="bf16", steps=steps, sigma=1e-3,
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000),
                     inject={2: [(7, 123, float("inf"))]}, subset=subset, fresh_grads=False, host_grads=True,
                     verify_norm={1, 2, 3, 10} | every25))
    assert pair.shapes[0][0] == "model.embed_tokens.weight" and pair.shapes[decay_n - 1][0] == "lm_head.weight"
    _run_full(pair, "qwen3_8b", check_at={1, 3, 10} | every25, skip_step=2)
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [2]
    _check_full(pair, "qwen3_8b", steps - 1)


def test_pass2_beyond_one_dispatch():
    """4.43e9 elements in 512-element chunks: 8,650,752 pass-2 work-groups,
    more than one dispatch packet's 32-bit work-item count holds at 512
    threads (8,388,607 work-groups), so pass 2 runs in two launches.  The
    tensor holding the first chunk of the second launch, and the first and
    last tensors, are checked bit for bit against the oracle; every step count
    covers the rest.  fp32 params, fp16 grads, 62 GB."""
    shapes = [(f"w{i}", (4096, 4096)) for i in range(264)]
    boundary = _tensor_at_chunk([s for _, s in shapes], 512, 0xFFFFFFFF // 512)
    subset = sorted({0, boundary, len(shapes) - 1})
    log(f"case: 264 x 4096x4096 fp32/fp16, chunk 512, 2 steps, second launch starts in tensor {boundary}")
    pair = Pair(Case(shapes=shapes, param_dtype="f32", grad_dtype="f16", steps=2, sigma=1e-3, scaler=None,
                     subset=subset, chunk_elems=512, host_grads=True))
    _run_full(pair, "two dispatches", check_at={1, 2})
    _check_full(pair, "two dispatches", 2)


def test_fp32_tensors_beyond_2gib():
    """fp32 parameters and fp32 gradients (the class torch's own fused step
    runs in the reference's loop on a GPU) with one tensor of 640M elements:
    2.56 GB each for the parameter, its gradient and both moments, so every
    stream's byte offsets pass 2^31 inside one tensor.  Heavy-tailed gradients
    (clipping every step), GradScaler, 3 steps; both tensors bit-exact against
    the oracle at every step."""
    shapes = [("big", (640, 1_000_000)), ("b", (1000,))]
    log("case: fp32 params/grads, one 640M-element tensor, 3 steps")
    pair = Pair(Case(shapes=shapes, param_dtype="f32", grad_dtype="f32", steps=3, sigma=1e-3, tail=(1000, 100.0),
                     scaler=dict(init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000),
                     subset=[0, 1], host_grads=True))
    _run_full(pair, "fp32 beyond 2 GiB", check_at={1, 2, 3})
    assert all(o["norm"] > 1.0 and not o["skipped"] for o in pair.outs)
    _check_full(pair, "fp32 beyond 2 GiB", 3)


def test_ragged_full_size():
    """20,000 tensors, log-uniform sizes 1..4M elements, 2.5B elements, fp32
    params, fp16 grads, GradScaler growth interval 50; 6 steps with a NaN at
    step 3."""
    shapes = mg.paramsets.WORKLOADS["ragged_20k"]()
    log("case: ragged_20k full size, 6 steps, NaN at step 3")
    # a spread of sizes: the 20 largest, 20 smallest and 20 in the middle (param_groups order)
    sizes = [(i, math.prod(s)) for i, (_, s) in enumerate([x for x in shapes if len(x[1]) >= 2] +
                                                            [x for x in shapes if len(x[1]) < 2])]
    by_size = sorted(sizes, key=lambda t: t[1])
    subset = sorted({i for i, _ in by_size[:20] + by_size[-20:] + by_size[len(by_size) // 2 - 10: len(by_size) // 2 + 10]})
    pair = Pair(Case(shapes=shapes, grad_dtype="f16", steps=6, sigma=1e-2,
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=50),
                     inject={3: [(by_size[-1][0], 5, float("nan"))]}, subset=subset, fresh_grads=False,
                     host_grads=True))
    _run_full(pair, "ragged_20k", check_at={1, 6}, skip_step=3)
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [3]
    _check_full(pair, "ragged_20k", 5)
