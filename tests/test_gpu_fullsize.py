"""GPU parity at the full sizes of the workloads the step is specified on.

At these sizes the oracle works from gradients it rebuilds on the host with
the generator the GPU fill uses (bit-identical), and checks three things at
every step:
  - the total norm and the non-finite flag, recomputed from the device
    gradients by torch in fp64 (no kernel of this engine involved) and, at
    some steps, rebuilt on the host: the GPU's norm must agree to 1e-5, the
    skip decision exactly;
  - a subset of tensors tracked from the first step -- the largest ones
    always among them -- stepped in the oracle's own arithmetic and compared
    with the GPU's bit for bit at the check steps;
  - every other tensor, once per run: its state is copied from the GPU before
    one step, stepped by the oracle, and compared bit for bit after it, so
    that every tensor of the set is value-checked in each run.
The rest is checked through size-independent properties on the device: the
bf16 model copy is the round-to-nearest-even image of the master everywhere,
a skipped step leaves every arena bit for bit unchanged (integer checksums of
the bit patterns), and every step count equals the number of steps taken.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests._compare import RTOL_NORM, exact_fraction, rel
from tests._gpu_harness import Case, Pair, log, mg, rotation_schedule, syn

pytestmark = pytest.mark.gpu


def _checksums(pair: Pair, piece: int = 1 << 28) -> list[int]:
    """Integer sums of the bit patterns of every optimizer arena and every
    parameter, summed in pieces (the int64 widening of one whole 98 GB arena
    would not fit beside the set)."""
    eng = pair.opt._engine
    arenas = [a.reshape(-1).view(torch.int32) for a in (eng.exp_avg, eng.exp_avg_sq, eng.master, eng.rows_arena)
              if a is not None]
    arenas += [p.detach().reshape(-1).view(torch.int32 if p.dtype == torch.float32 else torch.int16)
               for p in pair.params]
    return [sum(int(a[s: s + piece].sum()) for s in range(0, a.numel(), piece)) for a in arenas]


def _check_subset(pair: Pair, label: str, step: int) -> None:
    """The oracle's tracked tensors against the GPU's, bit for bit, after `step`."""
    torch.cuda.synchronize()
    pair.check_tracked(pair.case.subset, label, step)
    sizes = sorted((pair.orc.p[i].size for i in pair.case.subset), reverse=True)
    log(f"[{label}] step {step}: {len(pair.case.subset)} tracked tensors bit-exact (largest {sizes[:2]} elements)")


def _run_full(pair: Pair, label: str, check_at: set, skip_step: int | None = None) -> None:
    """Steps 1..case.steps: the rotated tensors' state copied out, the GPU
    step, the oracle's step (norm checked first), the rotated tensors
    compared; the tracked subset compared at the steps in check_at; at
    skip_step the whole state is checksummed before and after the (skipped)
    step."""
    c = pair.case
    assert c.host_grads
    for s in range(1, c.steps + 1):
        lr = mg.cosine_lr(s - 1, *c.lr_sched)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        rot = pair.rotation.get(s, [])
        if rot:
            pair.snapshot(rot)
        before = _checksums(pair) if s == skip_step else None
        pair.gpu_step()
        out = pair.oracle_step_full(s, lr, rot)
        if rot:
            pair.check_rotated(rot, label, s)
        if before is not None:
            torch.cuda.synchronize()
            assert out["skipped"]
            assert _checksums(pair) == before, "a skipped step changed the optimizer state"
        if s in check_at or s == skip_step or rot and len(rot) and s % 10 == 0:
            ng, no = out["norm_gpu"], out["norm"]
            log(f"[{label}] step {s}: norm {ng!r} (device fp64 {no!r}){' skipped' if out['skipped'] else ''}"
                f"{f'; {len(rot)} rotated tensors bit-exact' if rot else ''}")
        if s in check_at:
            _check_subset(pair, label, s)
    torch.cuda.synchronize()


def _check_full(pair: Pair, label: str, expect_steps: int) -> None:
    """After the run: the scale trajectory, every step count, the bf16 copies,
    and the coverage counts (every tensor value-checked at least once)."""
    if pair.case.scaler:
        assert [float(t) for t in pair.scale_gpu] == [o["scale"] for o in pair.outs]
    eng = pair.opt._engine
    assert bool((eng.steps == float(expect_steps)).all())
    if eng.master is not None:
        for i, p in enumerate(pair.params):
            m = pair.opt.state[p]["master_param"]
            assert torch.equal(m.to(p.dtype).view(torch.int16), p.detach().view(torch.int16)), (label, i)
    assert eng.device_bc_flag() == 0
    n = len(pair.shapes)
    tracked = len(pair.case.subset)
    if pair.case.rotate:
        assert pair.rotated_checked + tracked == n, (pair.rotated_checked, tracked, n)
    nc = pair.norm_checks
    assert nc["steps"] == pair.case.steps
    log(f"[{label}] {len(pair.outs)} steps; norms checked independently at {nc['steps']} of {pair.case.steps} steps "
        f"(device fp64, {nc['device_exact']} bit-equal) and {nc['host']} by host rebuild ({nc['host_exact']} "
        f"bit-equal); tensors value-checked: {tracked} tracked from step 1 + {pair.rotated_checked} rotated "
        f"= {tracked + pair.rotated_checked} of {n}")
    log(f"[{label}] seconds: " + ", ".join(f"{k} {v:.1f}" for k, v in sorted(pair.seconds.items(), key=lambda x: -x[1])))


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
    17 and 53, 200 steps.  Tracked from step 1: the tied token embedding
    (38.6M elements), three more matrices and every no-decay tensor; the other
    46 matrices rotated; the norm checked at every step on the device and by
    the host rebuild."""
    shapes = mg.paramsets.WORKLOADS["gpt2_small"]()
    rng = np.random.RandomState(17)
    inject = {s: [(int(rng.randint(len(shapes))), 0, float("inf"))] for s in (17, 53)}
    decay_n = sum(1 for _, s in shapes if len(s) >= 2)
    subset = [0, 1, 4, 5] + list(range(decay_n, len(shapes)))
    log("case: gpt2_small 200 steps")
    pair = Pair(Case(shapes=shapes, grad_dtype="f16", steps=200, sigma=1e-2,
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000),
                     inject=inject, subset=subset, lr_sched=(6e-4, 6e-5, 10, 200), host_grads=True, rotate=True))
    _run_full(pair, "gpt2_small_200", check_at={1, 17, 53, 100, 200})
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [17, 53]
    assert pair.outs[-1]["scale"] == 16384.0 and pair.outs[-1]["tracker"] == 200 - 53
    _check_full(pair, "gpt2_small_200", 198)


def test_gpt_1p3b_full_size_bf16_master():
    """1.3B GPT (24 layers, width 2048, vocab 50304): bf16 params and grads,
    fp32 master/m/v, grads N(0,1e-3) with 0.1% x100 so clipping acts every
    step; 100 steps.  Tracked from step 1: the token embedding (103M
    elements), four more matrices and every no-decay tensor; the other 187
    matrices rotated; the norm checked at every step on the device and at ten
    by the host rebuild."""
    shapes = mg.paramsets.WORKLOADS["gpt_1p3b"]()
    log("case: gpt_1p3b full size, 100 steps")
    decay = [s for _, s in shapes if len(s) >= 2]
    nodecay_idx = list(range(len(decay), len(shapes)))
    subset = [0, 1, 2, 3, len(decay) - 1] + nodecay_idx
    pair = Pair(Case(shapes=shapes, param_dtype="bf16", grad_dtype="bf16", steps=100, sigma=1e-3,
                     tail=(1000, 100.0), subset=subset, host_grads=True, rotate=True,
                     verify_norm={1, 2, 3, 4, 5, 10, 25, 50, 75, 100}))
    _run_full(pair, "gpt_1p3b", check_at={1, 10, 50, 100})
    assert all(o["norm"] > 1.0 for o in pair.outs)
    assert all(float(t) > 1.0 for t in pair.norms_gpu)
    _check_full(pair, "gpt_1p3b", 100)


def test_gpt_1p3b_full_size_fp32_params_with_scaler():
    """The class the reference's loop steps on a GPU (train.py:359-370: fp32
    parameters and gradients, a GradScaler for fp16 autocast, clip 1.0) at
    the 1.3B GPT's full size: 1,313,722,368 fp32 params, heavy-tailed grads
    (clipping every step), growth interval 5, 20 steps with an inf at step 4
    (a skipped step over the whole set).  Every norm checked against the
    device fp64 total, three also by the host rebuild; the token embedding,
    the last matrix and every no-decay tensor tracked from step 1, the other
    matrices rotated, so every tensor is value-checked."""
    shapes = mg.paramsets.WORKLOADS["gpt_1p3b"]()
    decay_n = sum(1 for _, s in shapes if len(s) >= 2)
    subset = [0, decay_n - 1] + list(range(decay_n, len(shapes)))
    log("case: gpt_1p3b full size, fp32 params and grads, scaler, 20 steps, inf at step 4")
    pair = Pair(Case(shapes=shapes, param_dtype="f32", grad_dtype="f32", steps=20, sigma=1e-3, tail=(1000, 100.0),
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=5),
                     inject={4: [(3, 77, float("inf"))]}, subset=subset, host_grads=True, rotate=True,
                     verify_norm={1, 4, 20}))
    _run_full(pair, "gpt_1p3b fp32", check_at={1, 10, 20}, skip_step=4)
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [4]
    assert pair.outs[-1]["scale"] == 65536.0 / 2 * 2 ** 3
    _check_full(pair, "gpt_1p3b fp32", 19)


def test_qwen3_8b_full_size():
    """Qwen3-8B-shaped set, 8,190,735,360 params (131 GB resident): bf16 params
    and grads, fp32 master/m/v, GradScaler, clip 1.0; 100 steps with +inf at
    step 2 (a skipped step over the whole set).  Tracked from step 1:
    model.embed_tokens and lm_head (622M elements each, the only tensors whose
    fp32 master exceeds 2 GiB), four layer matrices and every RMSNorm weight;
    the other 248 matrices rotated; the norm checked at every step on the
    device and at three by the host rebuild.  MGOPT_QWEN3_STEPS=N runs N
    steps instead (a multiple of 25), tracked tensors checked every 25."""
    steps = int(os.environ.get("MGOPT_QWEN3_STEPS", "100"))
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
                     rotate=True, verify_norm={1, 2, steps}))
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


def test_ragged_20k_full_size_2000_steps():
    """The ragged tensor-list stress at full size: 20,000 fp32 tensors with
    log-uniform sizes over 1..4M elements rescaled to 2,500,000,199 elements,
    half in the no-decay group, fp16 gradients N(0,1e-2) x 65536 filled once,
    GradScaler from 65536 with growth_interval 50, a NaN or an inf at one
    element in 1% of 2,000 steps (20 seeded steps), clip 1.0.

    Checked: the scale and growth-tracker trajectory against the oracle's
    state machine at every step, and with it every skip decision; every
    step's norm against the host total over all 20,000 gradients rebuilt on
    the host (the gradients are fixed, so the total depends on the scale only:
    it is computed directly at the starting, smallest and largest scales, and
    the others follow from the one at the starting scale by the exact
    power-of-two factor, which the direct totals confirm bit for bit); at the
    first bad step, every arena unchanged; at the end every step count, and
    60 tensors (the 20 largest, the 20 smallest and 20 in the middle) stepped
    by the oracle through all 2,000 steps from the same gradients, bit for
    bit; each of the other 19,940 tensors at one step of the run, from its
    state copied off the GPU before that step, with the scale and the clip
    coefficient of the host totals, bit for bit.  The scale climbs from 65536
    to 2^30 and comes back down, so clipping is active early and inactive
    late."""
    shapes = mg.paramsets.WORKLOADS["ragged_20k"]()
    rng = np.random.RandomState(11)
    bad_steps = sorted(rng.choice(np.arange(1, 2001), 20, replace=False).tolist())
    sc = dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=50)
    ordered = [s for _, s in shapes if len(s) >= 2] + [s for _, s in shapes if len(s) < 2]
    numel = [math.prod(s) for s in ordered]
    assert sum(numel) == 2_500_000_199
    by_size = sorted(range(len(ordered)), key=lambda i: (numel[i], i))
    mid = len(by_size) // 2
    subset = sorted(set(by_size[:20] + by_size[-20:] + by_size[mid - 10: mid + 10]))
    log(f"case: ragged 20k tensors full size, 2000 steps, bad steps {bad_steps}")
    pair = Pair(Case(shapes=shapes, grad_dtype="f16", steps=2000, sigma=1e-2, scaler=sc, max_norm=1.0,
                     fresh_grads=False, subset=subset))
    grads = pair.current_grads()
    k = O.synth_k(1e-2 * 65536)
    for i, g in enumerate(grads):
        syn.fill_(g, syn.GRAD_SEED, syn.grad_stream(1, i), 1e-2 * 65536)

    # every gradient as the GPU holds it, rebuilt on the host into one flat array
    offsets = np.concatenate([[0], np.cumsum(numel)])
    flat = np.empty(int(offsets[-1]), np.float32)
    list(O.pool().map(lambda i: O.synth_grad(numel[i], syn.GRAD_SEED, syn.grad_stream(1, i), k, "f16",
                                             out=flat[offsets[i]: offsets[i + 1]]), range(len(numel))))
    host = [flat[offsets[i]: offsets[i + 1]] for i in range(len(numel))]
    # the scale before each step, from the oracle's state machine
    scale, tracker, before_step = 65536.0, 0, []
    for s in range(1, 2001):
        before_step.append(scale)
        scale, tracker = O.scaler_update(scale, tracker, 1.0 if s in bad_steps else 0.0, 2.0, 0.5, 50)
    distinct = sorted(set(before_step))
    s0 = O.grads_sumsq([(flat, "f32")], inv=O.inv_scale(65536.0), unscale=True)
    assert not s0[1] and math.isfinite(s0[0])

    def derived(scale: float) -> float:
        # u = fp32(g * inv) scales by an exact power of two with inv (no fp32
        # overflow or underflow at these magnitudes), so every square, partial
        # sum and correction term of the fp64 total scales exactly too
        return s0[0] * (O.inv_scale(scale) / O.inv_scale(65536.0)) ** 2

    totals = {}
    for scale in {distinct[0], 65536.0, distinct[-1]}:
        direct = O.grads_sumsq([(flat, "f32")], inv=O.inv_scale(scale), unscale=True)
        assert not direct[1] and direct[0] == derived(scale), (scale, direct[0], derived(scale))
        totals[scale] = direct[0]
    for scale in distinct:
        totals.setdefault(scale, derived(scale))
    log(f"[ragged full] host gradients rebuilt; totals at {len(distinct)} distinct scales "
        f"({distinct[0]:g} .. {distinct[-1]:g})")

    # every tensor outside the tracked subset is checked at one step: its
    # state copied from the GPU before that step, stepped by the oracle from
    # the host gradient with the scale and the clip coefficient of the host
    # totals (nothing taken from the GPU), compared bit for bit after it
    rotation = rotation_schedule({i: numel[i] for i in range(len(numel)) if i not in set(subset)},
                                 [s for s in range(2, 2001) if s not in bad_steps])

    def rotated_step(idx: list[int], step: int) -> None:
        sc_before = before_step[step - 1]
        coef = O.clip_coef(O.norm_from_sumsq(totals[sc_before]), 1.0)
        jobs = []
        for i in idx:
            h = pair.orc.hparams[pair.orc.group_of[i]]
            pair.orc.steps[i] += 1.0
            jobs.append((host[i], pair.orc.p[i], pair.orc.m[i], pair.orc.v[i],
                         dict(inv=O.inv_scale(sc_before), unscale=True, coef=coef, lr=1e-4, beta1=h["betas"][0],
                              beta2=h["betas"][1], eps=h["eps"], wd=h["weight_decay"], step=pair.orc.steps[i])))
        O.unscale_clip_adamw_many(jobs)

    injected = {}
    for s in range(1, 2001):
        restore = None
        if s in bad_steps:
            ti = int(rng.randint(len(grads)))
            restore = (ti, grads[ti].view(-1)[0].clone())
            injected[s] = (ti, float("nan") if s % 2 else float("inf"))
            grads[ti].view(-1)[0] = injected[s][1]
        before = _checksums(pair) if s == bad_steps[0] else None
        rotated = rotation.get(s, [])
        if rotated:
            torch.cuda.synchronize()
            pair.snapshot(rotated)
        mg.set_optimizer_lr(pair.opt, 1e-4)
        pair.gpu_step()
        if before is not None:
            assert _checksums(pair) == before, "a skipped step changed the optimizer state"
        if rotated:
            rotated_step(rotated, s)
            torch.cuda.synchronize()
            pair.check_rotated(rotated, "ragged full rotated", s)
        if restore is not None:
            grads[restore[0]].view(-1)[0] = restore[1]
        if s % 500 == 0:
            log(f"[ragged full] GPU step {s}; {pair.rotated_checked} rotated tensors bit-exact so far")
    torch.cuda.synchronize()
    norms = torch.stack(pair.norms_gpu).cpu().numpy().tolist()
    gpu_scales = torch.stack(pair.scale_gpu).cpu().numpy().tolist()
    assert pair.rotated_checked == len(numel) - len(subset)
    log("[ragged full] GPU 2000 steps done; oracle replay of the 60-tensor subset")

    sub_grads = [host[i] if i in set(subset) else None for i in range(len(host))]
    exact_norms = 0
    for s in range(1, 2001):
        ng = norms[s - 1]
        if s in bad_steps:
            ti, val = injected[s]
            assert not math.isfinite(val)
            out = pair.orc.step(sub_grads, 1e-4, subset=subset, totals=(val * val, True), norm_override=ng)
            assert out["skipped"] and (math.isnan(ng) if math.isnan(val) else ng == math.inf), (s, ng)
        else:
            out = pair.orc.step(sub_grads, 1e-4, subset=subset, totals=(totals[pair.orc.scale], False),
                                norm_override=ng)
            assert not out["skipped"] and rel(ng, out["norm"]) <= RTOL_NORM, (s, ng, out["norm"])
            exact_norms += ng == out["norm"]
        pair.outs.append(out)
        assert gpu_scales[s - 1] == out["scale"], (s, gpu_scales[s - 1], out["scale"])
        if s % 500 == 0:
            log(f"[ragged full] oracle step {s}")
    assert pair.scaler._get_growth_tracker() == pair.outs[-1]["tracker"]
    assert max(o["scale"] for o in pair.outs) >= 2.0 ** 30
    clipped = sum(1 for n in norms if math.isfinite(n) and n > 1.0)
    assert 0 < clipped < 2000 - len(bad_steps)
    steps = pair.opt._engine.steps.cpu().numpy()
    assert np.all(steps == 2000 - len(bad_steps))
    for i in subset:
        st = pair.gpu_state(i)
        assert st["step"] == pair.orc.steps[i] == 2000 - len(bad_steps), i
        for key, ref in (("p", pair.orc.p[i]), ("m", pair.orc.m[i]), ("v", pair.orc.v[i])):
            assert exact_fraction(st[key], ref.ravel()) == 1.0, (key, i)
    assert pair.opt._engine.device_bc_flag() == 0
    sizes = sorted((numel[i] for i in subset), reverse=True)
    log(f"[ragged full] final scale {gpu_scales[-1]}; {2000 - len(bad_steps)} norms checked against the host total "
        f"({exact_norms} bit-equal), {len(bad_steps)} skips; {clipped} steps clipped; {len(subset)} tensors "
        f"(largest {sizes[0]}, smallest {sizes[-1]} elements) bit-exact after 2000 steps; tensors value-checked: "
        f"{len(subset)} tracked from step 1 + {pair.rotated_checked} rotated = {len(subset) + pair.rotated_checked} "
        f"of {len(numel)}")
