"""GPU parity: the HIP path (through the C ABI) against the CPU oracle, on the
workloads the optimizer step is specified on, and against torch's own CPU path
where torch's arithmetic is exact enough to be a reference.

Bars (tests/_compare.py): skip / found_inf / scale / tracker / step counts
bit-exact; fp32 state max relative error <= 1e-6; bf16 params <= 1 ulp; grad
norm <= 1e-5 relative.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests._compare import RTOL_STATE, maxrel
from tests._gpu_harness import Case, Pair, check_pair, log, mg, syn

pytestmark = pytest.mark.gpu


def test_synthetic_fill_matches_oracle():
    for dt in ("f32", "f16", "bf16"):
        for n in (1, 3, 4097, 1_000_003):
            t = torch.empty(n, dtype={"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt], device="cuda")
            syn.fill_(t, 5, 77, 0.7, 100, 1000.0)
            ref = O.synth(n, 5, 77, O.synth_k(0.7), 100, 1000.0)
            if dt == "f32":
                assert np.array_equal(t.cpu().numpy().view(np.uint32), ref.view(np.uint32))
            else:
                bits = t.view(torch.int16).cpu().numpy().view(np.uint16)
                assert np.array_equal(bits, O.to_f16(ref) if dt == "f16" else O.to_bf16(ref)), (dt, n)


@pytest.mark.parametrize("fold", [True, False], ids=["three_kernels", "five_kernels"])
def test_tiny_cpu_workload_100_steps_bit_exact(fold, monkeypatch):
    """MiniGPT tiny_cpu shapes (52 tensors, 822,016 fp32 params), grads
    N(0,1e-3), AdamW lr 3e-4 cosine (warm-up 10), betas (0.9, 0.95), eps 1e-8,
    wd 0.1 on matrices and embeddings, clip 1.0, 100 steps; the three-kernel
    step this small plan runs, and the five-kernel step (MGOPT_FOLD=0)."""
    if not fold:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    log(f"case: minigpt_tiny_cpu 100 steps, fold={fold}")
    pair = Pair(Case(shapes=mg.paramsets.WORKLOADS["minigpt_tiny_cpu"](), steps=100, sigma=1e-3))
    pair.run()
    assert pair.opt._engine.folded() == fold
    check_pair(pair, label="tiny_cpu")


def test_tiny_cpu_workload_against_torch_cpu():
    """Same workload, GPU against torch 2.10's own CPU AdamW + clip_grad_norm_
    (the reference's path): fp32 state within 1e-6 after 100 steps."""
    from oracle.torch_path import TorchReferencePath

    log("case: minigpt_tiny_cpu vs torch cpu")
    pair = Pair(Case(shapes=mg.paramsets.WORKLOADS["minigpt_tiny_cpu"](), steps=100, sigma=1e-3))
    init = [p.detach().cpu().numpy() for p in pair.params]
    hp = [dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1), dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)]
    ref = TorchReferencePath(init, pair.group_of, hp, max_norm=1.0)
    for s in range(1, 101):
        lr = mg.cosine_lr(s - 1, *pair.case.lr_sched)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        ref.step([g.detach().cpu().numpy() for g in pair.current_grads()], lr)
        pair.gpu_step()
    torch.cuda.synchronize()
    worst = 0.0
    for i in range(len(pair.params)):
        st = pair.gpu_state(i)
        p, m, v, step = ref.state(i)
        assert st["step"] == step
        for a, b in ((st["p"], p), (st["m"], m), (st["v"], v)):
            worst = max(worst, maxrel(a, b.ravel()))
    log(f"[tiny_cpu vs torch cpu] worst maxrel {worst:.3e}")
    assert worst <= RTOL_STATE


def test_bf16_master_with_heavy_tail_clipping():
    """bf16 params with fp32 master / m / v, bf16 grads N(0,1e-3) with 0.1% of
    elements x100 so clipping at 1.0 is active every step; a narrower GPT
    (4 layers, width 512, vocab 50304) for 100 steps; every tensor checked."""
    shapes = mg.paramsets.minigpt_shapes(vocab=50304, block=1024, n_layer=4, n_embd=512)
    log("case: bf16 master, heavy tail, 100 steps")
    pair = Pair(Case(shapes=shapes, param_dtype="bf16", grad_dtype="bf16", steps=100, sigma=1e-3,
                     tail=(1000, 100.0)))
    pair.run()
    assert all(o["norm"] > 1.0 for o in pair.outs)
    check_pair(pair, label="bf16_master")
    # the bf16 model copy is the round-to-nearest-even image of the master
    for i in range(len(pair.params)):
        st = pair.gpu_state(i)
        assert np.array_equal(st["lowp_bits"], O.to_bf16(st["p"]))


def test_past_the_first_bias_correction_table_doubling():
    """1,100 steps (the bias-correction table starts at 1,024 steps and grows
    by extending each group's row), with the no-decay group's betas changed at
    step 600 (its row is rebuilt): all state bit-exact against the oracle."""
    shapes = [("w", (48, 37)), ("b", (37,)), ("v", (513,))]
    log("case: 1100 steps across the bias-correction table growth, betas change at 600")
    pair = Pair(Case(shapes=shapes, steps=1, sigma=1e-2, max_norm=1.0))
    for s in range(1, 1101):
        if s == 600:
            pair.opt.param_groups[1]["betas"] = (0.8, 0.99)
            pair.orc.hparams[1]["betas"] = (0.8, 0.99)
        lr = mg.cosine_lr(s - 1, 3e-4, 3e-5, 10, 1100)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        pair.oracle_step(s, lr)
        pair.gpu_step()
    torch.cuda.synchronize()
    assert pair.opt._engine.bc_cap == 2048
    check_pair(pair, label="table_growth")
    assert all(float(pair.opt.state[p]["step"]) == 1100.0 for p in pair.params)


def test_bf16_gradient_arena_bit_exact():
    """bf16 params, bf16 gradients living in the optimizer's gradient arena
    (AdamW.use_grad_arena: each .grad a view of one flat buffer with 256-byte
    segment alignment), GradScaler with an inf at step 9, clip every step; 30
    steps on a narrower GPT: every tensor bit-exact against the oracle."""
    shapes = mg.paramsets.minigpt_shapes(vocab=4096, block=256, n_layer=2, n_embd=256)
    log("case: bf16 gradient arena, 30 steps, inf at step 9")
    pair = Pair(Case(shapes=shapes, param_dtype="bf16", grad_dtype="bf16", steps=30, sigma=1e-3, tail=(1000, 100.0),
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=7),
                     inject={9: [(3, 17, float("inf"))]}, arena=True, fresh_grads=False))
    views = [p.grad for p in pair.params]
    pair.run()
    assert all(p.grad is v for p, v in zip(pair.params, views))
    assert all(v.untyped_storage().data_ptr() == pair.arena.untyped_storage().data_ptr() for v in views)
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [9]
    check_pair(pair, label="bf16_arena")


def test_step_count_written_in_place_beyond_the_table():
    """A step count written straight into the live state tensor
    (state[p]["step"].fill_(...), which no Python hook sees) far beyond the
    host's bias-correction table: the next steps still update every tensor,
    with the bias corrections evaluated on the device, and the engine's flag
    reports it.  Against the oracle at the fp32 tolerance, bit-exact fraction
    logged."""
    shapes = [("w", (64, 33)), ("b", (33,))]
    pair = Pair(Case(shapes=shapes, steps=3, sigma=1e-2, max_norm=1.0))
    pair.run(steps=3)
    for i, p in enumerate(pair.params):
        pair.opt.state[p]["step"].fill_(5000.0 + i)
        pair.orc.steps[i] = 5000.0 + i
    log("case: step counts 5000/5001 written in place, 3 more steps")
    pair.run(steps=6, start=4)
    assert pair.opt._engine.device_bc_flag() == 1
    assert [float(pair.opt.state[p]["step"]) for p in pair.params] == [5003.0, 5004.0]
    check_pair(pair, expect_exact=False, label="in_place_step", device_bc=1)
