"""The drop-in inside a real training loop: a small MiniGPT-shaped model on the
GPU, gradients from autograd, the iteration of train.py:457-491
(set_optimizer_lr, zero_grad(set_to_none=True), scaler.scale(loss).backward(),
unscale_, clip_grad_norm_, step, update), run in lockstep with torch's own
AdamW(fused=False, foreach=False) + torch.amp.GradScaler on a copy of the same
model and data.

Two checks per step:
  - the optimizer step itself, bit for bit: before each step the engine's
    state and the gradients it will read are copied to the host, and after
    the step the GPU state must equal the CPU oracle's update of that copy
    (its norm within 1e-5, its clip coefficient from the engine's norm once
    that agreed, as in the full-size tests); the loss scale must equal the
    oracle's state machine;
  - the surface against torch: torch's side is clipped with the engine's
    norm (torch.nn.utils.clip_grads_with_norm_), so that the two runs differ
    only by torch's GPU AdamW arithmetic, which rounds differently from its
    CPU path (the oracle's), and by what that difference does to the later
    forward passes.  Skip decisions and the loss-scale trajectory must agree
    exactly; losses and norms within 1e-6; parameters within the bar each
    test states, set from the differences measured on MI355X.
"""

from __future__ import annotations

import copy
import math

import pytest
import torch
from torch import nn

from oracle import oracle as O
from tests._compare import RTOL_NORM, bits_equal, rel
from tests._gpu_harness import log, mg

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
#: parameter bars against torch's GPU AdamW (max |a - b| / max |b| per tensor),
#: about 1.5-2x the differences measured on MI355X (each test's docstring)
PARAM_BAR_TINY = 1.5e-6
PARAM_BAR_ARENA = 3e-6


@pytest.fixture(autouse=True, params=[True, False], ids=["three_kernels", "five_kernels"])
def step_form(request, monkeypatch):
    """Every test here runs with the step of a small plan in its three-kernel
    form and again in the five-kernel form of larger plans (MGOPT_FOLD=0 when
    the plans are made)."""
    if not request.param:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    return request.param


class Block(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.ln_1 = nn.LayerNorm(c)
        self.mix = nn.Linear(c, 3 * c)
        self.out_proj = nn.Linear(3 * c, c)
        self.ln_2 = nn.LayerNorm(c)
        self.fc = nn.Linear(c, 4 * c)
        self.proj = nn.Linear(4 * c, c)

    def forward(self, x):
        x = x + self.out_proj(torch.tanh(self.mix(self.ln_1(x))))
        return x + self.proj(nn.functional.gelu(self.fc(self.ln_2(x))))


class TinyLM(nn.Module):
    """Token + position embeddings, residual blocks, final norm, a head tied to
    the token embedding (the MiniGPT parameter structure, src/minigpt/model.py:271-312)."""

    def __init__(self, vocab=96, block=32, n_layer=3, c=64):
        super().__init__()
        self.token_embedding = nn.Embedding(vocab, c)
        self.position_embedding = nn.Embedding(block, c)
        self.blocks = nn.ModuleList(Block(c) for _ in range(n_layer))
        self.ln_f = nn.LayerNorm(c)
        self.lm_head = nn.Linear(c, vocab, bias=False)
        self.lm_head.weight = self.token_embedding.weight

    def forward(self, idx):
        pos = torch.arange(idx.shape[1], device=idx.device)
        x = self.token_embedding(idx) + self.position_embedding(pos)
        for b in self.blocks:
            x = b(x)
        return self.lm_head(self.ln_f(x))


class OracleCheck:
    """The CPU oracle stepped beside one of this package's AdamW optimizers
    inside an autograd loop: before() copies the engine's state and the
    gradients its step will read; after(norm) steps the oracle from that copy
    and compares the GPU's parameters, moments, step counts and loss scale
    with it, bit for bit."""

    def __init__(self, opt, scaler, growth_interval: int, max_norm: float = 1.0):
        self.opt, self.scaler, self.max_norm = opt, scaler, max_norm
        self.cfg = dict(init_scale=scaler.get_scale(), growth_factor=2.0, backoff_factor=0.5,
                        growth_interval=growth_interval)
        self.steps_checked = 0
        self.norms_exact = 0

    def before(self) -> None:
        eng = self.opt._get_engine()
        self.params = eng.params
        grads = eng.current_grads()
        self.grads = [None if g is None else g.detach().float().cpu().numpy().ravel().copy() for g in grads]
        group_of = list(eng.group_index)
        hp = [dict(betas=tuple(g["betas"]), eps=g["eps"], weight_decay=g["weight_decay"]) for g in self.opt.param_groups]
        self.lrs = [float(g["lr"]) for g in self.opt.param_groups]
        init = [p.detach().float().cpu().numpy().ravel().copy() for p in self.params]
        self.orc = O.OracleRun(init, group_of, hp, scaler=self.cfg, max_norm=self.max_norm)
        for i, p in enumerate(self.params):
            st = self.opt.state.get(p)
            if st:
                self.orc.load(i, init[i], st["exp_avg"].detach().cpu().numpy().ravel().copy(),
                              st["exp_avg_sq"].detach().cpu().numpy().ravel().copy(), float(st["step"]))
        self.orc.scale = float(self.scaler._scale)
        self.orc.tracker = int(self.scaler._get_growth_tracker())

    def after(self, norm: torch.Tensor) -> None:
        ng = float(norm)
        out = self.orc.step(self.grads, self.lrs, norm_override=ng)
        no = out["norm"]
        if math.isfinite(no):
            assert rel(ng, no) <= RTOL_NORM, (ng, no)
        else:
            assert (math.isnan(no) and math.isnan(ng)) or ng == no, (ng, no)
        self.norms_exact += ng == no or not math.isfinite(no)
        assert out["scale"] == self.scaler.get_scale(), (out["scale"], self.scaler.get_scale())
        for i, p in enumerate(self.params):
            st = self.opt.state.get(p)
            if self.grads[i] is None and not st:
                continue    # never had a gradient: no state on either side
            assert float(st["step"]) == self.orc.steps[i], (i, float(st["step"]), self.orc.steps[i])
            for got, ref in ((p, self.orc.p[i]), (st["exp_avg"], self.orc.m[i]), (st["exp_avg_sq"], self.orc.v[i])):
                assert bits_equal(got.detach().cpu().numpy().ravel(), ref), (i, self.steps_checked)
        self.steps_checked += 1


def _lockstep(ref, mine, batches, inject, set_to_none=True, micro=1, schedulers=(None, None), lr_warmup=5,
              check: OracleCheck | None = None):
    """Runs both sides over the same batches, one iteration at a time.
    ref / mine: (model, optimizer, scaler).  inject(model) puts an inf into one
    gradient at the step `inject.step`.  Returns per-side (losses, norms,
    scales); torch's norm is its own (get_total_norm), but its gradients are
    clipped with the engine's."""
    hist = {"ref": ([], [], []), "mine": ([], [], [])}
    for s, (x, y) in enumerate(batches, start=1):
        norms = {}
        for side, (model, opt, scaler), sched in (("mine", mine, schedulers[1]), ("ref", ref, schedulers[0])):
            if sched is None:
                mg.set_optimizer_lr(opt, mg.cosine_lr(s - 1, 3e-3, 3e-4, lr_warmup, len(batches)))
            opt.zero_grad(set_to_none=set_to_none)
            total = 0.0
            for xm, ym in zip(x.chunk(micro), y.chunk(micro)):
                loss = nn.functional.cross_entropy(model(xm).flatten(0, 1), ym.flatten()) / micro
                scaler.scale(loss).backward()
                total = total + loss.detach()
            if s == inject.step:
                inject(model)
            scaler.unscale_(opt)
            if side == "mine":
                if check is not None:
                    check.before()
                norms["mine"] = mg.clip_grad_norm_(model.parameters(), 1.0)
            else:
                grads = [p.grad for p in model.parameters() if p.grad is not None]
                norms["ref"] = torch.nn.utils.get_total_norm(grads)
                torch.nn.utils.clip_grads_with_norm_(model.parameters(), 1.0, norms["mine"].to(grads[0].device))
            scaler.step(opt)
            scaler.update()
            if side == "mine" and check is not None:
                check.after(norms["mine"])
            if sched is not None:
                sched.step()
            h = hist[side]
            h[0].append(total)
            h[1].append(norms[side])
            h[2].append(scaler.get_scale())
    torch.cuda.synchronize()
    return {k: ([float(v) for v in h[0]], [float(v) for v in h[1]], h[2]) for k, h in hist.items()}


class _Inject:
    def __init__(self, step, fn):
        self.step, self.fn = step, fn

    def __call__(self, model):
        self.fn(model)


def _compare(res, n_steps: int, bad: int, my_opt, ref_opt):
    mine, ref = res["mine"], res["ref"]
    assert mine[2] == ref[2], (mine[2], ref[2])            # loss-scale trajectory, skip included
    assert mg.optimizer_completed_steps(my_opt) == mg.optimizer_completed_steps(ref_opt) == n_steps - 1
    worst_loss = max(abs(a - b) / abs(b) for a, b in zip(mine[0], ref[0]))
    finite = [(a, b) for a, b in zip(mine[1], ref[1]) if math.isfinite(b)]
    assert len(finite) == n_steps - 1 and not math.isfinite(mine[1][bad - 1])
    worst_norm = max(abs(a - b) / abs(b) for a, b in finite)
    return worst_loss, worst_norm


def _worst_param(ref_model, my_model):
    worst = 0.0
    for p, q in zip(ref_model.parameters(), my_model.parameters()):
        d = (p.detach() - q.detach()).abs().max().item() / max(p.detach().abs().max().item(), 1e-30)
        worst = max(worst, d)
    return worst


def _batches(n, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for _ in range(n):
        x = torch.randint(0, 96, (8, 32), generator=g)
        out.append((x.to(DEV), torch.roll(x, -1, dims=1).to(DEV)))
    return out


def _fc_inf(model):
    model.blocks[1].fc.weight.grad.view(-1)[11] = float("inf")


def test_training_loop_matches_torch_on_the_same_model():
    """40 steps, cosine schedule, GradScaler growth every 10, an inf at step 13.
    Measured against torch on MI355X: parameters 7.5e-7 to 7.8e-7 (bar
    1.5e-6), losses 1.1e-7, norms 1.6e-7; every step bit-exact against the
    oracle."""
    torch.manual_seed(0)
    ref_model = TinyLM().to(DEV)
    my_model = copy.deepcopy(ref_model)
    batches = _batches(40, 1)
    ref_opt = torch.optim.AdamW(mg.build_adamw_param_groups(ref_model, 0.1), lr=3e-3, betas=(0.9, 0.95), eps=1e-8,
                                fused=False, foreach=False)
    ref_scaler = torch.amp.GradScaler("cuda", init_scale=2.0**12, growth_interval=10)
    my_opt = mg.AdamW(mg.build_adamw_param_groups(my_model, 0.1), lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    my_scaler = mg.GradScaler("cuda", init_scale=2.0**12, growth_interval=10)
    check = OracleCheck(my_opt, my_scaler, growth_interval=10)

    log("case: tiny LM training loop, 40 steps, inf at step 13")
    res = _lockstep((ref_model, ref_opt, ref_scaler), (my_model, my_opt, my_scaler), batches, _Inject(13, _fc_inf),
                    check=check)
    worst_loss, worst_norm = _compare(res, 40, 13, my_opt, ref_opt)
    worst_param = _worst_param(ref_model, my_model)
    log(f"[train loop] oracle: {check.steps_checked} steps bit-exact, norms bit-equal {check.norms_exact}; against "
        f"torch: worst rel loss {worst_loss:.2e} norm {worst_norm:.2e} param {worst_param:.2e}")
    assert check.steps_checked == 40
    assert worst_loss <= 1e-6 and worst_norm <= 1e-6 and worst_param <= PARAM_BAR_TINY
    assert my_opt._engine.device_bc_flag() == 0


def test_accumulation_in_place_zeroing_and_a_torch_scheduler():
    """The same loop with gradients accumulated over 4 micro-batches,
    zero_grad(set_to_none=False) (the .grad tensors persist and are zeroed in
    place, so the optimizer sees the same gradient storage every step) and
    torch's LambdaLR driving the learning rate.  Measured against torch on
    MI355X: parameters 9.5e-7 to 9.8e-7 (bar 1.5e-6); every step bit-exact
    against the oracle."""
    torch.manual_seed(2)
    ref_model = TinyLM().to(DEV)
    my_model = copy.deepcopy(ref_model)
    batches = _batches(30, 3)
    kw = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    ref_opt = torch.optim.AdamW(mg.build_adamw_param_groups(ref_model, 0.1), fused=False, foreach=False, **kw)
    my_opt = mg.AdamW(mg.build_adamw_param_groups(my_model, 0.1), **kw)
    decay = lambda s: 0.97 ** s
    ref_sched = torch.optim.lr_scheduler.LambdaLR(ref_opt, decay)
    my_sched = torch.optim.lr_scheduler.LambdaLR(my_opt, decay)
    ref_scaler = torch.amp.GradScaler("cuda", init_scale=2.0**12, growth_interval=7)
    my_scaler = mg.GradScaler("cuda", init_scale=2.0**12, growth_interval=7)
    check = OracleCheck(my_opt, my_scaler, growth_interval=7)

    log("case: tiny LM, 4 micro-batches, zero_grad(set_to_none=False), LambdaLR, 30 steps, inf at step 9")
    res = _lockstep((ref_model, ref_opt, ref_scaler), (my_model, my_opt, my_scaler), batches, _Inject(9, _fc_inf),
                    set_to_none=False, micro=4, schedulers=(ref_sched, my_sched), check=check)
    worst_loss, worst_norm = _compare(res, 30, 9, my_opt, ref_opt)
    assert my_opt.param_groups[0]["lr"] == ref_opt.param_groups[0]["lr"]
    worst_param = _worst_param(ref_model, my_model)
    log(f"[accumulation loop] oracle: {check.steps_checked} steps bit-exact, norms bit-equal {check.norms_exact}; "
        f"against torch: worst rel loss {worst_loss:.2e} norm {worst_norm:.2e} param {worst_param:.2e}")
    assert check.steps_checked == 30
    assert worst_loss <= 1e-6 and worst_norm <= 1e-6 and worst_param <= PARAM_BAR_TINY
    assert my_opt._engine.device_bc_flag() == 0


@pytest.mark.parametrize("set_to_none", [True, False])
def test_grad_arena_accumulation_matches_torch(set_to_none):
    """The gradient arena (AdamW.use_grad_arena: every .grad a view of one flat
    buffer, zero_grad one fill) inside the accumulation loop of
    train.py:465-481 -- 4 micro-batches, an inf at step 7 -- on a model with
    MiniGPT's parameter structure plus a module the forward never reads,
    against torch AdamW(fused=False, foreach=False) + GradScaler on a copy.
    torch never gives the unused parameters a gradient, so it never steps
    them and keeps no state for them: the arena must do the same under both
    zero_grad modes.  Every step is bit-exact against the oracle; against
    torch, parameters measured 1.69e-6 on MI355X (bar 3e-6).  With both
    sides clipped by the same norm and this engine's steps bit-exact, that
    figure is torch's GPU AdamW rounding and what it does to the later
    forward passes of this (larger) model."""
    from tests._minigpt import MiniGPT, batches

    torch.manual_seed(4)
    ref_model = MiniGPT(unused_module=True).to(DEV)
    my_model = copy.deepcopy(ref_model)
    data = batches(24, seed=5)
    kw = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    ref_opt = torch.optim.AdamW(mg.build_adamw_param_groups(ref_model, 0.1), fused=False, foreach=False, **kw)
    my_opt = mg.AdamW(mg.build_adamw_param_groups(my_model, 0.1), **kw)
    arena = my_opt.use_grad_arena()
    ref_scaler = torch.amp.GradScaler("cuda", init_scale=2.0**12, growth_interval=5)
    my_scaler = mg.GradScaler("cuda", init_scale=2.0**12, growth_interval=5)
    unused0 = [p.detach().clone() for p in my_model.unused.parameters()]
    check = OracleCheck(my_opt, my_scaler, growth_interval=5)

    def mlp_inf(model):
        model.blocks[1].mlp.fc.weight.grad.view(-1)[3] = float("inf")

    log(f"case: gradient arena, set_to_none={set_to_none}, 4 micro-batches, unused module, 24 steps")
    res = _lockstep((ref_model, ref_opt, ref_scaler), (my_model, my_opt, my_scaler), data, _Inject(7, mlp_inf),
                    set_to_none=set_to_none, micro=4, lr_warmup=3, check=check)

    # the arena stayed in place: every used parameter's gradient is still its view
    used = [p for n, p in my_model.named_parameters() if not n.startswith("unused.")]
    assert all(p.grad.untyped_storage().data_ptr() == arena.untyped_storage().data_ptr() for p in used)
    # the unused module: never stepped, no state, as in torch
    for p0, p, q in zip(unused0, my_model.unused.parameters(), ref_model.unused.parameters()):
        assert torch.equal(p.detach(), p0) and torch.equal(q.detach(), p0)
        assert not ref_opt.state.get(q) and not my_opt.state.get(p)
        assert q.grad is None
    # one entry per used parameter (named_parameters lists the tied head once)
    assert len(my_opt.state_dict()["state"]) == len(ref_opt.state_dict()["state"]) == len(used)
    worst_loss, worst_norm = _compare(res, 24, 7, my_opt, ref_opt)
    # The key third of each fused QKV bias (qkv_proj.bias[C:2C]) has an
    # exactly zero gradient in exact arithmetic: softmax ignores a constant
    # added to every score of a query.  Its computed gradient is rounding noise
    # (~1e-10), which Adam divides by sqrt(v) + eps ~ eps, so each optimizer
    # walks those elements by about lr * noise / eps per step along its own
    # noise.  They are compared by that bound; every other element by the bar.
    worst_param, worst_kbias = 0.0, 0.0
    for (name, p), q in zip(ref_model.named_parameters(), my_model.parameters()):
        a, b = p.detach().reshape(-1), q.detach().reshape(-1)
        if name.endswith("attn.qkv_proj.bias"):
            C = a.numel() // 3
            worst_kbias = max(worst_kbias, (a[C:2 * C] - b[C:2 * C]).abs().max().item())
            a, b = torch.cat([a[:C], a[2 * C:]]), torch.cat([b[:C], b[2 * C:]])
        worst_param = max(worst_param, (a - b).abs().max().item() / max(a.abs().max().item(), 1e-30))
    log(f"[arena set_to_none={set_to_none}] oracle: {check.steps_checked} steps bit-exact, norms bit-equal "
        f"{check.norms_exact}; against torch: worst rel loss {worst_loss:.2e} norm {worst_norm:.2e} param "
        f"{worst_param:.2e}; key-bias abs diff {worst_kbias:.2e}")
    assert check.steps_checked == 24
    assert worst_loss <= 1e-6 and worst_norm <= 1e-6 and worst_param <= PARAM_BAR_ARENA
    assert worst_kbias <= len(data) * 3e-3 * 1e-1      # far below one full-size update per step
