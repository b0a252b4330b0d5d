"""GPU parity on the special values of unscale / found_inf / the norm:
+inf, -inf and NaN at chunk edges, in the scalar tail loop and in a
one-element tensor; fp16's largest finite values; a norm that overflows the
fp32 range although every gradient is finite; and an unscale that overflows
at a loss scale below 1.

The last two are what torch does, not what one might expect: found_inf looks
at the scaled input only (grad_scaler.py:280-284 -> the non-finite check runs
before the multiply), and clip_grad_norm_ multiplies by a zero coefficient
when the norm is inf (clip_grad.py:165-174), so an element that overflowed in
the unscale becomes inf * 0 = NaN and the optimizer step is taken.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from tests._compare import RTOL_STATE, maxrel
from tests._gpu_harness import Case, Pair, check_pair, log, mg

pytestmark = pytest.mark.gpu

# decay: w0, w1 (3 x 4099: chunks of 4096, 4096, 4096 and 9 elements), w2 (2 x 4096:
# state in the row layout, two rows); no decay: b0 (7), s (one element), b1 (4101: a
# vector body and a scalar tail)
SHAPES = [("w0", (64, 130)), ("w1", (3, 4099)), ("w2", (2, 4096)), ("b0", (7,)), ("s", (1,)), ("b1", (4101,))]
CHUNK = 4096


@pytest.fixture(autouse=True, params=[True, False], ids=["three_kernels", "five_kernels"])
def step_form(request, monkeypatch):
    """Every case runs with the step of a small plan in its three-kernel form
    and again in the five-kernel form of larger plans (MGOPT_FOLD=0 when the
    plans are made): their pass-1 chunks and finalize differ."""
    if not request.param:
        monkeypatch.setenv("MGOPT_FOLD", "0")
    return request.param


def test_nonfinite_at_chunk_edges_and_tails():
    """fp32 params, fp16 grads, GradScaler 65536, chunks of 4096 elements: a
    non-finite value at each edge of the work decomposition skips exactly its
    step; fp16 +-65504 (finite) does not."""
    inject = {
        2: [(5, -1, math.inf)],          # last element of the last tensor (scalar tail)
        3: [(0, 0, -math.inf)],          # first element of the first tensor
        4: [(1, CHUNK - 1, math.nan)],   # last element of a full chunk
        5: [(1, CHUNK, math.nan)],       # first element of the next chunk
        6: [(1, 3 * 4099 - 1, math.inf)],  # last element of a 9-element tail chunk
        7: [(4, 0, -math.inf)],          # the one-element tensor
        9: [(2, 2 * CHUNK - 1, 65504.0), (3, 6, -65504.0)],  # fp16 extremes: finite
    }
    log("case: non-finite at chunk edges, fp16 grads, chunk 4096")
    pair = Pair(Case(shapes=SHAPES, grad_dtype="f16", steps=10, sigma=1e-2, chunk_elems=CHUNK,
                     scaler=dict(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000),
                     inject=inject))
    pair.run()
    assert [s + 1 for s, o in enumerate(pair.outs) if o["skipped"]] == [2, 3, 4, 5, 6, 7]
    assert pair.outs[-1]["scale"] == 65536.0 / 64
    check_pair(pair, label="chunk_edges")
    assert all(float(pair.opt.state[p]["step"]) == 4.0 for p in pair.params)
    assert pair.opt._engine.rows == [0, 0, 4096, 0, 0, 0]


def test_norm_overflow_with_finite_gradients():
    """bf16 params and grads, no scaler: two finite elements of 1e20 make the
    sum of squares exceed the fp32 range, so the norm is inf (as torch's fp32
    accumulation gives), the coefficient is 0 and the step applies zero
    gradients; the run continues normally afterwards."""
    inject = {2: [(0, 5, 1e20), (3, 0, -1e20)]}
    log("case: norm overflow with finite bf16 grads")
    pair = Pair(Case(shapes=SHAPES, param_dtype="bf16", grad_dtype="bf16", steps=4, sigma=1e-3, chunk_elems=CHUNK,
                     inject=inject))
    # what torch's own clip_grad_norm_ returns for the step-2 gradients
    captured = {}
    orig = pair.fill_grads

    def fill_and_capture(step):
        orig(step)
        if step == 2:
            captured["grads"] = [g.detach().cpu().clone() for g in pair.current_grads()]

    pair.fill_grads = fill_and_capture
    pair.run()
    ps = [torch.nn.Parameter(torch.zeros(g.shape, dtype=g.dtype)) for g in captured["grads"]]
    for p, g in zip(ps, captured["grads"]):
        p.grad = g
    torch_norm = float(torch.nn.utils.clip_grad_norm_(ps, 1.0))
    assert torch_norm == math.inf and all(float(p.grad.abs().max()) == 0.0 for p in ps)
    assert float(pair.norms_gpu[1]) == math.inf and pair.outs[1]["norm"] == math.inf
    assert not any(o["skipped"] for o in pair.outs)
    check_pair(pair, label="norm_overflow")


def _same_with_nans(a: np.ndarray, b: np.ndarray) -> tuple[bool, float]:
    """NaN in the same places, then the largest relative difference of the
    other elements (equal values, infinities included, count as equal)."""
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False, math.inf
    keep = ~na & (a != b)
    if not keep.any():
        return True, 0.0
    if np.isinf(a[keep]).any() or np.isinf(b[keep]).any():
        return False, math.inf
    return True, maxrel(a[keep], b[keep])


def test_unscale_overflow_below_unit_scale_propagates_nan_like_torch():
    """fp32 params and grads, loss scale 2**-20: a scaled gradient of 1e33 is
    finite (no skip) but unscales to inf, the norm is inf, the coefficient 0,
    and that element's clipped gradient inf * 0 = NaN reaches AdamW, exactly as
    torch's CPU path does; every other element takes a zero-gradient step."""
    from oracle.torch_path import TorchReferencePath

    sc = dict(init_scale=2.0 ** -20, growth_factor=2.0, backoff_factor=0.5, growth_interval=1000)
    inject = {2: [(1, 17, 1e33)]}
    log("case: unscale overflow at scale 2**-20")
    pair = Pair(Case(shapes=SHAPES, steps=3, sigma=1e-3, chunk_elems=CHUNK, scaler=sc, inject=inject))
    init = [p.detach().cpu().numpy().copy() for p in pair.params]
    hp = [dict(betas=pair.case.betas, eps=pair.case.eps, weight_decay=pair.case.wd),
          dict(betas=pair.case.betas, eps=pair.case.eps, weight_decay=0.0)]
    ref = TorchReferencePath(init, pair.group_of, hp, scaler=sc, max_norm=1.0)
    torch_norms = []
    for s in range(1, 4):
        lr = mg.cosine_lr(s - 1, *pair.case.lr_sched)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        pair.oracle_step(s, lr)
        torch_norms.append(ref.step([g.detach().cpu().numpy() for g in pair.current_grads()], lr)["norm"])
        pair.gpu_step()
    torch.cuda.synchronize()
    assert not any(o["skipped"] for o in pair.outs)
    assert float(pair.norms_gpu[1]) == math.inf == pair.outs[1]["norm"] == torch_norms[1]
    nan_tensors = []
    for i in range(len(pair.params)):
        st = pair.gpu_state(i)
        tp, tm, tv, tstep = ref.state(i)
        assert st["step"] == pair.orc.steps[i] == tstep == 3.0
        for k, orc, tor in (("p", pair.orc.p[i], tp), ("m", pair.orc.m[i], tm), ("v", pair.orc.v[i], tv)):
            ok, r = _same_with_nans(st[k], orc.ravel())
            assert ok and r == 0.0, ("oracle", k, i, r)
            ok, r = _same_with_nans(st[k], tor.ravel())
            assert ok and r <= RTOL_STATE, ("torch", k, i, r)
        if np.isnan(st["p"]).any():
            nan_tensors.append((i, np.flatnonzero(np.isnan(st["p"])).tolist()))
    assert nan_tensors == [(1, [17])], nan_tensors
    log(f"[unscale_overflow] NaN only at {nan_tensors}, as in torch")


def test_zero_eps_with_zero_gradients_gives_nan_where_torch_does():
    """eps = 0 and a zero gradient on fresh state: the first step divides
    m = 0 by sqrt(v) / sqrt(bc2) + eps = 0 (adam.py:537-547), so torch's CPU
    path writes NaN into exactly those parameter elements; the GPU does the
    same, and every other element agrees with the oracle bit for bit and with
    torch within the state tolerance."""
    from oracle.torch_path import TorchReferencePath

    inject = {1: [(0, 5, 0.0), (1, 4098, 0.0), (4, 0, 0.0)]}
    log("case: eps 0 with zero gradients at step 1")
    pair = Pair(Case(shapes=SHAPES, steps=3, sigma=1e-3, eps=0.0, max_norm=None, chunk_elems=1024, inject=inject))
    init = [p.detach().cpu().numpy().copy() for p in pair.params]
    hp = [dict(betas=pair.case.betas, eps=0.0, weight_decay=pair.case.wd), dict(betas=pair.case.betas, eps=0.0,
                                                                                 weight_decay=0.0)]
    ref = TorchReferencePath(init, pair.group_of, hp, scaler=None, max_norm=None)
    zeros_at_step1 = None
    for s in range(1, 4):
        lr = mg.cosine_lr(s - 1, *pair.case.lr_sched)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        if s == 1:   # the injected zeros, plus any the generator itself produced
            zeros_at_step1 = [(i, np.flatnonzero(g.detach().cpu().numpy().ravel() == 0.0).tolist())
                              for i, g in enumerate(pair.current_grads())]
            zeros_at_step1 = [z for z in zeros_at_step1 if z[1]]
        pair.oracle_step(s, lr)
        ref.step([g.detach().cpu().numpy() for g in pair.current_grads()], lr)
        pair.gpu_step()
    torch.cuda.synchronize()
    nan_at = []
    for i in range(len(pair.params)):
        st = pair.gpu_state(i)
        tp, tm, tv, _ = ref.state(i)
        for k, orc, tor in (("p", pair.orc.p[i], tp), ("m", pair.orc.m[i], tm), ("v", pair.orc.v[i], tv)):
            ok, r = _same_with_nans(st[k], orc.ravel())
            assert ok and r == 0.0, ("oracle", k, i, r)
            ok, r = _same_with_nans(st[k], tor.ravel())
            assert ok and r <= RTOL_STATE, ("torch", k, i, r)
        if np.isnan(st["p"]).any():
            nan_at.append((i, np.flatnonzero(np.isnan(st["p"])).tolist()))
    assert nan_at == zeros_at_step1, (nan_at, zeros_at_step1)
    assert {(0, 5), (1, 4098), (4, 0)} <= {(i, k) for i, ks in nan_at for k in ks}


def test_extreme_gradient_magnitudes_without_clipping():
    """fp32 gradients whose squares overflow (1e20, 3e38) or underflow (1e-30)
    the fp32 range, no scaler and no clip: v becomes inf (the update divides
    by inf) or stays 0 (the denominator is eps); every element agrees with the
    oracle bit for bit (NaN as NaN) and with torch's CPU path within the
    state tolerance."""
    from oracle.torch_path import TorchReferencePath

    inject = {1: [(0, 3, 1e20), (1, 10, 3e38), (2, 7, -1e-30), (5, 100, 1e-30)],
              2: [(0, 3, -1e20), (3, 2, 3e38)]}
    log("case: extreme fp32 gradient magnitudes, no clip")
    pair = Pair(Case(shapes=SHAPES, steps=3, sigma=1e-3, max_norm=None, chunk_elems=1024, inject=inject))
    init = [p.detach().cpu().numpy().copy() for p in pair.params]
    hp = [dict(betas=pair.case.betas, eps=pair.case.eps, weight_decay=pair.case.wd),
          dict(betas=pair.case.betas, eps=pair.case.eps, weight_decay=0.0)]
    ref = TorchReferencePath(init, pair.group_of, hp, scaler=None, max_norm=None)
    for s in range(1, 4):
        lr = mg.cosine_lr(s - 1, *pair.case.lr_sched)
        mg.set_optimizer_lr(pair.opt, lr)
        pair.fill_grads(s)
        pair.oracle_step(s, lr)
        ref.step([g.detach().cpu().numpy() for g in pair.current_grads()], lr)
        pair.gpu_step()
    torch.cuda.synchronize()
    for i in range(len(pair.params)):
        st = pair.gpu_state(i)
        tp, tm, tv, _ = ref.state(i)
        for k, orc, tor in (("p", pair.orc.p[i], tp), ("m", pair.orc.m[i], tm), ("v", pair.orc.v[i], tv)):
            ok, r = _same_with_nans(st[k], orc.ravel())
            assert ok and r == 0.0, ("oracle", k, i, r)
            ok, r = _same_with_nans(st[k], tor.ravel())
            assert ok and r <= RTOL_STATE, ("torch", k, i, r)
    # the overflowed square keeps v at inf (beta2 * inf); the underflowed one left v finite
    assert np.isinf(pair.gpu_state(1)["v"][10]) and np.isfinite(pair.gpu_state(5)["v"][100])
