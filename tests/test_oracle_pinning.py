"""Pins the CPU oracle (oracle/mgopt_oracle.c) before the GPU path is compared
against it.

Three kinds of evidence, none of which retypes the oracle's formulas:
  1. golden vectors written by torch 2.10.0 on the CPU (tests/golden/), i.e.
     the reference's own numerics for train.py:483-491;
  2. closed forms and invariants (first step from zero moments, zero
     gradient, skip invariance, exact norms, hand-computed schedules);
  3. planted mistakes: deliberately wrong AdamW variants must fail check 1.
"""

from __future__ import annotations

import hashlib
import json
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from tests._compare import RTOL_NORM, RTOL_STATE, exact_fraction, maxrel, rel

CASES = ["adamw_noclip", "adamw_clip", "adamw_noclipcall", "scaler_inf", "adamw_branches"]


def _digest(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _replay(d, adamw_fn=None, torch_norm=False):
    """Runs the oracle over a golden case's inputs; returns (run, per-step
    outputs).  torch_norm: clip with the norm torch computed at each step (its
    fp32 accumulation differs from the exact norm in the last bits), so that
    everything downstream of the norm can be compared bit for bit."""
    meta = json.loads(str(d["meta"]))
    sizes = [int(s) for s in d["sizes"]]
    params = [d[f"p0_{i}"] for i in range(len(sizes))]
    hparams = [dict(h, betas=tuple(h["betas"])) for h in meta["hparams"]]
    run = O.OracleRun(params, [int(g) for g in d["group_of"]], hparams, scaler=meta["scaler"], max_norm=meta["max_norm"])
    outs = []
    saved = O.adamw
    if adamw_fn is not None:
        O.adamw = adamw_fn
    try:
        for s in range(1, meta["steps"] + 1):
            scale = run.scale if meta["scaler"] else 1.0
            k = O.synth_k(meta["sigma"] * scale)
            grads = [O.synth(n, meta["grad_seed"], (s << 20) | i, k) for i, n in enumerate(sizes)]
            if s in meta["inf_at"]:
                grads[3][17] = np.inf
            if s in meta["nan_at"]:
                grads[4][4098] = np.nan
            assert _digest(grads) == str(d["grad_sha256"][s - 1]), "synthetic generator drifted from the fixture"
            lr = O.cosine_lr(s - 1, *meta["lr_sched"])
            assert lr == float(d["lrs"][s - 1])
            override = float(d["norms"][s - 1]) if torch_norm and meta["max_norm"] is not None else None
            outs.append(run.step(grads, lr, norm_override=override))
    finally:
        O.adamw = saved
    return run, outs


@pytest.mark.parametrize("case", CASES)
def test_oracle_norm_and_skips_match_torch_cpu(golden, case):
    d = golden(case)
    meta = json.loads(str(d["meta"]))
    run, outs = _replay(d)
    # norms: the oracle's exact (fp64) accumulation vs torch's fp32 one,
    # which is accurate to ~1e-7 on tensors this small
    for s, out in enumerate(outs):
        ref = float(d["norms"][s])
        if out["norm"] is None:
            assert math.isnan(ref)
        elif math.isfinite(ref):
            assert rel(out["norm"], ref) <= RTOL_NORM
        else:
            assert (math.isnan(ref) and math.isnan(out["norm"])) or out["norm"] == ref
    # skip decisions and the loss-scale trajectory: bit-exact
    if meta["scaler"]:
        assert [o["scale"] for o in outs] == [float(x) for x in d["scales"]]
        assert [o["tracker"] for o in outs] == [int(x) for x in d["trackers"]]
    for i in range(len(d["sizes"])):
        assert run.steps[i] == float(d[f"step_{i}"])


@pytest.mark.parametrize("case", CASES)
def test_oracle_update_matches_torch_cpu(golden, case):
    d = golden(case)
    run, _ = _replay(d, torch_norm=True)
    for i in range(len(d["sizes"])):
        assert run.steps[i] == float(d[f"step_{i}"])
        for name, mine in (("p", run.p[i]), ("m", run.m[i]), ("v", run.v[i])):
            ref = d[f"{name}_{i}"]
            assert maxrel(mine, ref) <= RTOL_STATE, (case, name, i, maxrel(mine, ref))
        # with the same clip coefficient the moments involve no square root,
        # so they agree with torch bit for bit
        assert exact_fraction(run.m[i], d[f"m_{i}"]) == 1.0
        assert exact_fraction(run.v[i], d[f"v_{i}"]) == 1.0
        # params differ only where torch's vectorised sqrt is not correctly rounded
        assert exact_fraction(run.p[i], d[f"p_{i}"]) >= 0.97


@pytest.mark.parametrize("mutant", [1, 2, 3, 4, 5, 6])
def test_planted_mistakes_fail_the_golden_check(golden, mutant):
    d = golden("adamw_noclip")

    def wrong(p, g, m, v, lr, b1, b2, eps, wd, step, maximize=False):
        O.adamw_mutant(p, g, m, v, lr, b1, b2, eps, wd, step, mutant)

    run, _ = _replay(d, adamw_fn=wrong)
    failures = 0
    for i in range(len(d["sizes"])):
        ok = all(maxrel(x, d[f"{n}_{i}"]) <= RTOL_STATE for n, x in (("p", run.p[i]), ("m", run.m[i]), ("v", run.v[i])))
        ok = ok and exact_fraction(run.m[i], d[f"m_{i}"]) == 1.0 and exact_fraction(run.v[i], d[f"v_{i}"]) == 1.0
        ok = ok and exact_fraction(run.p[i], d[f"p_{i}"]) >= 0.97
        failures += not ok
    assert failures > 0, f"mutant {mutant} passed the golden check"


# ---------------------------------------------------------------- element kernels
def test_dtype_rounding_matches_torch(golden):
    d = golden("elementwise")
    assert np.array_equal(O.to_bf16(d["x"]), d["bf16"])
    assert np.array_equal(O.to_f16(d["x"]), d["f16"])
    # widening is exact and inverts the rounding on representable values
    assert np.array_equal(O.to_bf16(O.from_bf16(d["bf16"])), d["bf16"])
    f16 = d["f16"]
    finite = (f16 & 0x7C00) != 0x7C00
    assert np.array_equal(O.to_f16(O.from_f16(f16))[finite], f16[finite])


def test_unscale_matches_torch(golden):
    d = golden("elementwise")
    for k, inv in enumerate(d["unscale_inv"]):
        for j in range(3):
            out, found = O.unscale(d["unscale_in"][j], float(inv))
            ref = d["unscale_out"][k][j]
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)) or np.array_equal(out, ref, equal_nan=True)
            assert float(found) == float(d["unscale_found"][k][j])


def test_clip_coefficient_matches_torch(golden):
    d = golden("elementwise")
    for r, mx in enumerate(d["clip_max"]):
        for c, n in enumerate(d["clip_norms"]):
            mine = O.clip_coef(float(n), float(mx))
            ref = float(d["clip_coefs"][r][c])
            assert (math.isnan(mine) and math.isnan(ref)) or np.float32(mine) == np.float32(ref), (n, mx, mine, ref)


def test_scaler_state_machine_matches_torch(golden):
    d = golden("elementwise")
    for k, (scale0, growth, backoff, interval) in enumerate(d["scaler_params"]):
        scale, tracker = float(np.float32(scale0)), 0
        for j, fi in enumerate(d["scaler_found"][k]):
            scale, tracker = O.scaler_update(scale, tracker, float(fi), float(growth), float(backoff), int(interval))
            assert np.float32(scale) == d["scaler_traj_scale"][k][j]
            assert tracker == d["scaler_traj_tracker"][k][j]


# ------------------------------------------------------------------ closed forms
def _one_step(p, g, lr=3e-4, wd=0.1, b1=0.9, b2=0.95, eps=1e-8):
    p, g = np.array(p, np.float32), np.array(g, np.float32)
    m, v = np.zeros_like(p), np.zeros_like(p)
    O.adamw(p, g, m, v, lr, b1, b2, eps, wd, 1.0)
    return p, m, v


def test_first_step_is_signed_lr():
    # t = 1 from zero moments: m = 0.1 g, v = 0.05 g^2; bias correction turns
    # them into g and g^2, so p moves by -lr * g / (|g| + eps) ~ -lr * sign(g).
    rng = np.random.RandomState(0)
    p0 = (rng.randn(5000) * 0.02).astype(np.float32)
    g = (rng.randn(5000) * 1e-2).astype(np.float32)
    p, m, v = _one_step(p0, g)
    g64 = g.astype(np.float64)
    expected = p0.astype(np.float64) * (1 - 3e-4 * 0.1) - 3e-4 * g64 / (np.abs(g64) + 1e-8)
    np.testing.assert_allclose(p, expected, rtol=0, atol=1e-8)  # a few ulps of |p| ~ 0.02
    np.testing.assert_allclose(m, 0.1 * g.astype(np.float64), rtol=2e-7)
    np.testing.assert_allclose(v, 0.05 * g.astype(np.float64) ** 2, rtol=3e-7)


def test_zero_gradient_only_decays():
    p0 = np.linspace(-1, 1, 101, dtype=np.float32)
    p, m, v = _one_step(p0, np.zeros(101, np.float32))
    assert np.array_equal(p, p0 * np.float32(1 - 3e-4 * 0.1))
    assert not m.any() and not v.any()
    p, _, _ = _one_step(p0, np.zeros(101, np.float32), wd=0.0)
    assert np.array_equal(p, p0)


def test_skipped_step_leaves_state_bitwise():
    params = [np.linspace(-0.5, 0.5, 1000, dtype=np.float32)]
    run = O.OracleRun(params, [0], [dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)],
                      scaler=dict(init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2),
                      max_norm=1.0)
    g = np.full(1000, 3.0, np.float32)
    run.step([g], 1e-3)
    before = (run.p[0].copy(), run.m[0].copy(), run.v[0].copy(), list(run.steps))
    g[999] = -np.inf
    out = run.step([g], 1e-3)
    assert out["skipped"] and out["found_inf"] and out["scale"] == 512.0 and out["tracker"] == 0
    assert np.array_equal(run.p[0], before[0]) and np.array_equal(run.m[0], before[1])
    assert np.array_equal(run.v[0], before[2]) and run.steps == before[3]


def test_bias_corrections_closed_form():
    bc1, bc2s = O.bias_corrections(0.9, 0.95, 1.0)
    assert bc1 == 1 - 0.9 and bc2s == (1 - 0.95) ** 0.5
    bc1, bc2s = O.bias_corrections(0.9, 0.999, 10.0)
    assert rel(bc1, 1 - 0.9**10) < 1e-15 and rel(bc2s, math.sqrt(1 - 0.999**10)) < 1e-15


def test_norm_is_the_correctly_rounded_exact_norm():
    rng = np.random.RandomState(3)
    for trial in range(20):
        grads = [(rng.randn(n) * 10.0 ** rng.uniform(-4, 2)).astype(np.float32) for n in rng.randint(1, 3000, 4)]
        exact = sum(Fraction(float(x)) ** 2 for g in grads for x in g)
        # correctly rounded sqrt of the exact rational, to float32
        s = float(exact)
        r = math.sqrt(s)
        cand = [np.nextafter(np.float32(r), np.float32(-np.inf)), np.float32(r), np.nextafter(np.float32(r), np.float32(np.inf))]
        best = min(cand, key=lambda c: abs(Fraction(float(c)) ** 2 - exact))
        assert np.float32(O.norm_from_sumsq(O.total_sumsq(grads))) == best


def test_norm_special_values():
    assert O.norm_from_sumsq(O.total_sumsq([np.array([1.0, np.inf], np.float32)])) == math.inf
    assert math.isnan(O.norm_from_sumsq(O.total_sumsq([np.array([np.inf], np.float32), np.array([np.nan], np.float32)])))
    # squares beyond the fp32 range overflow like torch's fp32 accumulation
    assert O.norm_from_sumsq(O.total_sumsq([np.array([3e19, 3e19], np.float32)])) == math.inf
    assert O.norm_from_sumsq(0.0) == 0.0
    assert O.norm_from_sumsq(O.total_sumsq([np.array([3.0, 4.0], np.float32)])) == 5.0


def test_cosine_lr_closed_form(mg):
    base, mn, w, mx = 3e-4, 3e-5, 10, 100
    assert mg.cosine_lr(0, base, mn, w, mx) == base / 10
    assert mg.cosine_lr(w - 1, base, mn, w, mx) == base
    assert mg.cosine_lr(w, base, mn, w, mx) == base          # cos(0) = 1
    assert mg.cosine_lr(55, base, mn, w, mx) == pytest.approx((base + mn) / 2, rel=1e-15)
    assert mg.cosine_lr(mx, base, mn, w, mx) == mn and mg.cosine_lr(10**6, base, mn, w, mx) == mn
    assert mg.cosine_lr(0, base, mn, 0, mx) == base           # no warm-up
    assert mg.cosine_lr(5, base, mn, 10, 5) == base * 6 / 10  # warm-up is tested before max_steps
    for s in range(0, 130):
        assert mg.cosine_lr(s, base, mn, w, mx) == O.cosine_lr(s, base, mn, w, mx)


def test_scaler_trajectory_closed_form():
    # init 65536, growth 2 every 2000 good steps, backoff 0.5; inf at 17 and 53
    scale, tracker, traj = 65536.0, 0, []
    for s in range(1, 201):
        scale, tracker = O.scaler_update(scale, tracker, 1.0 if s in (17, 53) else 0.0, 2.0, 0.5, 2000)
        traj.append(scale)
    assert traj[15] == 65536.0 and traj[16] == 32768.0 and traj[51] == 32768.0 and traj[52] == 16384.0
    assert traj[-1] == 16384.0 and tracker == 200 - 53


def test_synthetic_generator_statistics():
    x = O.synth(1_000_000, 9, 3, O.synth_k(1e-3)).astype(np.float64)
    assert abs(x.mean()) < 5e-6 and abs(x.std() / 1e-3 - 1) < 5e-3
    assert np.abs(x).max() <= 1e-3 * math.sqrt(3) * 2 + 1e-12
    t = O.synth(1_000_000, 9, 3, O.synth_k(1e-3), tail_every=1000, tail_mult=100.0)
    frac = np.mean(np.abs(t) > 1e-2)
    assert 0.0005 < frac < 0.0015


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_host_rebuilt_gradients_match_the_stored_path(dtype):
    """The full-size tests rebuild gradients on the host from the generator
    instead of copying them back: synth_grad equals the generator's values
    rounded to the gradient dtype (what mgopt_synth_fill stores), and
    synth_grads_sumsq equals grads_sumsq over those stored values, pieces and
    combination order included -- with the heavy tail, unscaled and not."""
    n, k = 3_000_001, O.synth_k(1e-2 * 1024.0)
    stored = O.round_to(O.synth(n, 2, 77, k, 1000, 100.0), dtype)
    rebuilt = O.synth_grad(n, 2, 77, k, dtype, 1000, 100.0, piece=1 << 20)
    assert np.array_equal(rebuilt.view(np.uint32), stored.view(np.uint32))
    raw = stored if dtype == "f32" else (O.to_f16(stored) if dtype == "f16" else O.to_bf16(stored))
    for unscale in (False, True):
        want = O.grads_sumsq([(raw, dtype)], inv=1 / 1024.0, unscale=unscale, piece=1 << 20)
        got = O.synth_grads_sumsq([(n, 2, 77, k, dtype, 1000, 100.0)], inv=1 / 1024.0, unscale=unscale,
                                  piece=1 << 20)
        assert got == want


def test_parallel_pieces_are_the_serial_arithmetic():
    """adamw_parallel, unscale_parallel and scale_parallel split the
    element-wise arithmetic into pieces run in threads: same bits as one
    serial call, found_inf included (an inf in the last piece only)."""
    rng = np.random.default_rng(7)
    n = 3 * O.PIECE + 12345
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    g[-3] = np.inf
    u1, f1 = O.unscale(g, np.float32(1 / 512.0))
    u2, f2 = O.unscale_parallel(g, np.float32(1 / 512.0))
    assert f1 and f2 and np.array_equal(u1.view(np.uint32), u2.view(np.uint32))
    g[-3] = 0.5
    a, b = g.copy(), g.copy()
    O.scale_(a, np.float32(0.37))
    O.scale_parallel(b, np.float32(0.37))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    p = rng.standard_normal(n).astype(np.float32)
    s1 = [p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)]
    s2 = [x.copy() for x in s1]
    for step in (1, 2, 3):
        O.adamw(s1[0], g, s1[1], s1[2], 1e-3, 0.9, 0.95, 1e-8, 0.1, step)
        O.adamw_parallel(s2[0], g, s2[1], s2[2], 1e-3, 0.9, 0.95, 1e-8, 0.1, step)
    for x, y in zip(s1, s2):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("unscale,clip,maximize,wd", [(True, True, False, 0.1), (False, True, False, 0.0),
                                                      (True, False, True, 0.1), (False, False, False, 0.1)])
def test_fused_tensor_step_is_the_three_separate_steps(unscale, clip, maximize, wd):
    """unscale_clip_adamw (one pass per tensor, used when the totals over all
    gradients are known in advance) against unscale(), scale_() and adamw()
    in turn: same bits for p, m and v over three steps, on a length that is
    no multiple of its internal block and with zeros, subnormals, huge
    values and a NaN among the gradients; and unscale_clip_adamw_many's
    pieces equal one call."""
    rng = np.random.default_rng(11)
    n = 3 * 2048 + 77
    g = (rng.standard_normal(n) * 3e2).astype(np.float32)
    g[:5] = [0.0, -0.0, 1e-42, -3e38, np.nan]
    inv, coef = np.float32(1 / 1024.0), np.float32(0.0173)
    p0 = rng.standard_normal(n).astype(np.float32)
    ref = [p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)]
    got = [x.copy() for x in ref]
    many = [x.copy() for x in ref]
    for step in (1, 2, 3):
        u = O.unscale(g, inv)[0] if unscale else g.copy()
        if clip:
            O.scale_(u, coef)
        O.adamw(ref[0], u, ref[1], ref[2], 3e-4, 0.9, 0.95, 1e-8, wd, step, maximize)
        O.unscale_clip_adamw(g, got[0], got[1], got[2], inv, unscale, coef if clip else None, 3e-4, 0.9, 0.95, 1e-8,
                             wd, step, maximize)
        kw = dict(inv=inv, unscale=unscale, coef=coef if clip else None, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                  wd=wd, step=step, maximize=maximize)
        O.unscale_clip_adamw_many([(g, many[0], many[1], many[2], kw)], piece=1000)
    for a, b, c in zip(ref, got, many):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


def test_oracle_step_given_totals_matches_the_plain_step():
    """OracleRun.step with the totals over every gradient given (the
    full-size tests' form: fused per-tensor update, tensors in parallel) and
    without (unscale, norm, clip and AdamW as separate passes): same norms,
    skip decisions, scales and bits over 12 steps with an inf at step 5."""
    rng = np.random.default_rng(5)
    sizes = [5000, 1, 300, 70000, 4097]
    init = [rng.standard_normal(n).astype(np.float32) * 0.02 for n in sizes]
    hp = [dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1), dict(betas=(0.8, 0.99), eps=1e-7, weight_decay=0.0)]
    sc = dict(init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=3)
    group_of = [0, 1, 0, 0, 1]
    a = O.OracleRun(init, group_of, hp, scaler=sc, max_norm=1.0)
    b = O.OracleRun(init, group_of, hp, scaler=sc, max_norm=1.0)
    for s in range(1, 13):
        grads = [(rng.standard_normal(n) * 0.3 * a.scale).astype(np.float32) for n in sizes]
        if s == 5:
            grads[3][9] = np.inf
        oa = a.step(grads, 1e-3)
        tot = O.grads_sumsq([(g, "f32") for g in grads], inv=O.inv_scale(b.scale), unscale=True)
        ob = b.step(grads, 1e-3, totals=tot)
        assert oa["skipped"] == ob["skipped"] == (s == 5)
        assert oa["scale"] == ob["scale"] and oa["tracker"] == ob["tracker"]
        assert oa["norm"] == ob["norm"] or (math.isinf(oa["norm"]) and math.isinf(ob["norm"]))
    for i in range(len(sizes)):
        assert a.steps[i] == b.steps[i] == 11
        for x, y in ((a.p[i], b.p[i]), (a.m[i], b.m[i]), (a.v[i], b.v[i])):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
