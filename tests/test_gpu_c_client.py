"""The library from a C program (tests/c_client/mgopt_client.c): include/mgopt.h
compiled as C99 and linked with the HIP runtime, no Python or torch in that
process.  Six steps over fp32/fp32, bf16-with-master/bf16 and fp32/fp16
tensors in two groups, with a NaN step; its norms, skip flags, scales,
trackers, step counts and final state against the oracle given the same
generated inputs, bit for bit."""

from __future__ import annotations

import math
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from tests._compare import RTOL_NORM, rel
from tests._gpu_harness import log

pytestmark = pytest.mark.gpu
BIN = Path(__file__).resolve().parent / "c_client" / "_build" / "mgopt_client"
NUMEL = (5000, 70000, 129)
PARAM = ("f32", "bf16", "f32")
GRAD = ("f32", "bf16", "f16")
GROUP = (0, 0, 1)


def test_c_program_steps_match_the_oracle(tmp_path):
    assert BIN.exists(), f"{BIN} is not built; run __graft_entry__.build()"
    out = tmp_path / "state.bin"
    log("case: C client, 6 steps, NaN at step 4")
    r = subprocess.run([str(BIN), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    data = out.read_bytes()
    pos = 0

    def take(dtype, n):
        nonlocal pos
        a = np.frombuffer(data, dtype=dtype, count=n, offset=pos)
        pos += a.nbytes
        return a

    per_step = []
    for _ in range(6):
        norm, found, scale = take(np.float32, 3)
        per_step.append((float(norm), float(found), float(scale), int(take(np.int32, 1)[0])))
    state = []
    for i, n in enumerate(NUMEL):
        p, m, v = take(np.float32, n), take(np.float32, n), take(np.float32, n)
        bits = take(np.uint16, n) if PARAM[i] == "bf16" else None
        state.append((p, m, v, bits))
    counts = take(np.float32, 3)
    assert pos == len(data)

    init = [O.round_to(O.synth(n, 1, i, O.synth_k(0.02)), PARAM[i]) for i, n in enumerate(NUMEL)]
    orc = O.OracleRun(init, list(GROUP), [dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1),
                                          dict(betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)],
                      scaler=dict(init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2),
                      max_norm=1.0)
    for s in range(1, 7):
        lr = 1e-3 * (0.5 + 0.1 * s)
        k = O.synth_k(1e-2 * orc.scale)
        grads = [O.synth_grad(n, 2, (s << 20) | i, k, GRAD[i]) for i, n in enumerate(NUMEL)]
        if s == 4:
            grads[2][-1] = math.nan
        o = orc.step(grads, lr)
        norm, found, scale, tracker = per_step[s - 1]
        assert (found != 0.0) == o["found_inf"] and scale == o["scale"] and tracker == o["tracker"], (s, per_step[s - 1], o)
        if math.isfinite(o["norm"]):
            assert rel(norm, o["norm"]) <= RTOL_NORM, (s, norm, o["norm"])
        else:
            assert math.isnan(norm) == math.isnan(o["norm"]), (s, norm, o["norm"])
    assert [s for s in range(1, 7) if per_step[s - 1][1] != 0.0] == [4]
    assert counts.tolist() == orc.steps == [5.0, 5.0, 5.0]
    for i, (p, m, v, bits) in enumerate(state):
        for got, ref in ((p, orc.p[i]), (m, orc.m[i]), (v, orc.v[i])):
            assert np.array_equal(got.view(np.uint32), ref.ravel().view(np.uint32)), i
        if bits is not None:
            assert np.array_equal(bits, O.to_bf16(orc.p[i].ravel())), i
    log(f"[c client] {r.stdout.strip()}; 6 steps bit-exact against the oracle, final scale {per_step[-1][2]}")
