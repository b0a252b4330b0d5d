"""Python face of the CPU oracle (mgopt_oracle.c).  TEST INFRASTRUCTURE ONLY:
imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
as the reference results the GPU path is compared against; never by the
product package.

OracleRun restates one iteration of the reference's training loop
(train.py:483-491) over numpy float32 arrays: GradScaler.unscale_, then
clip_grad_norm_, then GradScaler.step (AdamW, skipped on found_inf), then
GradScaler.update, calling the C restatement for every arithmetic step.
"""

from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib: ctypes.CDLL | None = None
_F = ctypes.POINTER(ctypes.c_float)
_U16 = ctypes.POINTER(ctypes.c_uint16)
_D = ctypes.POINTER(ctypes.c_double)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True, capture_output=True, text=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        i64, u64, dbl, i32 = ctypes.c_int64, ctypes.c_uint64, ctypes.c_double, ctypes.c_int32
        sig = {
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_bf16_array": (None, [_F, _U16, i64]),
            "orc_bf16_to_f32_array": (None, [_U16, _F, i64]),
            "orc_f32_to_f16_array": (None, [_F, _U16, i64]),
            "orc_f16_to_f32_array": (None, [_U16, _F, i64]),
            "orc_synth_key": (u64, [u64, u64]),
            "orc_synth_value": (ctypes.c_float, [u64, u64, dbl, u64, dbl]),
            "orc_synth_fill": (None, [_F, i64, u64, u64, dbl, u64, dbl]),
            "orc_inv_scale": (ctypes.c_float, [ctypes.c_float]),
            "orc_unscale": (None, [_F, _F, i64, ctypes.c_float, _F]),
            "orc_sumsq_acc": (None, [_F, i64, _D]),
            "orc_sumsq": (dbl, [_F, i64]),
            "orc_norm_from_sumsq": (ctypes.c_float, [dbl]),
            "orc_clip_coef": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "orc_scale": (None, [_F, i64, ctypes.c_float]),
            "orc_bias_corrections": (None, [dbl, dbl, dbl, _D]),
            "orc_adamw": (None, [_F, _F, _F, _F, i64, dbl, dbl, dbl, dbl, dbl, dbl, ctypes.c_int]),
            "orc_adamw_mutant": (None, [_F, _F, _F, _F, i64, dbl, dbl, dbl, dbl, dbl, dbl, ctypes.c_int]),
            "orc_unscale_clip_adamw": (None, [_F, _F, _F, _F, i64, ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                              ctypes.c_int, dbl, dbl, dbl, dbl, dbl, dbl, ctypes.c_int]),
            "orc_scaler_update": (None, [_F, ctypes.POINTER(i32), ctypes.c_float, dbl, dbl, i32]),
            "orc_cosine_lr": (dbl, [i64, dbl, dbl, i64, i64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _u16(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(_U16)


# --------------------------------------------------------------- conversions
def _convert(fn, x: np.ndarray, out: np.ndarray) -> None:
    """fn(in, out, n) over x, in parallel pieces when x is large."""
    fx, fo = x.reshape(-1), out.reshape(-1)
    if fx.size <= PIECE:
        fn(_fp(fx), _u16(fo), fx.size)
        return
    list(pool().map(lambda s: fn(_fp(fx[s:s + PIECE]), _u16(fo[s:s + PIECE]), min(PIECE, fx.size - s)),
                    range(0, fx.size, PIECE)))


def to_bf16(x: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    """bf16 bit patterns of x (round to nearest even), into `out` when given."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16) if out is None else out.reshape(x.shape)
    _convert(lib().orc_f32_to_bf16_array, x, out)
    return out


def from_bf16(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_array(_u16(h), _fp(out), h.size)
    return out


def to_f16(x: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    """fp16 bit patterns of x (round to nearest even), into `out` when given."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16) if out is None else out.reshape(x.shape)
    _convert(lib().orc_f32_to_f16_array, x, out)
    return out


def from_f16(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_u16(h), _fp(out), h.size)
    return out


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values after a round trip through dtype ('f32', 'f16', 'bf16')."""
    if dtype == "f32":
        return np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f16":
        return from_f16(to_f16(x))
    if dtype == "bf16":
        return from_bf16(to_bf16(x))
    raise ValueError(dtype)


# ------------------------------------------------------------ synthetic data
def synth_k(sigma: float) -> float:
    """Multiplier that gives the Irwin-Hall(4) generator standard deviation sigma."""
    return sigma * math.sqrt(3.0) / 65536.0


def synth(n: int, seed: int, stream: int, k: float, tail_every: int = 0, tail_mult: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_fill(_fp(out), n, seed, stream, k, tail_every, tail_mult)
    return out


# ---------------------------------------------------------------- arithmetic
def inv_scale(scale: float) -> float:
    return lib().orc_inv_scale(scale)


def unscale(g: np.ndarray, inv: float) -> tuple[np.ndarray, bool]:
    out = np.empty_like(g)
    found = np.zeros(1, np.float32)
    lib().orc_unscale(_fp(g), _fp(out), g.size, inv, _fp(found))
    return out, bool(found[0] != 0.0)


def sumsq(g: np.ndarray) -> float:
    return lib().orc_sumsq(_fp(np.ascontiguousarray(g, np.float32)), g.size)


def total_sumsq(grads: list[np.ndarray]) -> float:
    acc = np.zeros(2, np.float64)
    for g in grads:
        lib().orc_sumsq_acc(_fp(np.ascontiguousarray(g, np.float32)), g.size, acc.ctypes.data_as(_D))
    return float(acc[0] + acc[1])


_DTYPE_CODE = {np.dtype(np.float32): 0, "f16": 1, "bf16": 2}


def grads_sumsq(grads, inv: float = 1.0, unscale: bool = False, threads: int = 16,
                piece: int = 1 << 24) -> tuple[float, bool]:
    """Total sum of squares (after the unscale) and the non-finite flag over
    gradients given as (array, dtype) pairs, dtype in 'f32', 'f16', 'bf16'
    (f16/bf16 arrays hold raw uint16 bits).  Pieces of at most `piece`
    elements are summed in parallel threads (ctypes releases the GIL) and
    combined in a fixed order, so the result does not depend on `threads`."""
    from concurrent.futures import ThreadPoolExecutor

    L = lib()
    L.orc_grad_sumsq_acc.restype = None
    L.orc_grad_sumsq_acc.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_int, _D, _F]
    jobs = []
    for arr, dt in grads:
        arr = np.ascontiguousarray(arr).ravel()
        code = {"f32": 0, "f16": 1, "bf16": 2}[dt]
        for s in range(0, arr.size, piece):
            jobs.append((arr, code, s, min(arr.size, s + piece)))

    def run(job):
        arr, code, s, e = job
        acc = np.zeros(2, np.float64)
        found = np.zeros(1, np.float32)
        L.orc_grad_sumsq_acc(arr[s:].ctypes.data, code, e - s, inv, int(unscale), acc.ctypes.data_as(_D),
                             found.ctypes.data_as(_F))
        return acc, bool(found[0])

    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        return _combine(list(ex.map(run, jobs)))


def _combine(results) -> tuple[float, bool]:
    """Folds per-piece (compensated sum, correction) pairs and non-finite
    flags into one total, in the given (fixed) order."""
    acc = np.zeros(2, np.float64)
    found = False
    for a, f in results:
        found |= f
        for y in (a[0], a[1]):
            t = acc[0] + y
            if not np.isfinite(t):
                acc[0], acc[1] = t, 0.0
                continue
            acc[1] += (acc[0] - t) + y if abs(acc[0]) >= abs(y) else (y - t) + acc[0]
            acc[0] = t
    return float(acc[0] + acc[1]), found


_GRAD_DTYPE = {"f32": 0, "f16": 1, "bf16": 2}


def synth_grad(n: int, seed: int, stream: int, k: float, dtype: str = "f32", tail_every: int = 0,
               tail_mult: float = 1.0, threads: int = 16, piece: int = 1 << 22,
               out: np.ndarray | None = None) -> np.ndarray:
    """The synthetic gradient the GPU generator writes into a `dtype` tensor
    (mgopt_synth_fill), as fp32 values, generated in parallel pieces; written
    into `out` (float32, at least n elements; its first n are returned) when
    given, so that a caller can reuse one buffer across steps."""
    from concurrent.futures import ThreadPoolExecutor

    L = lib()
    L.orc_synth_grad.restype = None
    L.orc_synth_grad.argtypes = [_F, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double,
                                 ctypes.c_uint64, ctypes.c_double, ctypes.c_int]
    if out is None:
        out = np.empty(n, np.float32)
    else:
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size >= n
        out = out[:n]
    code = _GRAD_DTYPE[dtype]

    def run(s):
        e = min(n, s + piece)
        L.orc_synth_grad(out[s:].ctypes.data_as(_F), s, e, seed, stream, k, tail_every, tail_mult, code)

    if n <= piece:
        if n:
            run(0)
        return out
    if threads == THREADS:
        list(pool().map(run, range(0, n, piece)))
    else:
        with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
            list(ex.map(run, range(0, n, piece)))
    return out


def synth_grads_sumsq(specs, inv: float = 1.0, unscale: bool = False, threads: int = 16,
                      piece: int = 1 << 24) -> tuple[float, bool]:
    """grads_sumsq over synthetic gradients generated on the fly: specs is a
    list of (n, seed, stream, k, dtype, tail_every, tail_mult), one per tensor.
    The pieces and their combination order are those grads_sumsq uses for
    arrays of the same sizes, so the two give the same total."""
    from concurrent.futures import ThreadPoolExecutor

    L = lib()
    L.orc_synth_grad_sumsq_acc.restype = None
    L.orc_synth_grad_sumsq_acc.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64,
                                           ctypes.c_double, ctypes.c_uint64, ctypes.c_double, ctypes.c_int,
                                           ctypes.c_float, ctypes.c_int, _D, _F]
    jobs = []
    for n, seed, stream, k, dt, tail_every, tail_mult in specs:
        for s in range(0, n, piece):
            jobs.append((s, min(n, s + piece), seed, stream, k, _GRAD_DTYPE[dt], tail_every, tail_mult))

    def run(job):
        s, e, seed, stream, k, code, tail_every, tail_mult = job
        acc = np.zeros(2, np.float64)
        found = np.zeros(1, np.float32)
        L.orc_synth_grad_sumsq_acc(s, e, seed, stream, k, tail_every, tail_mult, code, inv, int(unscale),
                                   acc.ctypes.data_as(_D), found.ctypes.data_as(_F))
        return acc, bool(found[0])

    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        return _combine(list(ex.map(run, jobs)))


def norm_from_sumsq(s: float) -> float:
    return lib().orc_norm_from_sumsq(s)


def clip_coef(norm: float, max_norm: float) -> float:
    return lib().orc_clip_coef(norm, max_norm)


def scale_(g: np.ndarray, coef: float) -> None:
    lib().orc_scale(_fp(g), g.size, coef)


def bias_corrections(beta1: float, beta2: float, step: float) -> tuple[float, float]:
    out = np.zeros(2, np.float64)
    lib().orc_bias_corrections(beta1, beta2, step, out.ctypes.data_as(_D))
    return float(out[0]), float(out[1])


def adamw(p, g, m, v, lr, beta1, beta2, eps, wd, step, maximize=False) -> None:
    """In-place AdamW update of one tensor (p, m, v float32, step = new count)."""
    lib().orc_adamw(_fp(p), _fp(g), _fp(m), _fp(v), p.size, lr, beta1, beta2, eps, wd, float(step), int(maximize))


PIECE = 1 << 22          # elements per piece of the parallel element-wise helpers
THREADS = 16             # threads of the parallel helpers (the host cores available per GPU)
_POOL = None


def pool():
    """The module's persistent pool of THREADS worker threads (the C calls
    release the GIL), shared by the parallel helpers that run often."""
    global _POOL
    if _POOL is None:
        from concurrent.futures import ThreadPoolExecutor

        _POOL = ThreadPoolExecutor(max_workers=THREADS)
    return _POOL


def unscale_clip_adamw(g, p, m, v, inv, unscale, coef, lr, beta1, beta2, eps, wd, step, maximize=False) -> None:
    """One tensor's update in an iteration whose step is taken, in place on
    p, m, v: unscale by inv (when unscale), scale by coef (when coef is not
    None), then AdamW with the new step count.  Bit for bit what unscale(),
    scale_() and adamw() give in turn (pinned by test_oracle_pinning)."""
    lib().orc_unscale_clip_adamw(_fp(g), _fp(p), _fp(m), _fp(v), p.size, inv, int(unscale),
                                 1.0 if coef is None else coef, int(coef is not None), lr, beta1, beta2, eps, wd,
                                 float(step), int(maximize))


def unscale_clip_adamw_many(jobs, piece: int = PIECE) -> None:
    """unscale_clip_adamw over many tensors on the module's thread pool:
    jobs holds (g, p, m, v, kwargs) per tensor; tensors above `piece` elements
    are split into pieces (the update is element-wise, so the bits do not
    depend on the split)."""
    tasks = []
    for g, p, m, v, kw in jobs:
        fg, fp, fm, fv = (a.reshape(-1) for a in (g, p, m, v))
        for s in range(0, fp.size, piece):
            e = min(fp.size, s + piece)
            tasks.append((fg[s:e], fp[s:e], fm[s:e], fv[s:e], kw))
    if len(tasks) == 1:
        g, p, m, v, kw = tasks[0]
        unscale_clip_adamw(g, p, m, v, **kw)
        return
    list(pool().map(lambda t: unscale_clip_adamw(t[0], t[1], t[2], t[3], **t[4]), tasks))


def _pieces(n: int, fn, threads: int = THREADS, piece: int = PIECE) -> None:
    """fn(s, e) over [0, n) in pieces of `piece` elements, in parallel threads
    (the C calls release the GIL); serial when n fits one piece."""
    if n <= piece:
        fn(0, n)
        return
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        list(ex.map(lambda s: fn(s, min(n, s + piece)), range(0, n, piece)))


def adamw_parallel(p, g, m, v, lr, beta1, beta2, eps, wd, step, maximize=False, threads: int = THREADS,
                   piece: int = PIECE) -> None:
    """adamw() over pieces in parallel threads: the update is element-wise, so
    the result is the same bits.  Each piece goes through this module's
    adamw(), so a test that replaces it replaces every piece."""
    fp, fg, fm, fv = (a.reshape(-1) for a in (p, g, m, v))
    _pieces(fp.size, lambda s, e: adamw(fp[s:e], fg[s:e], fm[s:e], fv[s:e], lr, beta1, beta2, eps, wd, step, maximize),
            threads, piece)


def unscale_parallel(g: np.ndarray, inv: float) -> tuple[np.ndarray, bool]:
    """unscale() in parallel pieces (same bits; found is the OR of the pieces')."""
    out = np.empty_like(g)
    flags = np.zeros(-(-g.size // PIECE) if g.size > PIECE else 1, np.float32)
    L = lib()

    def run(s, e):
        k = s // PIECE if g.size > PIECE else 0
        L.orc_unscale(_fp(g[s:e]), _fp(out[s:e]), e - s, inv, flags[k:].ctypes.data_as(_F))

    _pieces(g.size, run)
    return out, bool((flags != 0.0).any())


def scale_parallel(g: np.ndarray, coef: float) -> None:
    L = lib()
    _pieces(g.size, lambda s, e: L.orc_scale(_fp(g[s:e]), e - s, coef))


def adamw_mutant(p, g, m, v, lr, beta1, beta2, eps, wd, step, mutant: int) -> None:
    lib().orc_adamw_mutant(_fp(p), _fp(g), _fp(m), _fp(v), p.size, lr, beta1, beta2, eps, wd, float(step), mutant)


def scaler_update(scale: float, tracker: int, found_inf: float, growth: float, backoff: float,
                  interval: int) -> tuple[float, int]:
    s = ctypes.c_float(scale)
    t = ctypes.c_int32(tracker)
    lib().orc_scaler_update(ctypes.byref(s), ctypes.byref(t), found_inf, growth, backoff, interval)
    return s.value, t.value


def cosine_lr(step: int, base_lr: float, min_lr: float, warmup: int, max_steps: int) -> float:
    return lib().orc_cosine_lr(step, base_lr, min_lr, warmup, max_steps)


# ------------------------------------------------------------ whole iteration
class OracleRun:
    """One optimizer over a list of float32 numpy tensors, stepped as
    train.py:483-491 steps torch's.

    params:    fp32 arrays (the fp32 master when lowp is set)
    group_of:  group index of each tensor
    hparams:   per group dict(betas, eps, weight_decay, maximize=False)
    scaler:    None (disabled) or dict(init_scale, growth_factor,
               backoff_factor, growth_interval)
    max_norm:  None (no clip_grad_norm_ call) or the clip threshold
    lowp:      None, 'bf16' or 'f16': the model copy rounded from the master
    """

    def __init__(self, params, group_of, hparams, scaler=None, max_norm=None, lowp=None):
        self.p = [np.array(x, dtype=np.float32, copy=True) for x in params]
        self.m = [np.zeros_like(x) for x in self.p]
        self.v = [np.zeros_like(x) for x in self.p]
        self.steps = [0.0] * len(self.p)
        self.group_of = list(group_of)
        self.hparams = hparams
        self.max_norm = max_norm
        self.lowp = lowp
        self.scaler = dict(scaler) if scaler else None
        if self.scaler:
            self.scale = float(np.float32(self.scaler["init_scale"]))
            self.tracker = 0

    def lowp_params(self) -> list[np.ndarray]:
        return [round_to(x, self.lowp) for x in self.p] if self.lowp else self.p

    def load(self, i: int, p: np.ndarray, m: np.ndarray, v: np.ndarray, step: float) -> None:
        """Takes over tensor i's state from elsewhere (the GPU's, before a
        step): the arrays are used in place, not copied."""
        for a in (p, m, v):
            assert a.dtype == np.float32 and a.flags.c_contiguous
        self.p[i], self.m[i], self.v[i], self.steps[i] = p, m, v, float(step)

    def unload(self, i: int) -> None:
        """Forgets tensor i's state (its arrays are released)."""
        empty = np.zeros(0, np.float32)
        self.p[i], self.m[i], self.v[i] = empty, empty, empty

    def step(self, grads: list[np.ndarray | None], lr: float | list[float], subset=None,
             norm_override: float | None = None, totals: tuple[float, bool] | None = None) -> dict:
        """grads: fp32 values as the GPU reads them (scaled, when the scaler is
        on).  subset: indices whose AdamW update is computed (all when None).
        norm_override: clip with this total norm instead of the oracle's own
        (used to compare the rest of the arithmetic against a reference whose
        norm differs).  totals: (sum of squares of the unscaled grads,
        non-finite flag) over every grad, computed elsewhere (grads_sumsq);
        then grads need only hold the tensors of `subset`, the others None.
        A sum of squares of None leaves the norm unverified (out["norm"] is
        None): the clip then uses norm_override, which must be given."""
        lrs = lr if isinstance(lr, list) else [lr] * len(self.hparams)
        if totals is not None:
            return self._step_from_totals(grads, lrs, subset, norm_override, totals)
        found = False
        work = []
        inv = inv_scale(self.scale) if self.scaler else 1.0
        for g in grads:
            if g is None:
                work.append(None)
            elif self.scaler:
                u, f = unscale_parallel(g, inv)
                found |= f
                work.append(u)
            else:
                work.append(np.array(g, np.float32, copy=True))
        present = [w for w in work if w is not None]
        norm = None
        if self.max_norm is not None and present:
            norm = norm_from_sumsq(total_sumsq(present))
            coef = clip_coef(norm if norm_override is None else norm_override, self.max_norm)
            for w in present:
                scale_parallel(w, coef)
        skipped = bool(self.scaler) and found
        if not skipped:
            idx = range(len(self.p)) if subset is None else subset
            for i in idx:
                if work[i] is None:
                    continue
                h = self.hparams[self.group_of[i]]
                self.steps[i] += 1.0
                adamw_parallel(self.p[i], work[i], self.m[i], self.v[i], lrs[self.group_of[i]], h["betas"][0],
                               h["betas"][1], h["eps"], h["weight_decay"], self.steps[i], h.get("maximize", False))
        return self._finish(norm, found, skipped)

    def _step_from_totals(self, grads, lrs, subset, norm_override, totals) -> dict:
        """step() given the totals over every gradient: the found flag and the
        clip coefficient are known before any tensor is touched, so each
        tensor of the subset is unscaled, clipped and updated in one pass
        (unscale_clip_adamw, bit for bit the separate steps), the tensors in
        parallel."""
        sumsq, found = totals[0], bool(totals[1]) and bool(self.scaler)
        inv = inv_scale(self.scale) if self.scaler else 1.0
        norm, coef = None, None
        if self.max_norm is not None:
            if sumsq is None:
                if norm_override is None:
                    raise ValueError("an unverified norm needs norm_override")
            else:
                norm = norm_from_sumsq(sumsq)
            coef = clip_coef(norm if norm_override is None else norm_override, self.max_norm)
        skipped = bool(self.scaler) and found
        if not skipped:
            jobs = []
            for i in (range(len(self.p)) if subset is None else subset):
                if grads[i] is None:
                    continue
                h = self.hparams[self.group_of[i]]
                self.steps[i] += 1.0
                kw = dict(inv=inv, unscale=bool(self.scaler), coef=coef, lr=lrs[self.group_of[i]],
                          beta1=h["betas"][0], beta2=h["betas"][1], eps=h["eps"], wd=h["weight_decay"],
                          step=self.steps[i], maximize=h.get("maximize", False))
                g = np.ascontiguousarray(grads[i], np.float32).reshape(-1)
                jobs.append((g, self.p[i], self.m[i], self.v[i], kw))
            unscale_clip_adamw_many(jobs)
        return self._finish(norm, found, skipped)

    def _finish(self, norm, found, skipped) -> dict:
        out = {"norm": norm, "found_inf": found, "skipped": skipped}
        if self.scaler:
            out["scale_before"] = self.scale
            self.scale, self.tracker = scaler_update(
                self.scale, self.tracker, 1.0 if found else 0.0, self.scaler["growth_factor"],
                self.scaler["backoff_factor"], self.scaler["growth_interval"])
            out["scale"] = self.scale
            out["tracker"] = self.tracker
        return out
