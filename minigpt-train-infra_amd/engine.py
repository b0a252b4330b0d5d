"""Device state and launch sequencing for one AdamW instance.

An engine owns, on one GPU:
  - flat fp32 arenas for exp_avg and exp_avg_sq (and an fp32 master copy for
    bf16/fp16 parameters), one 256-byte-aligned segment per parameter, whose
    per-parameter views are what optimizer.state[p] holds;
  - a float32 step counter per parameter (torch/optim/adam.py:168-176);
  - device scalars found_inf and clip coefficient for the current iteration;
  - per-group bias-correction tables (1 - beta1**t, (1 - beta2**t) ** 0.5),
    computed on the host with the expressions of adam.py:529-536;
  - a libmgopt plan (the device chunk table).

Per iteration the engine records what the caller asked for (a pending
unscale, a clip) and launches:
  norm(max_norm)  -> mgopt_grad_norm  (pass 1 + finalize)
  step()          -> mgopt_adamw_step (prologue + pass 2)
No call waits for the GPU.
"""

from __future__ import annotations

import ctypes
import math
import sys
import weakref
from typing import Sequence

import numpy as np
import torch

from . import _native as N

ALIGN_ELEMS = 64                    # 256 B of fp32 per arena segment
DEFAULT_CHUNK = 1024                # elements per pass-2 work-group (pass 1 has its own 128K-element chunks):
                                    # 512 threads over 1024 elements retire fast and keep half the waves
                                    # of a CU streaming; 2-13 % faster than 16384 from 124M to 8.2B params
SMALL_CHUNK = 2048                  # pass-2 chunk of a plan that runs the three-kernel step (below)
FOLD_ELEMS = 1 << 21                # the library's three-kernel limits: at most this many elements,
FOLD_TENSOR_CHUNKS = 256            # no tensor of more pass-2 chunks than this, no empty tensor
BC_INITIAL_CAP = 1024               # first bias-correction table size (steps)
CAPTURE_BC_CAP = 1 << 16            # fixed table size of a capturable engine (graph replays cannot grow it)
HP_SLOTS = 4                        # pinned host buffers for device hyper-parameter uploads


ROW_MAX = 16384                     # longest row (elements) laid out with its master / m / v rows side by side


def _align(n: int) -> int:
    return (n + ALIGN_ELEMS - 1) // ALIGN_ELEMS * ALIGN_ELEMS


def default_chunk(numels: Sequence[int]) -> int:
    """The pass-2 chunk for a parameter set: SMALL_CHUNK when the plan will
    run the three-kernel step at that chunk, else DEFAULT_CHUNK.  Measured on
    MI355X, 2,048-element chunks made the replayed step of three kernels
    1.4-2.2 us faster than 1,024 on the 0.8M-parameter MiniGPT set, on 0.26M
    elements in one tensor and on 1M and 2M elements in 16 tensors (0.7-1.0 us
    slower on 0.26M elements in 16 tensors of 16,384)."""
    total = sum(numels)
    if 0 < total <= FOLD_ELEMS and min(numels) > 0 and -(-max(numels) // SMALL_CHUNK) <= FOLD_TENSOR_CHUNKS:
        return SMALL_CHUNK
    return DEFAULT_CHUNK


def row_length(shape, chunk_elems: int) -> int:
    """Row length of a parameter's row-laid-out state: the smallest product of
    its trailing dimensions that is a multiple of the pass-2 chunk, up to
    ROW_MAX elements; 0 when there is none (its state then lives in the
    separate arenas).  Placing a row's master, exp_avg and exp_avg_sq side by
    side keeps the update's reads and write-backs of those rows in
    neighbouring DRAM rows: measured on MI355X with rows of 1,024-8,192
    elements, a pass-2-shaped stream over 4.3e9 elements ran at 6.57-6.61 TB/s
    against 6.07-6.38 TB/s with the three arrays apart (the best of three
    relative offsets)."""
    u = 1
    for d in reversed(tuple(shape)):
        u *= int(d)
        if u > ROW_MAX:
            return 0
        if u % chunk_elems == 0:
            return u
    return 0


def row_view(arena: torch.Tensor, offset: int, shape, row: int, fields: int) -> torch.Tensor:
    """The view with `shape` of a tensor whose consecutive rows of `row`
    elements lie fields * row elements apart in `arena`, from `offset`: the
    trailing dimensions that make up a row keep their contiguous strides, the
    leading ones step over the other fields' rows."""
    shape = tuple(int(d) for d in shape)
    strides, acc = [], 1
    for d in reversed(shape):
        strides.append(acc if acc < row else acc * fields)
        acc *= d
    return arena.as_strided(shape, tuple(reversed(strides)), offset)


def bias_correction_table(beta1: float, beta2: float, cap: int, start: int = 0) -> list[float]:
    """[bc1(t), sqrt(bc2)(t)] for t in start..cap-1, formed exactly as
    torch/optim/adam.py:529-536 forms them from step = state["step"].item();
    entry t = 0 (never a step's count) holds [beta1, beta2], which the kernel
    checks against the group's current betas before it uses the row."""
    out: list[float] = []
    if start == 0:
        out += [float(beta1), float(beta2)]
        start = 1
    for t in range(start, cap):
        step = float(t)
        bias_correction1 = 1 - beta1**step
        bias_correction2 = 1 - beta2**step
        out.append(bias_correction1)
        out.append(bias_correction2**0.5)
    return out


class _Engine:
    def __init__(self, optimizer: torch.optim.Optimizer, master_weights: bool | None, chunk_elems: int | None,
                 capturable: bool = False, state_layout: str = "rows"):
        # weak: the optimizer owns the engine, and a reference cycle would hold
        # the arenas (up to 100+ GB) until the cyclic collector happens to run
        self._opt_ref = weakref.ref(optimizer)
        self.params: list[torch.Tensor] = []
        self.group_index: list[int] = []
        seen: set[int] = set()
        for gi, group in enumerate(optimizer.param_groups):
            for p in group["params"]:
                if id(p) in seen:
                    raise ValueError("some parameters appear in more than one parameter group")
                seen.add(id(p))
                self.params.append(p)
                self.group_index.append(gi)
        if not self.params:
            raise ValueError("optimizer got an empty parameter list")
        if len(optimizer.param_groups) > N.MAX_GROUPS:
            raise ValueError(f"at most {N.MAX_GROUPS} parameter groups are supported")
        dev = self.params[0].device
        if dev.type != "cuda":
            raise RuntimeError("mgopt AdamW needs parameters on a ROCm GPU (device type 'cuda'); there is no CPU path")
        for p in self.params:
            if p.device != dev:
                raise RuntimeError("all parameters must live on one GPU")
            if not p.is_contiguous():
                raise RuntimeError("mgopt AdamW needs contiguous parameters")
            if p.dtype not in (torch.float32, torch.float16, torch.bfloat16):
                raise TypeError(f"unsupported parameter dtype {p.dtype}")
        self.device = dev
        N.lib()                              # a GPU is visible and the library is built
        self.chunk_elems = int(chunk_elems) if chunk_elems else default_chunk([p.numel() for p in self.params])
        lowp = [p.dtype != torch.float32 for p in self.params]
        if master_weights is False and any(lowp):
            raise ValueError("bf16/fp16 parameters need master_weights (fp32 master copy); master_weights=False is not supported")
        self.has_master = any(lowp)

        # per-parameter segments on 256-byte boundaries (the layout of the
        # gradient arena, AdamW.use_grad_arena)
        self.offsets: list[int] = []
        total = 0
        for p in self.params:
            self.offsets.append(total)
            total += _align(p.numel())
        self.total = total
        # optimizer state: a parameter with a row length (row_length) keeps its
        # master, exp_avg and exp_avg_sq rows side by side in the rows arena;
        # the others keep each in its own arena, one contiguous segment each
        self.rows = [row_length(p.shape, self.chunk_elems) if state_layout == "rows" else 0 for p in self.params]
        self.fields = [3 if lp else 2 for lp in lowp]        # fp32 arrays per row-laid-out parameter
        self.state_offsets: list[int] = []      # into exp_avg / exp_avg_sq (separate) or rows (row-laid-out)
        self.master_offsets: list[int | None] = []
        stotal = mtotal = rtotal = 0
        for p, lp, row, k in zip(self.params, lowp, self.rows, self.fields):
            if row:
                self.state_offsets.append(rtotal)
                self.master_offsets.append(None)
                rtotal += _align(k * p.numel())
                continue
            self.state_offsets.append(stotal)
            stotal += _align(p.numel())
            self.master_offsets.append(mtotal if lp else None)
            mtotal += _align(p.numel()) if lp else 0
        with torch.cuda.device(dev):
            self.exp_avg = torch.zeros(max(stotal, 1), dtype=torch.float32, device=dev)
            self.exp_avg_sq = torch.zeros(max(stotal, 1), dtype=torch.float32, device=dev)
            self.master = torch.empty(max(mtotal, 1), dtype=torch.float32, device=dev) if mtotal else None
            self.rows_arena = torch.zeros(max(rtotal, 1), dtype=torch.float32, device=dev) if rtotal else None
            self.steps = torch.zeros(len(self.params), dtype=torch.float32, device=dev)
            self.found_inf = torch.zeros((), dtype=torch.float32, device=dev)
            self.coef = torch.ones((), dtype=torch.float32, device=dev)
            # log-window record: norm_last, norm_max (fp32), skipped, taken (uint32)
            self.window = torch.zeros(4, dtype=torch.float32, device=dev)
        self.found_inf_ptr, self.coef_ptr = self.found_inf.data_ptr(), self.coef.data_ptr()
        self.master_synced = not self.has_master

        # views handed out through optimizer.state
        self.views: list[dict[str, torch.Tensor]] = []
        for i, (p, lp) in enumerate(zip(self.params, lowp)):
            off, n, row = self.state_offsets[i], p.numel(), self.rows[i]
            v = {"step": self.steps[i]}
            if row:
                k = self.fields[i]
                names = (["master_param"] if lp else []) + ["exp_avg", "exp_avg_sq"]
                for f, name in enumerate(names):
                    v[name] = row_view(self.rows_arena, off + f * row, p.shape, row, k)
            else:
                v["exp_avg"] = self.exp_avg[off : off + n].view(p.shape)
                v["exp_avg_sq"] = self.exp_avg_sq[off : off + n].view(p.shape)
                mo = self.master_offsets[i]
                if mo is not None:
                    v["master_param"] = self.master[mo : mo + n].view(p.shape)
            self.views.append(v)

        self.param_ptr_bytes = np.array([p.data_ptr() for p in self.params], np.int64).tobytes()
        self.param_dtype_codes = tuple(N.dtype_code(p.dtype) for p in self.params)
        self.pset = None
        self.plan: int | None = None
        self.plan_grad_dtypes: tuple[int, ...] | None = None
        self.grad_ptr_bytes: bytes | None = None
        self.grad_dtype_bytes: bytes | None = None
        self.grad_source: list[torch.Tensor | None] | None = None
        self.grad_source_checked = False
        # with a gradient arena: 1 where a parameter's gradient exists in the
        # sense of torch's p.grad is not None (set when autograd accumulates
        # into it, cleared by zero_grad(set_to_none=True)); None: every arena
        # gradient counts
        self.present: np.ndarray | None = None
        self.complete_keys: set[tuple[int, ...]] = set()   # id tuples of parameter lists equal to self.params
        self.t_bound = 0                     # upper bound of any step count reachable next step
        self.bc_cap = 0
        self.bc_keys: list[tuple[float, float]] = []
        self.bc_host: list[list[float]] = []     # host copy of each group's table row
        self.bc_src: list[tuple] | None = None   # the hp_key the table was last checked against
        self.bc_table: torch.Tensor | None = None
        self.hp = None                       # GroupHparams array passed to mgopt_adamw_step
        self.hp_addr = 0                     # its address
        self.hp_key: list[tuple] | None = None
        self.hp_raw: list[tuple] | None = None
        # capturable: the kernels read the group records from a fixed device
        # buffer (refreshed from param_groups by asynchronous copies outside
        # any capture), the bias-correction table has a fixed size, and once a
        # step was captured the plan's device tables may not be replaced
        self.capturable = capturable
        self.captured = False
        self.hp_dev: torch.Tensor | None = None
        self.hp_dev_key: list[tuple] | None = None
        if capturable:
            with torch.cuda.device(dev):
                self.hp_dev = torch.zeros(N.MAX_GROUPS * ctypes.sizeof(N.GroupHparams), dtype=torch.uint8, device=dev)
            self.hp_slots = [torch.empty(self.hp_dev.numel(), dtype=torch.uint8, pin_memory=True) for _ in range(HP_SLOTS)]
            self.hp_events: list[torch.cuda.Event | None] = [None] * HP_SLOTS
            self.hp_slot = 0
        self.reset_iteration()

    @property
    def opt(self) -> torch.optim.Optimizer:
        opt = self._opt_ref()
        if opt is None:
            raise RuntimeError("the optimizer that owned this engine was released")
        return opt

    # ------------------------------------------------------------------ plan
    def close(self) -> None:
        if self.plan is not None:
            N.load_library().mgopt_plan_destroy(ctypes.c_void_p(self.plan))
            self.plan = None

    def __del__(self, _finalizing=sys.is_finalizing):
        # At interpreter shutdown module globals (sys, the library handle) may
        # already be None, so the check is bound when the class is defined;
        # then the HIP runtime may be gone too and the process releases
        # everything itself.
        try:
            if _finalizing():
                return
            self.close()
        except Exception:
            pass

    def _build_plan(self, grad_dtypes: tuple[int, ...]) -> None:
        if self.captured:
            raise RuntimeError("the gradient dtypes changed after a step of this optimizer was captured in a HIP "
                               "graph; the graph reads this plan's device tables, so it cannot be rebuilt")
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the optimizer's device plan does not exist yet: run one step outside graph capture "
                               "before capturing")
        self.close()
        lib = N.lib()
        descs = (N.TensorDesc * len(self.params))()
        for i, p in enumerate(self.params):
            d = descs[i]
            v = self.views[i]
            if "master_param" not in v:
                d.param_dev = p.data_ptr()
                d.lowp_dev = None
                d.lowp_dtype = N.NONE
            else:
                d.param_dev = v["master_param"].data_ptr()
                d.lowp_dev = p.data_ptr()
                d.lowp_dtype = N.dtype_code(p.dtype)
            d.exp_avg_dev = v["exp_avg"].data_ptr()
            d.exp_avg_sq_dev = v["exp_avg_sq"].data_ptr()
            d.numel = p.numel()
            d.group = self.group_index[i]
            d.grad_dtype = grad_dtypes[i]
            row = self.rows[i]
            if row:
                pitch = self.fields[i] * row
                d.row_elems = row
                d.state_pitch = pitch
                d.param_pitch = pitch if "master_param" in v else row
        plan = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            N.check(
                lib.mgopt_plan_create(descs, len(self.params), len(self.opt.param_groups), self.steps.data_ptr(),
                                      self.chunk_elems, ctypes.byref(plan)),
                "mgopt_plan_create",
            )
        self.plan = plan.value
        N.check(lib.mgopt_plan_set_window(ctypes.c_void_p(self.plan), ctypes.c_void_p(self.window.data_ptr())),
                "mgopt_plan_set_window")
        self.plan_grad_dtypes = grad_dtypes
        self.grad_ptr_bytes = None

    def set_grad_source(self, grads: Sequence[torch.Tensor | None] | None) -> None:
        if grads is not None:
            grads = list(grads)
            if len(grads) != len(self.params):
                raise ValueError("need one gradient (or None) per parameter")
            for g, p in zip(grads, self.params):
                if g is not None and g.shape != p.shape:
                    raise ValueError("gradient shape does not match its parameter")
        self.grad_source = grads
        self.grad_source_checked = False
        self.pset = None

    def current_grads(self) -> list[torch.Tensor | None]:
        if self.grad_source is not None:
            return self.grad_source
        if self.present is not None:
            return [p.grad if k else None for p, k in zip(self.params, self.present)]
        return [p.grad for p in self.params]

    def prepare(self) -> None:
        """Validates pointers and uploads the grad table for this iteration
        (once per iteration: the norm pass and the step share it)."""
        if self.prepared:
            return
        ps = self._param_set()
        if self.plan is None or not ps.unchanged():
            self._prepare()
            ps.remember()
        self.prepared = True

    def clear_grads(self) -> None:
        """zero_grad(set_to_none=True) in one native pass over the parameters."""
        self._param_set().clear_grads()

    def _param_set(self):
        """The native view of the parameters (and gradient source) that
        gathers the gradient table and launches the per-step entry points."""
        if self.pset is None:
            ps = N.host().ParamSet(self.params, [] if self.grad_source is None else self.grad_source)
            ps.bind(N.entry_address("mgopt_grad_norm"), N.entry_address("mgopt_adamw_step"))
            ps.set_mask(0 if self.present is None else self.present.ctypes.data)
            self.pset = ps
        return self.pset

    def set_present(self, present: np.ndarray | None) -> None:
        """The arena's gradient-presence record (kept by backward hooks), or
        None when every arena gradient counts."""
        self.present = present
        if self.pset is not None:
            self.pset.set_mask(0 if present is None else present.ctypes.data)

    def _prepare(self) -> None:
        ps = self._param_set()
        if self.grad_source is not None and self.grad_source_checked and self.plan is not None:
            # a fixed gradient source is validated and uploaded once; only the
            # parameters' storage is re-checked
            if ps.param_ptrs() != self.param_ptr_bytes:
                self._moved()
            return
        pptrs, gptrs, gdt, gflags = ps.gather()
        if pptrs != self.param_ptr_bytes:
            self._moved()
        if self.present is not None and not self.present.all():
            # arena gradients that torch would hold as None take no part
            absent = self.present == 0
            g = np.frombuffer(gptrs, np.int64).copy()
            d = np.frombuffer(gdt, np.int8).copy()
            g[absent], d[absent] = 0, -1
            gptrs, gdt = g.tobytes(), d.tobytes()
        if gptrs == self.grad_ptr_bytes and gdt == self.grad_dtype_bytes and self.plan is not None:
            return
        flags = np.frombuffer(gflags, np.int8)
        if flags.any():
            i = int(np.flatnonzero(flags)[0])
            f = int(flags[i])
            what = ("is sparse" if f & 8 else "lives on another device" if f & 4 else
                    "has a different size than its parameter" if f & 2 else "is not contiguous")
            raise RuntimeError(f"gradient of parameter {i} {what}; mgopt AdamW needs dense contiguous "
                               "gradients on the parameters' GPU")
        codes = np.frombuffer(gdt, np.int8)
        if (codes == -2).any():
            i = int(np.flatnonzero(codes == -2)[0])
            raise TypeError(f"gradient of parameter {i} has an unsupported dtype; expected float32, float16 or bfloat16")
        # a tensor without a grad this step keeps the dtype it had (or its parameter's)
        prev = self.plan_grad_dtypes if self.plan_grad_dtypes is not None else self.param_dtype_codes
        dtypes_t = tuple(prev[i] if c < 0 else int(c) for i, c in enumerate(codes))
        if self.plan is None or dtypes_t != self.plan_grad_dtypes:
            self._build_plan(dtypes_t)
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the gradient tensors changed since the last step outside graph capture; a captured "
                               "step reads gradients from fixed buffers (keep .grad tensors in place, for instance "
                               "with use_grad_arena or zero_grad(set_to_none=False))")
        arr = ctypes.cast(ctypes.c_char_p(gptrs), ctypes.POINTER(ctypes.c_void_p))
        N.check(N.lib().mgopt_plan_set_grads(self.plan, arr, self._stream()),
                "mgopt_plan_set_grads")
        self.grad_ptr_bytes, self.grad_dtype_bytes = gptrs, gdt
        if self.grad_source is not None:
            self.grad_source_checked = True

    def _moved(self) -> None:
        raise RuntimeError(
            "a parameter's storage moved (param.data was replaced) after the optimizer was built; "
            "copy new values in place with param.data.copy_() instead"
        )

    # ------------------------------------------------------- iteration state
    def reset_iteration(self) -> None:
        self.scale_src: torch.Tensor | None = None   # pending lazy unscale (GradScaler scale tensor)
        self.norm_done = False
        self.clip_pending = False
        self.prepared = False

    def request_unscale(self, scale: torch.Tensor) -> torch.Tensor:
        """GradScaler.unscale_: deferred; returns the found_inf tensor the
        coming pass 1 will fill."""
        if scale.device != self.device or scale.dtype != torch.float32 or scale.numel() != 1:
            raise RuntimeError("scale must be a float32 scalar on the optimizer's device")
        self.scale_src = scale
        self.norm_done = False
        return self.found_inf

    def _stream(self) -> int:
        return N.stream_handle(self.device)

    def norm(self, max_norm: float | None) -> torch.Tensor:
        """Pass 1 + finalize; returns the pre-clip total norm (fresh 0-dim tensor)."""
        if self.norm_done and self.clip_pending:
            raise RuntimeError("clip_grad_norm_ was already called for this optimizer step")
        self.prepare()
        out = self._launch_norm(True, max_norm)
        self.norm_done = True
        self.clip_pending = max_norm is not None
        return out

    def _launch_norm(self, want_norm: bool, max_norm: float | None) -> torch.Tensor | None:
        """Pass 1 (+ finalize); returns a fresh norm tensor when want_norm.
        max_norm None: no clipping requested, the coefficient is not written."""
        scale = self.scale_src
        out = self.pset.grad_norm(
            self.plan,
            scale.data_ptr() if scale is not None else 0,
            float(max_norm) if max_norm is not None else 0.0,
            want_norm,
            self.coef_ptr if max_norm is not None else 0,
            self.found_inf_ptr if scale is not None else 0,
            self._stream(),
        )
        if isinstance(out, int):
            N.check(out, "mgopt_grad_norm")
        return out

    def _ensure_bc(self) -> None:
        """(Re)builds the bias-correction table when the reachable step bound
        outgrows it or a group's betas changed.  A capturable engine's table
        has a fixed size and is rewritten in place (a captured graph holds its
        address); counts beyond it take the kernels' device evaluation."""
        keys = [(k[2], k[3]) for k in self.hp_key]
        need = self.t_bound + 2
        if self.bc_table is not None and keys == self.bc_keys and (need <= self.bc_cap or self.capturable):
            self.bc_src = self.hp_key
            return
        if torch.cuda.is_current_stream_capturing():
            if self.bc_table is None:
                raise RuntimeError("run one step outside graph capture before capturing")
            return   # betas changed under capture: the kernels see a row built for other betas and evaluate on the device
        self.bc_src = self.hp_key
        if self.capturable:
            cap = CAPTURE_BC_CAP
        else:
            cap = max(BC_INITIAL_CAP, self.bc_cap)
            while cap < need:
                cap *= 2
        # the host rows of groups whose betas are unchanged are extended, not
        # recomputed: a doubling at step t costs t new entries, not 2t
        old = dict(zip(self.bc_keys, self.bc_host)) if self.bc_table is not None else {}
        rows = []
        for b1, b2 in keys:
            row = old.get((b1, b2))
            row = list(row) if row is not None else []
            row.extend(bias_correction_table(b1, b2, cap, start=len(row) // 2))
            rows.append(row)
        host = torch.tensor([x for row in rows for x in row], dtype=torch.float64)
        if self.capturable and self.bc_table is not None:
            self.bc_table.copy_(host)
            table = self.bc_table
        else:
            table = host.to(self.device)
        self.bc_table, self.bc_cap, self.bc_keys, self.bc_host = table, cap, keys, rows

    def sync_master(self) -> None:
        """Copies bf16/fp16 parameters into the fp32 master (exact widening)."""
        if not self.has_master:
            return
        if self.plan is None:
            self.prepare()
        N.check(N.lib().mgopt_sync_master(self.plan, self._stream()), "mgopt_sync_master")
        self.master_synced = True

    def step(self, found_inf: torch.Tensor | None = None, grad_scale: torch.Tensor | None = None,
             writeback: bool = False) -> None:
        self.prepare()
        if not self.master_synced:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("the master weights must be synced from the parameters outside graph capture "
                                   "(run one step after loading or replacing parameters)")
            self.sync_master()
        scale = self.scale_src
        skip_src = None
        if scale is not None:
            if not self.norm_done:
                self._launch_norm(False, None)   # found_inf only, no clipping
            skip_src = self.found_inf
        else:
            if grad_scale is not None:
                scale = grad_scale
            skip_src = found_inf
        capturing = torch.cuda.is_current_stream_capturing()
        self.read_hparams()
        self.t_bound += 1
        if self.t_bound + 2 > self.bc_cap or self.bc_src is not self.hp_key:
            self._ensure_bc()
        flags = N.WRITEBACK_GRADS if writeback else 0
        groups_addr = self.hp_addr
        if self.capturable:
            if capturing:
                if self.hp_dev_key is None:
                    raise RuntimeError("run one step outside graph capture before capturing")
                self.captured = True
            elif self.hp_dev_key != self.hp_key:
                self.upload_hparams()
            groups_addr = self.hp_dev.data_ptr()
            flags |= N.GROUPS_ON_DEVICE
        rc = self.pset.adamw_step(
            self.plan, groups_addr, self.bc_table.data_ptr(), self.bc_cap,
            scale.data_ptr() if scale is not None else 0,
            self.coef_ptr if self.clip_pending else 0,
            skip_src.data_ptr() if skip_src is not None else 0,
            flags, self._stream(),
        )
        if rc:
            N.check(rc, "mgopt_adamw_step")
        self.reset_iteration()

    def read_hparams(self) -> None:
        """Reads the groups' hyper-parameters into the record array passed to
        the kernels.  The groups' values are compared as stored and converted
        only when one changed (a tensor lr is always re-read)."""
        groups = self.opt.param_groups
        # betas copied into a tuple: a list mutated in place must not compare equal to its earlier self
        raw = [(g["lr"], g["weight_decay"], tuple(g["betas"]), g["eps"], g.get("maximize", False),
                g.get("amsgrad", False)) for g in groups]
        if not any(isinstance(r[0], torch.Tensor) for r in raw) and raw == self.hp_raw:
            return
        key = []
        for lr, wd, betas, eps, maximize, amsgrad in raw:
            if amsgrad:
                raise NotImplementedError("amsgrad is not supported by mgopt AdamW")
            key.append((float(lr.item() if isinstance(lr, torch.Tensor) else lr), float(wd),
                        float(betas[0]), float(betas[1]), float(eps), bool(maximize)))
        if key != self.hp_key:
            # the record block is rewritten only when a group changed
            hp = (N.GroupHparams * len(groups))()
            for d, (lr, wd, b1, b2, eps, maximize) in zip(hp, key):
                d.lr, d.weight_decay, d.beta1, d.beta2, d.eps, d.maximize = lr, wd, b1, b2, eps, int(maximize)
            self.hp, self.hp_key = hp, key
            self.hp_addr = ctypes.addressof(hp)
        self.hp_raw = None if any(isinstance(r[0], torch.Tensor) for r in raw) else raw

    def upload_hparams(self) -> None:
        """Copies the group records into the device buffer a capturable
        engine's kernels read (asynchronous, from a pinned slot, on the
        current stream)."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("hyper-parameters cannot be uploaded during graph capture")
        k = self.hp_slot
        if self.hp_events[k] is not None:
            self.hp_events[k].synchronize()     # the slot may still feed an earlier copy
        data = np.frombuffer(bytes(self.hp), np.uint8)
        slot = self.hp_slots[k]
        slot.numpy()[: data.size] = data
        with torch.cuda.device(self.device):
            self.hp_dev[: data.size].copy_(slot[: data.size], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
        self.hp_events[k] = ev
        self.hp_slot = (k + 1) % HP_SLOTS
        self.hp_dev_key = self.hp_key

    def refresh_hparams(self) -> None:
        """Brings a capturable engine's device records up to date with
        param_groups (before a graph replay)."""
        self.read_hparams()
        if self.capturable and self.hp_dev_key != self.hp_key:
            if self.bc_table is not None and [(k[2], k[3]) for k in self.hp_key] != self.bc_keys:
                self._ensure_bc()                # new betas: rewrite the table rows in place
            self.upload_hparams()

    def window_metrics(self, reset: bool = True) -> dict:
        """Reads the log-window record (one device-to-host copy)."""
        w = self.window.detach().cpu()
        counts = w.view(torch.int32)
        out = {
            "grad_norm_last": float(w[0]),
            "grad_norm_max": float(w[1]),
            "skipped_steps": int(counts[2]),
            "optimizer_steps": int(counts[3]),
        }
        if reset:
            self.window.zero_()
        return out

    def folded(self) -> bool:
        """True when the plan runs a step as three kernels (a small plan: pass
        1 finalizes in its last work-group, pass 2 forms the step counts)."""
        return self.plan is not None and N.load_library().mgopt_plan_folded(ctypes.c_void_p(self.plan)) == 1

    def device_bc_flag(self) -> int:
        """1 once a step has computed bias corrections on the device (a step
        count outside the host table), else 0.  Waits for the GPU."""
        out = ctypes.c_int(0)
        if self.plan is not None:
            N.check(N.lib().mgopt_plan_flags(ctypes.c_void_p(self.plan), ctypes.byref(out)), "mgopt_plan_flags")
        return out.value

    def set_step_counts(self, counts: Sequence[float]) -> None:
        self.steps.copy_(torch.tensor([float(c) for c in counts], dtype=torch.float32))
        self.t_bound = int(math.ceil(max(counts))) if counts else 0
