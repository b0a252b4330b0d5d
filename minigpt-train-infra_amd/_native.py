"""ctypes binding of libmgopt.so (the C ABI declared in include/mgopt.h).

The library is loaded from this package's _build/ directory only.  There is no
fallback: if the library is missing or no GPU is visible, every entry point
that needs it raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libmgopt.so"

F32, F16, BF16, NONE = 0, 1, 2, -1
MAX_GROUPS = 16
WRITEBACK_GRADS = 1
GROUPS_ON_DEVICE = 2

#: every symbol include/mgopt.h declares
EXPORTS = (
    "mgopt_plan_create",
    "mgopt_plan_destroy",
    "mgopt_plan_num_chunks",
    "mgopt_plan_folded",
    "mgopt_plan_set_grads",
    "mgopt_grad_norm",
    "mgopt_adamw_step",
    "mgopt_scaler_update",
    "mgopt_scale_grads",
    "mgopt_sync_master",
    "mgopt_plan_set_window",
    "mgopt_plan_flags",
    "mgopt_grad_norm_noalloc",
    "mgopt_synth_fill",
    "mgopt_last_error",
    "mgopt_version",
)


class TensorDesc(ctypes.Structure):
    _fields_ = [
        ("param_dev", ctypes.c_void_p),
        ("lowp_dev", ctypes.c_void_p),
        ("exp_avg_dev", ctypes.c_void_p),
        ("exp_avg_sq_dev", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("group", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("lowp_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("row_elems", ctypes.c_int64),
        ("param_pitch", ctypes.c_int64),
        ("state_pitch", ctypes.c_int64),
    ]


class GroupHparams(ctypes.Structure):
    _fields_ = [
        ("lr", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("maximize", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class MgoptError(RuntimeError):
    """A libmgopt call returned a nonzero status."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    vp, i32, i64, u64, dbl = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double
    sig = {
        "mgopt_plan_create": (ctypes.c_int, [ctypes.POINTER(TensorDesc), i32, i32, vp, i64, ctypes.POINTER(vp)]),
        "mgopt_plan_destroy": (ctypes.c_int, [vp]),
        "mgopt_plan_num_chunks": (i64, [vp]),
        "mgopt_plan_folded": (ctypes.c_int, [vp]),
        "mgopt_plan_set_grads": (ctypes.c_int, [vp, ctypes.POINTER(vp), vp]),
        "mgopt_grad_norm": (ctypes.c_int, [vp, vp, dbl, vp, vp, vp, vp]),
        "mgopt_adamw_step": (ctypes.c_int, [vp, vp, vp, i64, vp, vp, vp, i32, vp]),
        "mgopt_scaler_update": (ctypes.c_int, [vp, vp, ctypes.POINTER(vp), i32, dbl, dbl, i32, vp]),
        "mgopt_scale_grads": (ctypes.c_int, [vp, vp, vp]),
        "mgopt_sync_master": (ctypes.c_int, [vp, vp]),
        "mgopt_plan_set_window": (ctypes.c_int, [vp, vp]),
        "mgopt_plan_flags": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_int)]),
        "mgopt_grad_norm_noalloc": (ctypes.c_int, [vp, i32, i64, vp, dbl, vp, vp, vp, vp]),
        "mgopt_synth_fill": (ctypes.c_int, [vp, i32, i64, u64, u64, dbl, u64, dbl, vp]),
        "mgopt_last_error": (ctypes.c_char_p, []),
        "mgopt_version": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load_library() -> ctypes.CDLL:
    """Loads libmgopt.so without touching the GPU (safe on a CPU-only host)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                    "python minigpt-train-infra_amd/build.py"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            _declare(lib)
            _lib = lib
        return _lib


_gpu_seen = False


def lib() -> ctypes.CDLL:
    """The library, for calls that launch GPU work: requires a visible GPU."""
    global _gpu_seen
    if not _gpu_seen:
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("libmgopt needs a ROCm GPU; none is visible (there is no CPU fallback)")
        _gpu_seen = True
    return load_library()


HOST_PATH = Path(__file__).resolve().parent / "_build" / "host" / "mgopt_host.so"
_host = None


def host():
    """The host-side helper module (per-step pointer gathering in C++)."""
    global _host
    if _host is None:
        import importlib.util

        import torch  # noqa: F401  (loads the libtorch libraries the helper links against)

        if not HOST_PATH.exists():
            raise RuntimeError(f"{HOST_PATH} is not built; run __graft_entry__.build()")
        spec = importlib.util.spec_from_file_location("mgopt_host", HOST_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _host = mod
    return _host


_addresses: dict[str, int] = {}


def entry_address(name: str) -> int:
    """The address of one of the library's entry points (for the host helper,
    which calls the per-step ones directly)."""
    addr = _addresses.get(name)
    if addr is None:
        addr = _addresses[name] = ctypes.cast(getattr(lib(), name), ctypes.c_void_p).value
    return addr


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().mgopt_last_error().decode(errors="replace")
        raise MgoptError(f"{what} failed with status {rc}: {msg}")


def stream_handle(device) -> int:
    """The raw HIP stream behind torch's current stream on `device` (what
    torch.cuda.current_stream(device).cuda_stream returns, without building a
    Stream object: this is called several times per optimizer step)."""
    import torch

    index = device.index if isinstance(device, torch.device) else device
    if index is None:
        index = torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(index)
    return torch.cuda.current_stream(index).cuda_stream


def dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
    if dtype not in codes:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16")
    return codes[dtype]
