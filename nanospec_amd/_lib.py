"""ctypes binding of ``libnanospec_hip.so`` (the C ABI in include/nanospec_hip.h).

Tensors cross the boundary as raw device pointers plus sizes; every call is
enqueued on torch's current HIP stream.  Negative status codes become
``ValueError`` and HIP errors ``RuntimeError`` (the reference raises
``ValueError`` for bad configuration, config.py:62-66).  There is no fallback:
if the library is missing, loading raises.
"""

from __future__ import annotations

import ctypes
import os
import re

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnanospec_hip.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "nanospec_hip.h")

ABI_VERSION = 6
NS_BF16, NS_F32 = 0, 1
NS_WS_LOGITS, NS_WS_LMHEAD, NS_WS_LMHEAD_BWD, NS_WS_FP8 = 0, 1, 2, 3
NS_PART_STATS, NS_PART_EMIT = 1, 2
NS_WS_RMS_NORM_BWD, NS_WS_LMHEAD_NORM_BWD, NS_WS_TEACHER_LOGITS = 4, 5, 6

_c = ctypes
_P = _c.c_void_p
_I64 = _c.c_int64
_F = _c.c_float
_I = _c.c_int
_SZ = _c.c_size_t


class RmsNormBwd(ctypes.Structure):
    """struct ns_rms_norm_args of the header."""

    _fields_ = [("x", _P), ("ldx", _I64), ("inv", _P), ("weight", _P), ("dx", _P), ("lddx", _I64),
                ("weight_grad", _P)]


_NORM = ctypes.POINTER(RmsNormBwd)


class TeacherArgs(ctypes.Structure):
    """struct ns_teacher_args of the header."""

    _fields_ = [("rows", _P), ("n_rows", _I64), ("lse", _P)]


_TEACH = ctypes.POINTER(TeacherArgs)

# argtypes of every exported entry point (kept in the header's order)
SIGNATURES = {
    "ns_abi_version": ([], _I),
    "ns_last_error": ([], _c.c_char_p),
    "ns_workspace_bytes": ([_I, _I64, _I64, _I64], _SZ),
    "ns_ce_kl_logits_fwd": (
        [_P, _I, _I64, _P, _I, _I64, _P, _P, _P, _I64, _I64, _I64, _F, _F, _F, _P, _I64, _P, _P, _P, _SZ, _P],
        _I,
    ),
    "ns_ce_kl_logits_bwd": (
        [_P, _I, _I64, _P, _I, _I64, _P, _P, _I64, _I64, _F, _F, _F, _P, _P, _I64, _P],
        _I,
    ),
    "ns_lmhead_ce_kl_fwd_part": (
        [_I, _P, _I64, _P, _I64, _P, _I64, _P, _I, _I64, _TEACH, _P, _P, _I64, _I64, _I64, _F, _F, _F,
         _P, _I64, _P, _P, _SZ, _P],
        _I,
    ),
    "ns_objective_metrics": ([_P, _P, _P, _I64, _I64, _F, _F, _P, _P], _I),
    "ns_copy_rows": ([_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P], _I),
    "ns_lmhead_ce_kl_fwd": (
        [_P, _I64, _P, _I64, _P, _I64, _P, _I, _I64, _TEACH, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _F, _F,
         _P, _I64, _P, _P, _P, _SZ, _P],
        _I,
    ),
    "ns_device_init": ([], _I),
    "ns_lmhead_ce_kl_fwd_noalloc": (
        [_P, _I64, _P, _I64, _P, _I64, _P, _I, _I64, _TEACH, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _F, _F,
         _P, _I64, _P, _P, _P],
        _I,
    ),
    "ns_lmhead_markov_ce_kl_fwd": (
        [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _P, _I, _I64, _TEACH, _P, _P, _P, _I64, _I64, _I64,
         _I64, _F, _F, _F, _P, _I64, _P, _P, _P, _SZ, _P],
        _I,
    ),
    "ns_lmhead_ce_kl_bwd": (
        [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _P, _I, _I64, _TEACH, _P, _P, _I64, _I64,
         _I64, _F, _F, _F, _P, _P, _I64, _P, _SZ, _P],
        _I,
    ),
    "ns_lmhead_teacher_logits": (
        [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _SZ, _P],
        _I,
    ),
    "ns_lmhead_bwd": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P], _I),
    "ns_rms_norm_fwd": ([_P, _I64, _P, _I64, _I64, _F, _P, _I64, _P, _I64, _P, _P], _I),
    "ns_rms_norm_bwd": ([_P, _I64, _NORM, _I64, _I64, _P, _SZ, _P], _I),
    "ns_lmhead_norm_bwd": ([_P, _I64, _P, _I64, _NORM, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P], _I),
    "ns_lmhead_markov_bwd_workspace_bytes": ([_I64, _I64, _I64, _I64], _SZ),
    "ns_lmhead_markov_bwd": (
        [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _P, _I64, _NORM, _P, _I64, _P, _I64, _I64, _I64,
         _I64, _P, _SZ, _P],
        _I,
    ),
    "ns_pooled_tail": ([_P, _I64, _I64, _I64, _P, _P], _I),
    "ns_scale_gradient": ([_P, _I, _I64, _P, _P], _I),
    "ns_lmhead_linear": ([_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P], _I),
    "ns_fp8_teacher_logits": ([_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _SZ, _P], _I),
    "ns_fp8_quantize_rows": ([_P, _I64, _I64, _I64, _P, _P, _P], _I),
    "ns_prepare_slots": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P, _P, _P], _I),
}


class KernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_int), ("total_ms", ctypes.c_double)]


SIGNATURES["ns_profile_begin"] = ([], _I)
SIGNATURES["ns_profile_select"] = ([ctypes.c_char_p], _I)
SIGNATURES["ns_profile_end"] = ([ctypes.POINTER(KernelTime), _I, ctypes.POINTER(_I)], _I)

_lib = None


def header_symbols(path: str = HEADER) -> list[str]:
    """Function names declared in the public header."""
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(ns_\w+)\s*\(", text, re.M)))


def load():
    """Load the library once; raises if it is not built or the ABI differs."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m nanospec_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    version = lib.ns_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libnanospec_hip ABI {version} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(status: int, name: str) -> None:
    if status == 0:
        return
    msg = load().ns_last_error().decode(errors="replace")
    if status < 0:
        raise ValueError(f"{name}: {msg}")
    raise RuntimeError(f"{name}: HIP error {status}: {msg}")


def ptr(t: torch.Tensor | None):
    return None if t is None else _c.c_void_p(t.data_ptr())


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return NS_BF16
    if t.dtype == torch.float32:
        return NS_F32
    raise ValueError(f"unsupported dtype {t.dtype}; expected bfloat16 or float32")


def stream(device: torch.device):
    """hipStream_t of torch's current stream on ``device``."""
    return _c.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"tensors must live on a HIP device (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def workspace(kind: int, n: int, v: int, d: int, device: torch.device) -> torch.Tensor:
    nbytes = int(load().ns_workspace_bytes(kind, n, v, d))
    # torch's caching allocator returns 256-byte aligned blocks
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def rows_2d(t: torch.Tensor, cols: int) -> tuple[torch.Tensor, int]:
    """View ``t`` as [rows, cols] with unit column stride; returns (view, ld)."""
    t2 = t.reshape(-1, cols)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < cols):
        t2 = t2.contiguous()
    ld = t2.stride(0) if t2.shape[0] > 1 else cols
    return t2, ld


def copy_rows(src: torch.Tensor, rows_map: torch.Tensor, n_dst: int, out: torch.Tensor) -> torch.Tensor:
    """out row r = src row rows_map[r], zeros where rows_map[r] is outside [0, src rows)
    (ns_copy_rows); src and out [rows, cols] views with unit column stride, the same dtype."""
    row_bytes = src.shape[1] * src.element_size()
    status = load().ns_copy_rows(ptr(src), src.stride(0) * src.element_size(), src.shape[0], ptr(rows_map), n_dst,
                                 row_bytes, ptr(out), out.stride(0) * out.element_size(), stream(src.device))
    check(status, "ns_copy_rows")
    return out


def pow2_ratio(emitted: int, wanted: int):
    """emitted / wanted when it is a power of two (1/4, 2, ...), else None.  dl is linear in
    1/accumulation_steps, and every rounding on its way commutes with a power-of-two scale, so
    dl emitted for `emitted` steps times this ratio is, bit for bit, the dl emitted for `wanted`
    (for normal values; a result below 2^-126 can differ in its last bits)."""
    from fractions import Fraction

    f = Fraction(int(emitted), int(wanted))
    if f.numerator & (f.numerator - 1) == 0 and f.denominator & (f.denominator - 1) == 0:
        return float(f)
    return None


def scale_inplace(t: torch.Tensor, factor: float) -> None:
    """t *= factor on the device (ns_scale_gradient), t contiguous bf16 or fp32."""
    if not t.is_contiguous():
        raise ValueError("scale_inplace needs a contiguous tensor")
    f = torch.full((), float(factor), dtype=torch.float32, device=t.device)
    check(load().ns_scale_gradient(ptr(t), dtype_code(t), t.numel(), ptr(f), stream(t.device)), "ns_scale_gradient")


class KernelTimer:
    """Context manager around ns_profile_begin/end: per-kernel launches and
    total milliseconds, measured with HIP events on each launch's stream.
    ``only``: the timer names to time (the others run without events); None: all."""

    def __init__(self, only=None):
        self.only = only

    def __enter__(self):
        lib = load()
        names = ",".join(sorted(self.only)) if self.only else ""
        check(lib.ns_profile_select(names.encode()), "ns_profile_select")
        check(lib.ns_profile_begin(), "ns_profile_begin")
        self.times = {}
        return self

    def __exit__(self, *exc):
        buf = (KernelTime * 64)()
        count = _c.c_int(0)
        lib = load()
        status = lib.ns_profile_end(buf, 64, _c.byref(count))
        lib.ns_profile_select(b"")
        for i in range(min(count.value, 64)):
            name = buf[i].name.decode()
            self.times[name] = (buf[i].launches, buf[i].total_ms)
        if exc[0] is None:
            check(status, "ns_profile_end")
        return False

    def mean_ms(self, name: str) -> float:
        launches, total = self.times[name]
        return total / max(launches, 1)
