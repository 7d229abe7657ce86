"""ctypes binding of libocto_head.so (the C ABI declared in include/octo_head.h).

Every entry point returns an int status; `call` turns a non-zero status into the Python exception the
reference raises for the same condition (ValueError for bad arguments, NotImplementedError for an
unsupported dtype or option, RuntimeError for a HIP failure). The library is required: there is no
fallback, and importing a GPU entry point without it raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libocto_head.so")

# status codes and enums (include/octo_head.h)
OK, EINVAL, EWORKSPACE, EUNSUPPORTED, EHIP = 0, -1, -2, -3, -4
BF16, F16, F32, FP8E4M3 = 0, 1, 2, 3
ROWS_VIA_IDX, OUT_SCATTER, GRADW_ACCUMULATE, WS_BACKWARD, WS_NO_GRADW, WS_GATHER, LSE_PAIR = 1, 2, 4, 8, 16, 32, 64
WS_STEP = 128
WS_NO_GRADH = 256
PAIRS_NONE_AS_COUNT = 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t



class GrpoTail(ctypes.Structure):
    """octo_grpo_tail: the GRPO weight octo_head_fwd_grpo computes per compact row."""
    _fields_ = [("prox", _p), ("old", _p), ("adv", _p), ("mask", _p), ("n_tokens", _i64),
                ("eps_lo", _f32), ("eps_hi", _f32), ("reject_upper", _f32), ("g", _p), ("loss", _p)]


# name -> argument types (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "octo_version": [],
    "octo_last_error": [],
    "octo_timing_enable": [_i32],
    "octo_timing_read": [ctypes.c_char_p, ctypes.POINTER(_i32), ctypes.POINTER(ctypes.c_double)],
    "octo_head_workspace_bytes": [_i64, _i32, _i32, _i32, _i32, ctypes.POINTER(_sz)],
    "octo_head_bwd_plan": [_i64, _i32, _i32, _i32, _i32, _sz, ctypes.POINTER(_i64)],
    "octo_compact_rows": [_p, _i64, _p, _p, _p],
    "octo_head_fwd": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                      _f32, _f32, _f32, _i32, _p, _p, _p, _p, _i64, _p, _sz, _p],
    "octo_head_fwd_grpo": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                           _f32, _f32, _f32, _i32, _p, _p, _p, _p, _i64, ctypes.POINTER(GrpoTail), _p, _sz, _p],
    "octo_head_fwd_noalloc": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                              _f32, _f32, _f32, _i32, _p, _p, _p, _p, _i64, _p],
    "octo_head_bwd": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                      _f32, _f32, _f32, _i32, _p, _p, _p, _i64, _i32, _p, _i32, _p, _sz, _p],
    "octo_head_step_grpo": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                            _f32, _f32, _f32, _i32, _p, _p, _p, _p, _i64, ctypes.POINTER(GrpoTail),
                            _p, _i64, _i32, _p, _i32, _p, _sz, _p],
    "octo_head_step_grpo_pairs": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                                  _f32, _f32, _f32, _i32, _p, _p, _i64, _p, _i64, ctypes.POINTER(GrpoTail),
                                  _p, _i64, _i32, _p, _i32, _p, _sz, _p],
    "octo_columns_fwd": [_p, _i64, _i32, _p, _i64, _i32, _f32, _p, _p, _p],
    "octo_columns_bwd": [_p, _i64, _i32, _p, _i64, _i32, _f32, _p, _p, _p, _i64, _p],
    "octo_pairs_expand": [_p, _i64, _i32, _p, _i64, _p, _p],
    "octo_pairs_grad": [_p, _i64, _i32, _p, _i64, _p, _p],
    "octo_rows_scatter": [_p, _i64, _i32, _p, _p, _i64, _i32, _p, _i64, _i32, _i32, _p],
    "octo_gather_f32": [_p, _i64, _p, _p, _i64, _p, _p],
    "octo_scale_add": [_p, _p, _i32, _i64, _p, _p, _p],
    "octo_grpo_fit": [_p, _i64, _p, _p, _i64, _p, _f32, _p, _p, _p, _p, _p],
    "octo_label_pairs_workspace_bytes": [_i64, _i64, ctypes.POINTER(_sz)],
    "octo_label_pairs": [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _i32, _p, _sz, _p],
    "octo_quantise_fp8_rows": [_p, _i64, _i32, _i64, _i32, _p, _i64, _p, _p],
    "octo_grpo_workspace_bytes": [ctypes.POINTER(_sz)],
    "octo_grpo_grad": [_p, _p, _p, _p, _p, _i64, _f32, _f32, _f32, _p, _p, _p, _sz, _p],
}
_RESTYPES = {"octo_version": ctypes.c_char_p, "octo_last_error": ctypes.c_char_p}

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """The loaded library with every signature bound. Raises RuntimeError when it has not been built."""
    global _lib
    # torch first: the library binds libamdhip64 by soname, so in a torch process it must resolve to the
    # HIP runtime torch already loaded (one runtime per process)
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(f"{path} is missing: build it with `python -m octopus_amd.build` "
                                   "(the LM head has no non-HIP GPU path)")
            lib = ctypes.CDLL(path)
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def last_error() -> str:
    return load().octo_last_error().decode(errors="replace")


def call(name: str, *args) -> None:
    """Call an entry point; raise on a non-zero status."""
    rc = getattr(load(), name)(*args)
    if rc == OK:
        return
    msg = f"{name}: {last_error()}"
    if rc in (EINVAL, EWORKSPACE):
        raise ValueError(msg)
    if rc == EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(f"{msg} (status {rc})")


def workspace_bytes(n_max: int, d: int, V: int, w_dtype: int, flags: int) -> int:
    out = _sz(0)
    call("octo_head_workspace_bytes", n_max, d, V, w_dtype, flags, ctypes.byref(out))
    return out.value


def bwd_plan(n_max: int, d: int, V: int, w_dtype: int, flags: int, ws_bytes: int) -> tuple[int, int, int, int]:
    """(rows per pass, passes, vocabulary columns per chunk, chunks) that octo_head_bwd runs in ws_bytes; with
    WS_STEP in flags, octo_head_step_grpo's (rows per pass, passes, V rounded up to 256, 1)."""
    out = (_i64 * 4)()
    call("octo_head_bwd_plan", n_max, d, V, w_dtype, flags, ws_bytes, out)
    return tuple(out)


def timing_read(kernel: str) -> tuple[int, float]:
    """(launches, summed ms) of one kernel name recorded by the timing hook (octo_timing_enable)."""
    n, ms = _i32(0), ctypes.c_double(0.0)
    call("octo_timing_read", kernel.encode(), ctypes.byref(n), ctypes.byref(ms))
    return n.value, ms.value


def grpo_workspace_bytes() -> int:
    out = _sz(0)
    call("octo_grpo_workspace_bytes", ctypes.byref(out))
    return out.value
