"""ctypes bindings for libtnpa.so: the public C ABI (include/tnpa.h: polynomial attention; include/tnce.h: the
fused cross-entropy epilogues) and the internal launch-level entry points (csrc/tnpa_internal.h) that the benchmark
and the tests use.

The library must be built in-tree (``python -m tensor_train_ing_amd.build``); there is no fallback: loading fails
loudly when the shared library is missing.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtnpa.so"
ABI_VERSION = 4

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_LAUNCH = 0, 1, 2, 3
BF16, F32, F16 = 0, 1, 2
SIGNED_PRODUCT, OFFSET_SQUARE, LOWER_DEGREE_MIX, POWER = 0, 1, 2, 3
CE_BF16, CE_F32, CE_F16, CE_F64 = 0, 1, 2, 3


class Tensor(ctypes.Structure):
    """tnpa_tensor_t"""
    _fields_ = [("data", ctypes.c_void_p), ("stride_b", ctypes.c_int64), ("stride_h", ctypes.c_int64),
                ("stride_t", ctypes.c_int64)]


class Problem(ctypes.Structure):
    """tnpa_problem_t"""
    _fields_ = [("batch", ctypes.c_int32), ("heads", ctypes.c_int32), ("seq_len", ctypes.c_int32),
                ("head_dim_k", ctypes.c_int32), ("head_dim_v", ctypes.c_int32), ("kind", ctypes.c_int32),
                ("degree", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("q1", Tensor), ("k1", Tensor), ("q2", Tensor), ("k2", Tensor), ("v", Tensor),
                ("doc_start", ctypes.c_void_p), ("query_end", ctypes.c_void_p), ("row_scale", ctypes.c_void_p),
                ("coef", ctypes.c_void_p), ("offset", ctypes.c_void_p), ("score_norms", ctypes.c_void_p),
                ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p)]


class Grads(ctypes.Structure):
    """tnpa_grads_t"""
    _fields_ = [("dout", Tensor), ("dq1", Tensor), ("dk1", Tensor), ("dq2", Tensor), ("dk2", Tensor),
                ("dv", Tensor), ("dpar", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_int64)]


# public ABI (include/tnpa.h, include/tnce.h)
_SIGNATURES = {
    "tnpa_abi_version": (ctypes.c_int, []),
    "tnpa_last_error": (ctypes.c_char_p, []),
    "tnpa_doc_bounds": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "tnpa_forward": (ctypes.c_int, [ctypes.POINTER(Problem), ctypes.POINTER(Tensor), ctypes.c_void_p]),
    "tnpa_rope": (ctypes.c_int, [ctypes.POINTER(Tensor), ctypes.POINTER(Tensor), ctypes.c_int32, ctypes.c_int32,
                                 ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_int32, ctypes.c_void_p]),
    "tnpa_backward_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(Problem)]),
    "tnpa_backward": (ctypes.c_int, [ctypes.POINTER(Problem), ctypes.POINTER(Grads), ctypes.c_void_p]),
    "tnpa_backward_noalloc": (ctypes.c_int, [ctypes.POINTER(Problem), ctypes.POINTER(Grads), ctypes.c_void_p]),
    "tnce_forward_chunk": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "tnce_accumulate": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                       ctypes.c_void_p]),
    "tnce_backward_chunk": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p]),
}
# internal entry points (csrc/tnpa_internal.h): the backward's launches one by one, and its plan options
_INTERNAL = {
    "tnpa_x_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(Problem), ctypes.c_int32]),
    "tnpa_x_launches": (ctypes.c_int32, [ctypes.POINTER(Problem), ctypes.c_int32]),
    "tnpa_x_launch_name": (ctypes.c_char_p, [ctypes.POINTER(Problem), ctypes.c_int32, ctypes.c_int32]),
    "tnpa_x_backward": (ctypes.c_int, [ctypes.POINTER(Problem), ctypes.POINTER(Grads), ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_void_p]),
}
X_PRESCALE_ON, X_PRESCALE_OFF, X_DS_OFF = 1, 2, 4

_LIB = None


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Loads (once) and returns libtnpa.so with argument types set; raises if it is missing or mismatched."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build the HIP library first (python -m tensor_train_ing_amd.build). "
                           "There is no CPU fallback for the HIP attention operator.")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in {**_SIGNATURES, **_INTERNAL}.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.tnpa_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {v}, expected {ABI_VERSION}; rebuild the library")
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    """Maps a nonzero tnpa_status to the Python exception the reference operator would raise."""
    if rc == OK:
        return
    msg = (_LIB or load()).tnpa_last_error().decode(errors="replace")
    if rc in (ERR_INVALID, ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")
