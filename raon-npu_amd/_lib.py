"""ctypes binding of librmoe.so (the C ABI declared in include/raon_moe.h).

The library is loaded from this package directory.  There is no fallback: if it
is missing or does not load, ``load()`` raises, and so does every product entry
point that needs it.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librmoe.so"

RMOE_OK = 0
RMOE_EINVAL = 1
RMOE_ENOTFOUND = 2
RMOE_EDEVICE = 3
RMOE_ENOMEM = 4

ACT_SITU = 0
ACT_SWIGLU = 1
SCORE_SIGMOID = 0
SCORE_SOFTMAX = 1
FMT_Q4NX = 0
FMT_BFP16 = 1
BUNDLE_B1 = 1
BUNDLE_B2 = 2
PART_GATE_UP = 3
PART_DOWN = 2

_p = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t
_pi = C.POINTER(C.c_int)

# name -> argtypes; every function returns int unless listed in _RESTYPES.
SIGNATURES: dict[str, list] = {
    "rmoe_last_error": [],
    "rmoe_version": [],
    "rmoe_create": [_i, C.POINTER(_p)],
    "rmoe_destroy": [_p],
    "rmoe_synchronize": [_p],
    "rmoe_stream": [_p],
    "rmoe_matrix_upload": [_p, _p, _sz, _i, _i, _pi],
    "rmoe_matrix_quantize_dev": [_p, _p, _i, _i, _pi, _p],
    "rmoe_matrix_download": [_p, _i, _p, _sz],
    "rmoe_matrix_free": [_p, _i],
    "rmoe_matrix_shape": [_p, _i, _pi, _pi],
    "rmoe_matrix_upload_bfp16": [_p, _p, _sz, _i, _i, _pi],
    "rmoe_matrix_format": [_p, _i, _pi],
    "rmoe_matrix_upload_q4k": [_p, _p, _sz, _i, _i, _pi],
    "rmoe_linear": [_p, _i, _p, _i, _i, _p],
    "rmoe_linear_dev": [_p, _i, _p, _i, _p, _p],
    "rmoe_reserve_linear": [_p, _i, _i],
    "rmoe_layer_create": [_p, _i, _i, _i, _i, _i, _i],
    "rmoe_reserve": [_p, _i, _i],
    "rmoe_layer_upload_experts": [_p, _i, _p, _sz, _p, _sz],
    "rmoe_layer_upload_expert_q4k": [_p, _i, _i, _i, _p, _sz],
    "rmoe_layer_create_d": [_p, _i, _i, _i, _i, _i],
    "rmoe_layer_upload_d": [_p, _i, _i, _i, _i, _p, _sz],
    "rmoe_layer_quantize_expert_dev": [_p, _i, _i, _p, _p, _p],
    "rmoe_layer_synthesize_dev": [_p, _i, C.c_uint64, _f, _p],
    "rmoe_layer_download_expert": [_p, _i, _i, _p, _sz, _p, _sz],
    "rmoe_layer_expert_matrix": [_p, _i, _i, _i, _pi],
    "rmoe_layer_set_router": [_p, _i, _p, _p, _i, _i, _f],
    "rmoe_layer_set_router_dev": [_p, _i, _p, _p, _i, _i, _f],
    "rmoe_layer_free": [_p, _i],
    "rmoe_route": [_p, _i, _p, _i, _p, _p, _p],
    "rmoe_moe_experts": [_p, _i, _p, _p, _p, _i, _i, _f, _f, _p],
    "rmoe_moe_experts_dev": [_p, _i, _p, _p, _p, _i, _i, _f, _f, _p, _p],
    "rmoe_moe_experts_static_dev": [_p, _i, _p, _p, _p, _i, _i, _f, _f, _p, _p],
    "rmoe_moe_decode_dev": [_p, _i, _p, _p, _i, _i, _f, _f, _p, _p, _p],
    "rmoe_moe_decode_stage_dev": [_p, _i, _i, _p, _p, _i, _i, _f, _f, _p],
    "rmoe_reserve_decode_stack": [_p, _p, _i],
    "rmoe_set_stack_wait_limit": [_p, C.c_uint],
    "rmoe_moe_decode_stack_dev": [_p, _p, _i, _p, _p, _i, _i, _f, _f, _p, _p, _p],
    "rmoe_moe_decode_stack": [_p, _p, _i, _p, _p, _i, _i, _f, _f, _p, _p],
    "rmoe_moe_decode": [_p, _i, _p, _p, _i, _i, _f, _f, _p, _p],
    "rmoe_dispatch": [_p, _p, _i, _i, _i, _p, _p],
    "rmoe_moe_experts_grouped": [_p, _i, _p, _i, _p, _p, _p, _i, _f, _f, _p, _p],
    "rmoe_moe_prefill_dev": [_p, _i, _p, _i, _p, _i, _i, _f, _f, _p, _p, _p],
    "rmoe_moe_experts_grouped_dev": [_p, _i, _p, _i, _p, _p, _p, _i, _f, _f, _p, _p, _p],
}
_RESTYPES = {"rmoe_last_error": C.c_char_p, "rmoe_version": C.c_char_p, "rmoe_stream": _p}


class RmoeError(RuntimeError):
    """Device-side failure (RMOE_EDEVICE / RMOE_ENOMEM)."""


_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load librmoe.so once and bind every exported entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RmoeError(
            f"{LIB_PATH} is missing: build it with `python raon-npu_amd/build.py` "
            "(the HIP library is required; there is no CPU fallback)"
        )
    lib = C.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, C.c_int)
    _lib = lib
    return lib


def check(status: int) -> None:
    """Map a status code to the reference's exception types (npu/backend.py conventions)."""
    if status == RMOE_OK:
        return
    msg = load().rmoe_last_error().decode(errors="replace")
    if status == RMOE_EINVAL:
        raise ValueError(msg)
    if status == RMOE_ENOTFOUND:
        raise KeyError(msg)
    raise RmoeError(msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def ptr(a) -> int | None:
    """Raw pointer of a NumPy array or a torch tensor (None passes NULL)."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data
