"""ctypes binding of ``libjangq_amd.so`` (the C ABI declared in ``include/jangq_amd.h``).

The library is loaded from the package directory only. There is no fallback: if it is
missing the import of any operator raises, so a run can never silently compute on the CPU.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libjangq_amd.so"

JQ_F32, JQ_BF16, JQ_F16 = 0, 1, 2

#: Every symbol the header declares, with (restype, argtypes).
_P = C.c_void_p
_I = C.c_int
_L = C.c_int64
SIGNATURES = {
    "jq_abi_version": (_I, []),
    "jq_status_string": (C.c_char_p, [_I]),
    "jq_unpack": (_I, [_P, _I, _L, _L, _P, _P]),
    "jq_dequantize": (_I, [_P, _P, _P, _I, _I, _I, _L, _L, _P, _I, _P]),
    "jq_quantize": (_I, [_P, _I, _I, _I, _L, _L, _P, _P, _P, _I, _P]),
    "jq_expand_1bit_to_2bit": (_I, [_P, _L, _P, _P]),
    "jq_quantized_matmul": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _L, _L, _L, _P, _I, _P]),
    "jq_quantized_matmul_workspace_size": (_L, [_L, _L, _L, _I, _I, _I, _I]),
    "jq_quantized_matmul_ws": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _L, _L, _L, _P, _I, _P, _L, _P]),
    "jq_quantized_matmul_multi": (
        _I,
        [_I, _P, _I, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P],
    ),
    "jq_moe_route": (_I, [_P, _L, _L, _I, _I, _P, _P, _P]),
    "jq_gather_workspace_size": (_L, [_L, _L, _L]),
    "jq_gather_qmm": (
        _I,
        [_P, _I, _L, _L, _P, _P, _P, _I, _I, _I, _L, _L, _L, _P, _P, _L, _I, _P, _I, _P, _L, _P],
    ),
    "jq_moe_combine": (_I, [_P, _P, _P, _L, _I, _L, _P, _I, _P]),
    "jq_quantized_swiglu": (
        _I,
        [_P, _I, _L, _L, _L, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _I, _P],
    ),
    "jq_switch_glu": (
        _I,
        [_P, _I, _L, _L, _L, _L, _P, _I,
         _P, _P, _P, _P, _P, _P, _I,
         _P, _P, _P, _I, _I, _I, _P, _P, _I, _P, _L, _P],
    ),
    "jq_mx_dequantize": (_I, [_P, _P, _I, _L, _L, _P, _I, _P]),
    "jq_mx_quantized_matmul": (_I, [_P, _I, _P, _P, _I, _L, _L, _L, _P, _I, _P]),
    "jq_moe_experts": (
        _I,
        [_P, _I, _L, _L, _L, _L, _P, _I, _I, _P, _P,
         _P, _P, _P, _P, _P, _P, _I,
         _P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _I, _P, _L, _P],
    ),
    "jq_switch_glu_combine": (
        _I,
        [_P, _I, _L, _L, _L, _L, _P, _P, _I,
         _P, _P, _P, _P, _P, _P, _I,
         _P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _I, _P, _L, _P],
    ),
    "jq_quantized_matmul_noalloc": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _L, _L, _L, _P, _I, _P]),
    "jq_moe_route_ex": (_I, [_P, _I, _L, _L, _I, _P, _P, _P, _P]),
    "jq_mx_gather_qmm": (_I, [_P, _I, _L, _L, _P, _P, _I, _L, _L, _L, _P, _P, _L, _P, _I, _P]),
    "jq_swiglu": (_I, [_P, _P, _L, C.c_float, _P, _I, _P]),
    "jq_quantized_swiglu_ex": (
        _I,
        [_P, _I, _L, _L, _L, _P, _P, _P, _P, _P, _P, _I, _I, _I, C.c_float, _P, _P, _I, _P],
    ),
    "jq_moe_block_workspace_size": (_L, [_L, _L, _L, _L, _I, _L, _I]),
    "jq_moe_block": (
        _I,
        [_P, _I, _L, _L, _L, _L, _I, _P, _I, _P, _P, _P, _P, _L, _P, _P, _P, _P, _P,
         _P, _P, _P, _P, _L, _P],
    ),
}

JQ_SCORE = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}
JQ_COMBINE = {"after": 0, "before": 1}


class RouteOpts(C.Structure):
    """jq_route_opts (include/jangq_amd.h)."""
    _fields_ = [("score", C.c_int), ("renorm", C.c_int), ("renorm_eps", C.c_float),
                ("scaling", C.c_float), ("score_bias", C.c_void_p), ("n_group", C.c_int),
                ("topk_group", C.c_int)]


class QWeight(C.Structure):
    """jq_qweight (include/jangq_amd.h)."""
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("sb_dtype", C.c_int), ("bits", C.c_int), ("group_size", C.c_int)]


class MoeOpts(C.Structure):
    """jq_moe_opts (include/jangq_amd.h)."""
    _fields_ = [("combine", C.c_int), ("swiglu_limit", C.c_float)]


_lib: C.CDLL | None = None


class JangqError(RuntimeError):
    """Raised when the native library is missing or a launch fails."""


def lib() -> C.CDLL:
    """The loaded library (loaded once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise JangqError(
                f"{LIB_PATH} is missing: build it with `python -m jangq_amd.build` "
                "(the gfx950 kernels have no CPU fallback)"
            )
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def status_string(status: int) -> str:
    return lib().jq_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    """Map a negative jq_status to ValueError (bad arguments) or JangqError (launch)."""
    if status == 0:
        return
    msg = f"{what}: {status_string(status)} (status {status})"
    if status == -6:
        raise JangqError(msg)
    raise ValueError(msg)
