"""ctypes binding of libkxw4.so (the C ABI in include/kxw4.h).

This mirrors how the reference's Python tools reach its native library
(xpu/tools/gemm_check.py:24-31: ctypes.CDLL + explicit argtypes). Loading
fails loudly when the library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkxw4.so")

OK, EARG, ESHAPE, EPREP, ESPLIT, ETIER, EHIP = 0, -1, -2, -3, -4, -5, -6
SCALE_FP16, SCALE_FP16_ZP4, SCALE_W8 = 0, 1, 2
F32, BF16 = 0, 1


class Weight(C.Structure):
    _fields_ = [("M", C.c_int32), ("K", C.c_int32), ("group", C.c_int32),
                ("scale_enc", C.c_int32), ("codes", C.c_void_p), ("scales", C.c_void_p)]


class TqfTensor(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("kind", C.c_int32), ("M", C.c_int32), ("K", C.c_int32),
                ("scale_rows", C.c_int32), ("scale_cols", C.c_int32), ("offset", C.c_uint64),
                ("bytes", C.c_uint64)]


class Act(C.Structure):
    _fields_ = [("T", C.c_int32), ("K", C.c_int32), ("block", C.c_int32),
                ("q", C.c_void_p), ("scale", C.c_void_p), ("sum", C.c_void_p)]


# name -> (restype, argtypes); the exported C ABI, in header order
P, I, F = C.c_void_p, C.c_int, C.c_float
WP = C.POINTER(Weight)
AP = C.POINTER(Act)
SIGNATURES = {
    "kxw4_abi_version": (I, []),
    "kxw4_error_string": (C.c_char_p, [I]),
    "kxw4_set_option": (I, [C.c_char_p, I, C.POINTER(I)]),
    "kxw4_code_bytes": (C.c_size_t, [I, I]),
    "kxw4_scale_count": (C.c_size_t, [I, I, I]),
    "kxw4_gemv_splits": (I, [I]),
    "kxw4_gemm_splits": (I, [I, I, I, I]),
    "kxw4_pack_weight": (I, [P, P, I, I, I, P, P, P]),
    "kxw4_unpack_weight": (I, [WP, P, P, P]),
    "kxw4_pack_weight_s8": (I, [P, P, I, I, P, P, P]),
    "kxw4_repack_e2m3_s8": (I, [P, P, I, I, I, P, P, P]),
    "kxw4_import_ref_weight": (I, [P, P, I, I, I, P, P, P]),
    "kxw4_repack_e2m3": (I, [P, P, I, I, I, I, P, P, P]),
    "kxw4_quantize_act": (I, [P, I, I, I, I, P, P, P, P]),
    "kxw4_silu_mul_quant": (I, [P, P, P, I, I, I, P, P, P, P]),
    "kxw4_rmsnorm_quant": (I, [P, P, P, I, I, F, I, P, P, P, P]),
    "kxw4_rmsnorm": (I, [P, P, P, I, I, F, P]),
    "kxw4_quantize_act_s4": (I, [P, I, I, I, P, P, P, P]),
    "kxw4_gemv": (I, [WP, AP, P, I, P, I, P]),
    "kxw4_gemv_fanout": (I, [C.POINTER(WP), C.POINTER(P), I, AP, I, P]),
    "kxw4_gemm": (I, [WP, AP, P, I, P, C.POINTER(I), I, I, P]),
    "kxw4_gemm_fanout": (I, [C.POINTER(WP), C.POINTER(P), I, AP, I, C.POINTER(I), I, I, P]),
    "kxw4_gemm_w4a4": (I, [WP, P, P, P, I, P, I, P, P]),
    "kxw4_gemv_x_noalloc": (I, [WP, P, I, I, P, I, P, P]),
    "kxw4_tqf_open": (I, [C.c_char_p, C.POINTER(P)]),
    "kxw4_tqf_close": (None, [P]),
    "kxw4_tqf_count": (I, [P]),
    "kxw4_tqf_header": (I, [P, P, P, P]),
    "kxw4_tqf_tensor": (I, [P, I, C.POINTER(TqfTensor)]),
    "kxw4_tqf_find": (I, [P, C.c_char_p]),
    "kxw4_tqf_load_qmma": (I, [P, I, I, P, P, P]),
    "kxw4_probe_mfma_i8": (I, [I, I, P, I, C.POINTER(C.c_double), P]),
    "kxw4_probe_read": (I, [P, C.c_size_t, I, P, I, P]),
    "kxw4_probe_read_shapes": (I, []),
    "kxw4_probe_issue": (I, [I, I, I, P, I, C.POINTER(C.c_double), P]),
    "kxw4_probe_hold": (I, [P, I, P, P]),
    "kxw4_partials": (I, [WP, AP, P, P]),
}

_lib = None


class KxError(RuntimeError):
    def __init__(self, fn: str, code: int):
        self.code = code
        msg = lib().kxw4_error_string(code).decode() if _lib is not None else str(code)
        super().__init__(f"{fn} returned {code} ({msg})")


def lib():
    """Load libkxw4.so once; raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C knivesysl_xe_amd/csrc` "
                "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, rc: int) -> int:
    if rc != 0:
        raise KxError(fn, rc)
    return rc
