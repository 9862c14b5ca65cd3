"""ctypes + numpy front end of the CPU oracle (oracle/w4a8_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. The product package never
imports it.

Arrays follow the reference's names: a weight is codes[M][K] (int4 values held
in int8) with scales[M][K/group] (uint16 FP16 bits, optionally carrying the
zero point in the low nibble); activations are q[T][K] int8 with
scale[T][K/32] (block 32) or [T] (per token) and sum[T][K/32]; s4 activations
of the W4A4 GEMM are q[T][K] codes in [-7, 7] with scale and sum [T][K/64]
(block 64).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libw4a8_oracle.so")

SCALE_FP16 = 0
SCALE_FP16_ZP4 = 1
SCALE_S8 = 2
VAR_GEMV = 0
VAR_FANOUT = 1
VAR_GEMM = 2

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (g++, no GPU toolchain needed)."""
    cmd = ["make", "-s", "-C", HERE]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)
    return LIB_PATH


class _Weight(C.Structure):
    _fields_ = [("M", C.c_int), ("K", C.c_int), ("group", C.c_int), ("scale_enc", C.c_int),
                ("codes", C.c_void_p), ("scales", C.c_void_p)]


class _Act(C.Structure):
    _fields_ = [("T", C.c_int), ("K", C.c_int), ("block", C.c_int),
                ("q", C.c_void_p), ("scale", C.c_void_p), ("sum", C.c_void_p)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        sigs = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_e2m3": (C.c_float, [C.c_uint32]),
            "orc_e2m3_code_at": (C.c_uint32, [P, C.c_int, C.c_int, C.c_int]),
            "orc_f32_to_f16_n": (None, [P, P, C.c_size_t]),
            "orc_f16_to_f32_n": (None, [P, P, C.c_size_t]),
            "orc_f32_to_bf16_n": (None, [P, P, C.c_size_t]),
            "orc_quantize_act": (C.c_int, [P, C.c_int, C.c_int, C.c_int, P, P, P]),
            "orc_quantize_act_s4": (C.c_int, [P, C.c_int, C.c_int, P, P, P]),
            "orc_silu_mul": (None, [P, P, P, C.c_int]),
            "orc_rmsnorm": (None, [P, P, C.c_int, C.c_float, P]),
            "orc_fit_int4_asym": (C.c_uint16, [P, C.c_int, C.c_int, C.c_int, P]),
            "orc_repack_e2m3": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, P]),
            "orc_fit_int8": (C.c_uint16, [P, C.c_int, C.c_int]),
            "orc_repack_e2m3_s8": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, P, P]),
            "orc_pack_ref_layout": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, P, P]),
            "orc_unpack_ref_layout": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, P, P]),
            "orc_gemv_splits": (C.c_int, [C.c_int]),
            "orc_gemm_splits": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int]),
            "orc_segment_splits": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]),
            "orc_partials": (C.c_int, [P, P, P]),
            "orc_project": (C.c_int, [P, P, C.c_int, P, C.c_int, P, C.c_int, P, C.c_int, C.c_int]),
            "orc_num_threads": (C.c_int, []),
            "orc_set_num_threads": (None, [C.c_int]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- conversions -----------------------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = _c(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---- activation side -------------------------------------------------------

def quantize_act(x, block: int):
    """x[T][K] fp32 -> (q[T][K] int8, scale, sum[T][K/32])."""
    x = _c(x, np.float32)
    T, K = x.shape
    q = np.empty((T, K), np.int8)
    scale = np.empty((T, K // 32) if block == 32 else (T,), np.float32)
    s = np.empty((T, K // 32), np.int32)
    rc = lib().orc_quantize_act(_ptr(x), T, K, block, _ptr(q), _ptr(scale), _ptr(s))
    if rc:
        raise ValueError(f"orc_quantize_act rc={rc}")
    return q, scale, s


def quantize_act_s4(x):
    """x[T][K] fp32 -> (q[T][K] int8 in [-7, 7], scale[T][K/64], sum[T][K/64])."""
    x = _c(x, np.float32)
    T, K = x.shape
    q = np.empty((T, K), np.int8)
    scale = np.empty((T, K // 64), np.float32)
    s = np.empty((T, K // 64), np.int32)
    rc = lib().orc_quantize_act_s4(_ptr(x), T, K, _ptr(q), _ptr(scale), _ptr(s))
    if rc:
        raise ValueError(f"orc_quantize_act_s4 rc={rc}")
    return q, scale, s


def silu_mul(gate, up) -> np.ndarray:
    g, u = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty(g.shape, np.float32)
    lib().orc_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def rmsnorm(x, w_bf16, eps: float) -> np.ndarray:
    x, w = _c(x, np.float32), _c(w_bf16, np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().orc_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
    return out


# ---- weight side -----------------------------------------------------------

def fit_int4_asym(wf, reserve_nibble: bool = True, contract: bool = True):
    wf = _c(wf, np.float32)
    z = np.zeros(1, np.int32)
    sh = lib().orc_fit_int4_asym(_ptr(wf), wf.size, int(reserve_nibble), int(contract), _ptr(z))
    return int(sh), int(z[0])


def repack_e2m3(payload, block_scale_inv, scale_cols: int, M: int, K: int, mode: int,
                contract: bool = True):
    payload = _c(payload, np.uint8)
    bs = _c(block_scale_inv, np.float32)
    group = {0: 32, 1: 16, 2: 64}[mode]
    codes = np.empty((M, K), np.int8)
    scales = np.empty((M, K // group), np.uint16)
    rc = lib().orc_repack_e2m3(_ptr(payload), _ptr(bs), scale_cols, M, K, mode, int(contract),
                               _ptr(codes), _ptr(scales))
    if rc:
        raise ValueError(f"orc_repack_e2m3 rc={rc}")
    return codes, scales


def fit_int8(wf, contract: bool = True) -> int:
    wf = _c(wf, np.float32)
    return int(lib().orc_fit_int8(_ptr(wf), wf.size, int(contract)))


def repack_e2m3_s8(payload, block_scale_inv, scale_cols: int, M: int, K: int,
                   contract: bool = True):
    """W8A8 tier: int8 codes [M][K] and plain FP16 scales [M][K/32]."""
    payload = _c(payload, np.uint8)
    bs = _c(block_scale_inv, np.float32)
    codes = np.empty((M, K), np.int8)
    scales = np.empty((M, K // 32), np.uint16)
    rc = lib().orc_repack_e2m3_s8(_ptr(payload), _ptr(bs), scale_cols, M, K, int(contract),
                                  _ptr(codes), _ptr(scales))
    if rc:
        raise ValueError(f"orc_repack_e2m3_s8 rc={rc}")
    return codes, scales


def pack_ref_layout(codes, scales, group: int):
    codes, scales = _c(codes, np.int8), _c(scales, np.uint16)
    M, K = codes.shape
    rc_codes = np.empty(M * K // 2, np.uint8)
    rc_scales = np.empty(M * (K // group), np.uint16)
    rc = lib().orc_pack_ref_layout(_ptr(codes), _ptr(scales), M, K, group, _ptr(rc_codes),
                                   _ptr(rc_scales))
    if rc:
        raise ValueError(f"orc_pack_ref_layout rc={rc}")
    return rc_codes, rc_scales


def unpack_ref_layout(ref_codes, ref_scales, M: int, K: int, group: int):
    ref_codes, ref_scales = _c(ref_codes, np.uint8), _c(ref_scales, np.uint16)
    codes = np.empty((M, K), np.int8)
    scales = np.empty((M, K // group), np.uint16)
    rc = lib().orc_unpack_ref_layout(_ptr(ref_codes), _ptr(ref_scales), M, K, group,
                                     _ptr(codes), _ptr(scales))
    if rc:
        raise ValueError(f"orc_unpack_ref_layout rc={rc}")
    return codes, scales


# ---- split plans -----------------------------------------------------------

def gemv_splits(groups: int) -> int:
    return lib().orc_gemv_splits(groups)


def gemm_splits(rgroups: int, tgroups: int, ktiles: int, forced: int = 0) -> int:
    return lib().orc_gemm_splits(rgroups, tgroups, ktiles, forced)


def segment_splits(T: int, M: int, K: int, offsets=None, forced: int = 0) -> np.ndarray:
    out = np.empty(T, np.int32)
    if offsets is None:
        rc = lib().orc_segment_splits(None, 0, T, M, K, forced, _ptr(out))
    else:
        off = _c(offsets, np.int32)
        rc = lib().orc_segment_splits(_ptr(off), len(off) - 1, T, M, K, forced, _ptr(out))
    if rc:
        raise ValueError(f"orc_segment_splits rc={rc}")
    return out


# ---- projection ------------------------------------------------------------

def _structs(codes, scales, group, scale_enc, q, scale, asum, block):
    M, K = codes.shape
    T = q.shape[0]
    w = _Weight(M, K, group, scale_enc, _ptr(codes), _ptr(scales))
    a = _Act(T, K, block, _ptr(q), _ptr(scale), _ptr(asum))
    return w, a


def partials(codes, scales, group, scale_enc, q, scale, asum, block) -> np.ndarray:
    codes, scales = _c(codes, np.int8), _c(scales, np.uint16)
    q, scale = _c(q, np.int8), _c(scale, np.float32)
    asum = None if asum is None else _c(asum, np.int32)
    w, a = _structs(codes, scales, group, scale_enc, q, scale, asum, block)
    unit = 32 if block == 32 else 64 if block == 64 else group
    P = np.empty((q.shape[0], codes.shape[0], codes.shape[1] // unit), np.int32)
    rc = lib().orc_partials(C.byref(w), C.byref(a), _ptr(P))
    if rc:
        raise ValueError(f"orc_partials rc={rc}")
    return P


def project(codes, scales, group, scale_enc, q, scale, asum, block, variant, splits,
            contract=True, residual=None, out_bf16=False, rows=None) -> np.ndarray:
    """y[T][M]; `splits` is an int (all tokens) or a per-token int array.

    rows=(begin, end) computes only that row range (other entries are zero).
    """
    codes, scales = _c(codes, np.int8), _c(scales, np.uint16)
    q, scale = _c(q, np.int8), _c(scale, np.float32)
    asum = None if asum is None else _c(asum, np.int32)
    T, M = q.shape[0], codes.shape[0]
    sp = np.full(T, splits, np.int32) if np.isscalar(splits) else _c(splits, np.int32)
    res = None if residual is None else _c(residual, np.float32)
    y = np.zeros((T, M), np.uint16 if out_bf16 else np.float32)
    rb, re = (0, M) if rows is None else rows
    w, a = _structs(codes, scales, group, scale_enc, q, scale, asum, block)
    rc = lib().orc_project(C.byref(w), C.byref(a), variant, _ptr(sp), int(contract), _ptr(res),
                           int(out_bf16), _ptr(y), rb, re)
    if rc:
        raise ValueError(f"orc_project rc={rc}")
    return y


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(n)


def num_threads() -> int:
    return lib().orc_num_threads()
