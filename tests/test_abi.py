"""C-ABI checks that need no GPU: libkxw4.so loads, exports every function
include/kxw4.h declares, its split plans equal the oracle's restatement of
the reference heuristics, and argument checks return the reference's codes
before any HIP call is made."""
import ctypes as C
import os
import re

import pytest

from knivesysl_xe_amd import _lib
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kxw4_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared("kxw4.h")
    assert len(names) >= 18
    for name in names:
        assert hasattr(L, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    assert L.kxw4_abi_version() == 1


def test_split_plans_match_oracle():
    L = _lib.lib()
    for g in list(range(0, 70)) + [255, 256, 320, 2176, 4095, 4096, 10000]:
        assert L.kxw4_gemv_splits(g) == O.gemv_splits(g)
    for rg in (1, 3, 16, 64, 320, 1088, 2048, 2176):
        for tg in (1, 2, 3, 8, 64, 256):
            for kt in (1, 2, 4, 8, 16, 160, 544):
                for forced in (0, 1, 2, 3, 4, 8, 16, 32):
                    assert L.kxw4_gemm_splits(rg, tg, kt, forced) == O.gemm_splits(rg, tg, kt, forced)


def test_sizes():
    L = _lib.lib()
    assert L.kxw4_code_bytes(17408, 5120) == 44564480
    assert L.kxw4_scale_count(5120, 17408, 64) == 5120 * 272
    assert L.kxw4_scale_count(5120, 17408, 48) == 0


def W(M=256, K=1024, group=128, enc=0, codes=1, scales=1):
    return _lib.Weight(M, K, group, enc, codes, scales)


def A(T=8, K=1024, block=0, q=1, scale=1, s=1):
    return _lib.Act(T, K, block, q, scale, s)


def test_argument_checks_return_reference_codes():
    L = _lib.lib()
    y = C.c_void_p(1)
    # x_gemv_w4a8_prepared_impl: -1 weight/output missing (kernels_dpas.cpp:1633)
    assert L.kxw4_gemv(None, C.byref(A()), y, 0, None, 0, None) == _lib.EARG
    assert L.kxw4_gemv(C.byref(W(codes=0)), C.byref(A()), y, 0, None, 0, None) == _lib.EARG
    assert L.kxw4_gemv(C.byref(W()), C.byref(A()), None, 0, None, 0, None) == _lib.EARG
    # shape checks (repack: M % 16, K % 128; kernels_dpas.cpp:406)
    assert L.kxw4_gemv(C.byref(W(M=250)), C.byref(A()), y, 0, None, 0, None) == _lib.ESHAPE
    assert L.kxw4_gemv(C.byref(W(K=1000)), C.byref(A(K=1000)), y, 0, None, 0, None) == _lib.ESHAPE
    assert L.kxw4_gemv(C.byref(W(group=48)), C.byref(A()), y, 0, None, 0, None) == _lib.ESHAPE
    # -2 unprepared / mismatched activation (kernels_dpas.cpp:1636)
    assert L.kxw4_gemv(C.byref(W()), C.byref(A(K=2048)), y, 0, None, 0, None) == _lib.ESHAPE
    assert L.kxw4_gemv(C.byref(W()), C.byref(A(q=0)), y, 0, None, 0, None) == _lib.ESHAPE
    assert L.kxw4_gemv(C.byref(W()), C.byref(A(T=65)), y, 0, None, 0, None) == _lib.ESHAPE
    assert L.kxw4_gemv(C.byref(W()), C.byref(A()), y, 0, None, 3, None) == _lib.ESHAPE
    # zero-point weights need the exact activation sums
    assert L.kxw4_gemv(C.byref(W(enc=1)), C.byref(A(s=0)), y, 0, None, 0, None) == _lib.EPREP
    assert L.kxw4_gemv(C.byref(W(enc=7)), C.byref(A()), y, 0, None, 0, None) == _lib.ETIER


def test_fanout_checks():
    L = _lib.lib()
    w1, w2 = W(), W(K=2048)
    arr = (C.POINTER(_lib.Weight) * 2)(C.pointer(w1), C.pointer(w2))
    ys = (C.c_void_p * 2)(1, 1)
    a = A()
    # kernels_dpas.cpp:947-967: -1 bad set, -2 mixed K/tier, -3 unprepared
    assert L.kxw4_gemv_fanout(arr, ys, 0, C.byref(a), 0, None) == _lib.EARG
    assert L.kxw4_gemv_fanout(arr, ys, 5, C.byref(a), 0, None) == _lib.EARG
    assert L.kxw4_gemv_fanout(arr, ys, 2, C.byref(a), 0, None) == _lib.ESHAPE
    w3 = W(group=64)
    arr2 = (C.POINTER(_lib.Weight) * 2)(C.pointer(w1), C.pointer(w3))
    assert L.kxw4_gemv_fanout(arr2, ys, 2, C.byref(a), 0, None) == _lib.ESHAPE
    arr1 = (C.POINTER(_lib.Weight) * 1)(C.pointer(w1))
    assert L.kxw4_gemv_fanout(arr1, ys, 1, C.byref(A(q=0)), 0, None) == _lib.EPREP
    assert L.kxw4_gemv_fanout(arr1, ys, 1, None, 0, None) == _lib.EPREP


def test_gemm_offsets_checks():
    L = _lib.lib()
    y = C.c_void_p(1)
    w, a = W(), A(T=24)

    def call(off, nseg):
        arr = None if off is None else (C.c_int * len(off))(*off)
        return L.kxw4_gemm(C.byref(w), C.byref(a), y, 0, None, arr, nseg, 0, None)

    # kernels_dpas.cpp:1349-1356: offsets must start at 0, end at T, grow
    assert call([1, 8, 24], 2) == _lib.ESHAPE
    assert call([0, 8, 20], 2) == _lib.ESHAPE
    assert call([0, 8, 8, 24], 3) == _lib.ESHAPE
    assert call([0] * 10 + [24], 10) == _lib.ESHAPE
    assert call(None, 2) == _lib.ESHAPE
    assert L.kxw4_gemm(None, C.byref(a), y, 0, None, None, 0, 0, None) == _lib.EARG
    assert L.kxw4_gemm(C.byref(w), C.byref(A(T=0)), y, 0, None, None, 0, 0, None) == _lib.ESHAPE
    assert L.kxw4_gemm(C.byref(w), C.byref(a), y, 5, None, None, 0, 0, None) == _lib.ESHAPE


def test_weight_and_quantizer_checks():
    L = _lib.lib()
    p = C.c_void_p(1)
    assert L.kxw4_pack_weight(None, p, 16, 128, 32, p, p, None) == _lib.EARG
    assert L.kxw4_pack_weight(p, p, 24, 128, 32, p, p, None) == _lib.ESHAPE
    assert L.kxw4_import_ref_weight(p, p, 16, 128, 128, p, p, None) == _lib.ESHAPE
    # x_w4_repack_weight_mode: -2 shape (its -3, an odd K32 tile count for
    # K64, cannot follow a passed K % 128 check); modes 0 (K32), 1 (K16) and
    # 2 (K64) exist
    assert L.kxw4_repack_e2m3(p, p, 4, 16, 100, 0, p, p, None) == _lib.ESHAPE
    assert L.kxw4_repack_e2m3(p, p, 3, 16, 128, 0, p, p, None) == _lib.ESHAPE
    assert L.kxw4_repack_e2m3(p, p, 4, 16, 128, 3, p, p, None) == _lib.ESHAPE
    # W8 weights keep K32 scales; K16 weights FP16|zp scales (checked before
    # any launch)
    w8 = _lib.Weight(16, 128, 64, _lib.SCALE_W8, 1, 1)
    w16 = _lib.Weight(16, 128, 16, _lib.SCALE_FP16, 1, 1)
    assert L.kxw4_unpack_weight(C.byref(w8), p, p, None) == _lib.ESHAPE
    assert L.kxw4_unpack_weight(C.byref(w16), p, p, None) == _lib.ESHAPE
    assert L.kxw4_quantize_act(None, 0, 1, 128, 0, p, p, p, None) == _lib.EARG
    assert L.kxw4_quantize_act(p, 0, 1, 96, 0, p, p, p, None) == _lib.ESHAPE
    assert L.kxw4_quantize_act(p, 0, 1, 128, 16, p, p, p, None) == _lib.ESHAPE
    assert L.kxw4_quantize_act(p, 2, 1, 128, 0, p, p, p, None) == _lib.ESHAPE
    assert L.kxw4_error_string(_lib.ETIER).decode() == "tier not built by this library"


@pytest.mark.parametrize("name", ["cfg0", "cfg1", "cfg2_m1", "cfg2_m512", "cfg3", "cfg4"])
def test_algorithmic_bytes_match_baseline_table(name):
    from knivesysl_xe_amd import workloads
    want = {"cfg0": 8675328, "cfg1": 92553216, "cfg2_m1": 47405056, "cfg2_m512": 66748416,
            "cfg3": 65945600, "cfg4": 664396800}
    assert workloads.CONFIGS[name].algorithmic_bytes() == want[name]


def test_set_option_checks_names_ranges_and_restores():
    import ctypes as C
    from knivesysl_xe_amd import ops
    L = _lib.lib()
    prev = C.c_int(-99)
    assert L.kxw4_set_option(b"no_such_option", 0, None) == -1
    assert L.kxw4_set_option(None, 0, None) == -1
    assert L.kxw4_set_option(b"decode_kernel", 3, None) == -2
    assert L.kxw4_set_option(b"gemm3_tile", 12, None) == -2
    assert L.kxw4_set_option(b"gemm3_tile", -2, None) == -2
    assert L.kxw4_set_option(b"gemm3_tile", -1, C.byref(prev)) == 0
    assert prev.value == -1
    with ops.option("gemm3_tile", 7):
        assert L.kxw4_set_option(b"gemm3_tile", 7, C.byref(prev)) == 0 and prev.value == 7
        with ops.option("w4a4_tile", 2):
            pass
    assert L.kxw4_set_option(b"gemm3_tile", -1, C.byref(prev)) == 0 and prev.value == -1
    assert L.kxw4_set_option(b"w4a4_tile", -1, C.byref(prev)) == 0 and prev.value == -1
    assert L.kxw4_set_option(b"gemmr_tile", 10, None) == -2
    with ops.option("gemmr_tile", 8):
        assert L.kxw4_set_option(b"gemmr_tile", 8, C.byref(prev)) == 0 and prev.value == 8
    assert L.kxw4_set_option(b"gemmr_tile", -1, C.byref(prev)) == 0 and prev.value == -1
    with pytest.raises(_lib.KxError):
        with ops.option("rowwave_spw", 17):
            pass
