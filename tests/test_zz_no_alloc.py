"""kxw4_gemv_x_noalloc, the allocation-free x_gemv_w4a8 (its quantized
activations live in a fixed device array of the library), against the entry
points it is built from: kxw4_quantize_act (block 32) into caller buffers
followed by kxw4_gemv, bit for bit. Two calls in a row, the second on a
smaller input, so the array's contents from the first call cannot leak into
the second. Every tier the GEMV takes is covered (K32/K64 FP16|zp, K128
FP16, K16, W8), with and without a residual, F32 and BF16 activations."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from knivesysl_xe_amd import _lib, ops  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def make_weight(rng, M, K, group, enc):
    if enc == _lib.SCALE_W8:
        codes = torch.from_numpy(rng.integers(-128, 128, (M, K)).astype(np.int8)).cuda()
        sc = (np.abs(rng.standard_normal((M, K // 32))) * 0.002).astype(np.float16).view(np.int16)
        return ops.W4Weight.from_codes_s8(codes, torch.from_numpy(sc).cuda())
    codes = torch.from_numpy(rng.integers(-8, 8, (M, K)).astype(np.int8)).cuda()
    mags = (np.abs(rng.standard_normal((M, K // group))) * 0.02).astype(np.float16).view(np.uint16)
    if enc == _lib.SCALE_FP16_ZP4:
        mags = ((mags & 0xFFF0) | (rng.integers(-8, 8, mags.shape) & 0xF)).astype(np.uint16)
    return ops.W4Weight.from_codes(codes, torch.from_numpy(mags.view(np.int16)).cuda(), group, enc)


def noalloc(w, x, residual=None, dtype=torch.float32):
    T = x.shape[0]
    y = torch.empty(T, w.M, dtype=dtype, device="cuda")
    wc = w.c()
    rc = _lib.lib().kxw4_gemv_x_noalloc(
        C.byref(wc), C.c_void_p(x.data_ptr()), ops._dtype_code(x.dtype), T, C.c_void_p(y.data_ptr()),
        ops._dtype_code(dtype), None if residual is None else C.c_void_p(residual.data_ptr()),
        ops._stream())
    _lib.check("kxw4_gemv_x_noalloc", rc)
    return y


def existing(w, x, residual=None, dtype=torch.float32):
    a = ops.quantize_act(x, 32)
    return ops.gemv(w, a, dtype, residual=residual)


def bits(y):
    return y.view(torch.int16 if y.dtype == torch.bfloat16 else torch.int32).cpu().numpy()


def test_noalloc_first_call_captured_in_graph():
    # The use the entry point is for: its first call in the process (this is
    # the file's first test, and no other file calls it) is recorded into a
    # HIP graph by torch.cuda.graph, whose default capture mode fails on any
    # allocation or other call not allowed under capture. The graph is then
    # replayed on new inputs, with eager work and synchronizations between
    # the replays, and every replay is checked bit for bit against the eager
    # quantize + GEMV on the same inputs.
    rng = np.random.default_rng(11)
    L = _lib.lib()
    M, K, T = 1024, 4096, 4
    w = make_weight(rng, M, K, 32, _lib.SCALE_FP16_ZP4)
    wc = w.c()
    x = torch.zeros(T, K, device="cuda")
    res = torch.from_numpy(rng.standard_normal((T, M)).astype(np.float32)).cuda()
    y = torch.empty(T, M, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = L.kxw4_gemv_x_noalloc(C.byref(wc), C.c_void_p(x.data_ptr()), ops._dtype_code(x.dtype), T,
                                   C.c_void_p(y.data_ptr()), ops._dtype_code(y.dtype),
                                   C.c_void_p(res.data_ptr()), ops._stream())
    assert rc == 0
    for i in range(4):
        print(f"noalloc graph replay {i}", flush=True)
        x.copy_(torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)))
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        want = existing(w, x, res, torch.float32)
        torch.cuda.synchronize()
        assert np.array_equal(bits(y), bits(want)), f"replay {i}"
    del g


# (M, K, group, enc, T) pairs: the second of each pair is the smaller input
CASES = [
    ((1024, 4096, 32, _lib.SCALE_FP16_ZP4, 8), (256, 2048, 32, _lib.SCALE_FP16_ZP4, 1)),
    ((5120, 17408, 64, _lib.SCALE_FP16_ZP4, 16), (512, 4096, 64, _lib.SCALE_FP16_ZP4, 3)),
    ((2048, 5120, 128, _lib.SCALE_FP16, 4), (1024, 1024, 128, _lib.SCALE_FP16, 2)),
    ((1024, 5120, 16, _lib.SCALE_FP16_ZP4, 5), (256, 1024, 16, _lib.SCALE_FP16_ZP4, 1)),
    ((2048, 4096, 32, _lib.SCALE_W8, 8), (512, 2048, 32, _lib.SCALE_W8, 2)),
]


@pytest.mark.parametrize("first,second", CASES)
@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_quantize_then_gemv(first, second, xdtype):
    rng = np.random.default_rng(first[0] + first[1] + first[4])
    for M, K, group, enc, T in (first, second):
        print(f"noalloc M={M} K={K} group={group} enc={enc} T={T} x={xdtype}", flush=True)
        w = make_weight(rng, M, K, group, enc)
        x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).cuda().to(xdtype)
        res = torch.from_numpy(rng.standard_normal((T, M)).astype(np.float32)).cuda()
        for r in (None, res):
            for dt in (torch.float32, torch.bfloat16):
                got = noalloc(w, x, r, dt)
                want = existing(w, x, r, dt)
                torch.cuda.synchronize()
                assert np.array_equal(bits(got), bits(want)), \
                    f"M={M} K={K} group={group} enc={enc} T={T} residual={r is not None} out={dt}"


class TqWeight(C.Structure):
    # tq_qmma_weight_t as include/kxw4_compat.hpp declares it
    _fields_ = [("M", C.c_int), ("K", C.c_int), ("Mt", C.c_int), ("Kt", C.c_int),
                ("inv_scale", C.c_float), ("d_A", C.c_void_p), ("d_block_scale_inv", C.c_void_p),
                ("block_scaled", C.c_int), ("row_major", C.c_int), ("word_major", C.c_int),
                ("e2m3", C.c_int), ("e2m1", C.c_int), ("e2m3_byte", C.c_int),
                ("scale_rows", C.c_int), ("scale_cols", C.c_int),
                ("d_s4", C.c_void_p), ("d_s4_scale", C.c_void_p),
                ("s4_ready", C.c_int), ("s4_k16", C.c_int), ("s4_k64", C.c_int),
                ("d_s8", C.c_void_p), ("d_s8_scale", C.c_void_p), ("s8_ready", C.c_int)]


@pytest.mark.parametrize("group", [32, 64])
def test_noalloc_matches_x_gemv_w4a8(group):
    # the reference-signature entry point itself (x_gemv_w4a8 / _add, one
    # FP32 token, library-allocated scratch), two calls in a row, the second
    # on a smaller weight
    L = _lib.lib()
    gemv = getattr(L, "_Z11x_gemv_w4a8PK16tq_qmma_weight_tPKfPf")
    gemv_add = getattr(L, "_Z15x_gemv_w4a8_addPK16tq_qmma_weight_tPKfS3_Pf")
    for f in (gemv, gemv_add):
        f.restype = C.c_int
    rng = np.random.default_rng(group)
    for M, K in ((5120, 17408), (1024, 2048)):
        print(f"x_gemv_w4a8 M={M} K={K} group={group}", flush=True)
        w = make_weight(rng, M, K, group, _lib.SCALE_FP16_ZP4)
        tq = TqWeight()
        tq.M, tq.K, tq.Mt, tq.Kt = M, K, M // 16, K // 32
        tq.d_s4, tq.d_s4_scale = w.codes.data_ptr(), w.scales.data_ptr()
        tq.s4_ready, tq.s4_k64 = 1, 1 if group == 64 else 0
        x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).cuda()
        res = torch.from_numpy(rng.standard_normal((1, M)).astype(np.float32)).cuda()
        y_ref = torch.empty(1, M, device="cuda")
        y_add = torch.empty(1, M, device="cuda")
        torch.cuda.synchronize()
        assert gemv(C.byref(tq), C.c_void_p(x.data_ptr()), C.c_void_p(y_ref.data_ptr())) == 0
        assert gemv_add(C.byref(tq), C.c_void_p(x.data_ptr()), C.c_void_p(res.data_ptr()),
                        C.c_void_p(y_add.data_ptr())) == 0
        torch.cuda.synchronize()
        got = noalloc(w, x)
        got_add = noalloc(w, x, res)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(y_ref)), f"x_gemv_w4a8 M={M} K={K}"
        assert np.array_equal(bits(got_add), bits(y_add)), f"x_gemv_w4a8_add M={M} K={K}"


# multi-token cases checked against the CPU oracle itself: the longest K at
# the most tokens (group 64, where the W4 activations exceed one work-group's
# LDS and the K-parallel kernel runs), and T > 1 on the W8 and K16 tiers
ORACLE_CASES = [
    (5120, 17408, 64, _lib.SCALE_FP16_ZP4, 16),
    (2048, 4096, 32, _lib.SCALE_W8, 8),
    (1024, 5120, 16, _lib.SCALE_FP16_ZP4, 5),
]


@pytest.mark.parametrize("M,K,group,enc,T", ORACLE_CASES)
def test_noalloc_multi_token_matches_oracle(M, K, group, enc, T):
    from oracle import oracle as O
    O.set_num_threads(16)
    print(f"noalloc vs oracle M={M} K={K} group={group} enc={enc} T={T}", flush=True)
    rng = np.random.default_rng(M + K + T)
    if enc == _lib.SCALE_W8:
        codes = rng.integers(-128, 128, (M, K)).astype(np.int8)
        sc = (np.abs(rng.standard_normal((M, K // 32))) * 0.002).astype(np.float16).view(np.uint16)
        w = ops.W4Weight.from_codes_s8(torch.from_numpy(codes).cuda(),
                                       torch.from_numpy(sc.view(np.int16)).cuda())
        o_enc = O.SCALE_S8
    else:
        codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
        sc = (np.abs(rng.standard_normal((M, K // group))) * 0.02).astype(np.float16).view(np.uint16)
        sc = ((sc & 0xFFF0) | (rng.integers(-8, 8, sc.shape) & 0xF)).astype(np.uint16)
        w = ops.W4Weight.from_codes(torch.from_numpy(codes).cuda(),
                                    torch.from_numpy(sc.view(np.int16)).cuda(), group, enc)
        o_enc = O.SCALE_FP16_ZP4
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    q, s, sm = O.quantize_act(x, 32)
    S = O.gemv_splits(M // 16)
    for r in (None, res):
        got = noalloc(w, torch.from_numpy(x).cuda(), None if r is None else torch.from_numpy(r).cuda())
        torch.cuda.synchronize()
        want = O.project(codes, sc, group, o_enc, q, s, sm, 32, O.VAR_GEMV, S, residual=r)
        g = got.cpu().numpy()
        rel = np.max(np.abs(g.astype(np.float64) - want) / (np.abs(want.astype(np.float64)) + 1e-3))
        assert rel <= 1e-3, f"M={M} K={K} T={T} residual={r is not None}: max rel {rel}"
        assert np.array_equal(g.view(np.uint32), want.view(np.uint32)), \
            f"M={M} K={K} T={T} residual={r is not None}: not bit-exact"


def test_noalloc_limits_and_arguments():
    rng = np.random.default_rng(5)
    L = _lib.lib()
    w = make_weight(rng, 256, 1024, 32, _lib.SCALE_FP16_ZP4)
    wc = w.c()
    x = torch.zeros(32, 1024, device="cuda")
    y = torch.empty(32, 256, device="cuda")
    xp, yp = C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr())
    assert L.kxw4_gemv_x_noalloc(C.byref(wc), xp, 0, 17, yp, 0, None, None) == -2   # T > 16
    assert L.kxw4_gemv_x_noalloc(C.byref(wc), xp, 0, 0, yp, 0, None, None) == -2    # T < 1
    assert L.kxw4_gemv_x_noalloc(C.byref(wc), xp, 7, 1, yp, 0, None, None) == -2    # x dtype
    assert L.kxw4_gemv_x_noalloc(None, xp, 0, 1, yp, 0, None, None) == -1
    assert L.kxw4_gemv_x_noalloc(C.byref(wc), None, 0, 1, yp, 0, None, None) == -1
    assert L.kxw4_gemv_x_noalloc(C.byref(wc), xp, 0, 1, None, 0, None, None) == -1
    big = ops.W4Weight(256, 32768 + 128, 32, _lib.SCALE_FP16_ZP4, w.codes, w.scales)
    bc = big.c()
    assert L.kxw4_gemv_x_noalloc(C.byref(bc), xp, 0, 1, yp, 0, None, None) == -2   # K > 32768
    torch.cuda.synchronize()
