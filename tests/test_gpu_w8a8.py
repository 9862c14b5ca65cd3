"""Parity of the W8A8 tier (int8 weights, kernels_dpas.cpp:346-399, 771-844,
1578-1629) on the GPU with the CPU oracle: packed layout and repack bit for
bit, integer partials bit for bit, GEMV / GEMM outputs within max relative
error 1e-3 (denominator |ref| + 1e-3) and bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from knivesysl_xe_amd import ops  # noqa: E402
from knivesysl_xe_amd._lib import KxError  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests.test_oracle import random_payload  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-3


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    O.set_num_threads(16)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def w8_weight(rng, M, K):
    codes = rng.integers(-128, 128, (M, K)).astype(np.int8)
    scales = (np.abs(rng.standard_normal((M, K // 32))) * 0.002).astype(np.float16).view(np.uint16)
    return codes, scales, ops.W4Weight.from_codes_s8(dev(codes), dev(scales.view(np.int16)))


def assert_parity(got, ref, what):
    rel = np.max(np.abs(got.astype(np.float64) - ref) / (np.abs(ref.astype(np.float64)) + 1e-3))
    assert rel <= REL_TOL, f"{what}: max rel {rel}"
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        f"{what}: within tolerance (max rel {rel:.2e}) but {np.count_nonzero(got != ref)} of {got.size} differ"


def test_pack_s8_layout_and_roundtrip():
    rng = np.random.default_rng(40)
    M, K = 48, 384
    codes, scales, w = w8_weight(rng, M, K)
    got = w.codes.cpu().numpy()
    # include/kxw4.h W8 tiles: (rg, kb) of 2048 bytes; half h at 1024h, lane l
    # owns 16 bytes of row l%16: unit j = 2h (bytes 0..7) and 2h+1 (8..15),
    # byte b of unit j is k = 32j + 8(l/16) + b
    want = np.zeros(M * K, np.uint8)
    cu = codes.view(np.uint8)
    NT = K // 128
    for rg in range(M // 16):
        for kb in range(NT):
            for h in range(2):
                for lane in range(64):
                    for jj in range(2):
                        j = 2 * h + jj
                        for b in range(8):
                            row, k = rg * 16 + lane % 16, kb * 128 + 32 * j + 8 * (lane // 16) + b
                            want[(rg * NT + kb) * 2048 + 1024 * h + 16 * lane + 8 * jj + b] = cu[row, k]
    assert np.array_equal(got, want)
    c2, s2 = w.unpack()
    assert np.array_equal(c2.cpu().numpy(), codes)
    assert np.array_equal(s2.cpu().numpy().view(np.uint16), scales)


def test_repack_e2m3_s8_matches_oracle():
    rng = np.random.default_rng(41)
    M, K = 256, 1024
    payload, bs, scale_cols = random_payload(rng, M, K)
    want_codes, want_scales = O.repack_e2m3_s8(payload, bs, scale_cols, M, K)
    w = ops.W4Weight.repack_e2m3_s8(dev(payload), dev(bs), scale_cols, M, K)
    c, s = w.unpack()
    assert np.array_equal(s.cpu().numpy().view(np.uint16), want_scales)
    assert np.array_equal(c.cpu().numpy(), want_codes)


@pytest.mark.parametrize("M,K,T", [(64, 128, 1), (1040, 5120, 1), (512, 2048, 8), (2064, 1024, 16)])
@pytest.mark.parametrize("splits", [0, 1, 4])
def test_w8a8_gemv(M, K, T, splits):
    print(f"w8a8 gemv M={M} K={K} T={T} splits={splits}", flush=True)
    rng = np.random.default_rng(M + K + T + splits)
    codes, scales, w = w8_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    S = splits or O.gemv_splits(M // 16)
    y = ops.gemv(w, a, residual=dev(res), splits=splits).cpu().numpy()
    ref = O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMV, S, residual=res)
    assert_parity(y, ref, f"gemv {M}x{K} T={T} S={S}")


@pytest.mark.parametrize("T", [8, 16])
def test_w8a8_gemv_long_k(T):
    # K = 17408 (the down projection): at T >= 7 the activations do not fit
    # in one work-group's LDS, so the launcher runs the tokens in chunks
    M, K = 1040, 17408
    print(f"w8a8 gemv long K M={M} K={K} T={T}", flush=True)
    rng = np.random.default_rng(630 + T)
    codes, scales, w = w8_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    S = O.gemv_splits(M // 16)
    y = ops.gemv(w, a, residual=dev(res)).cpu().numpy()
    for rb, re in ((0, 272), (M - 144, M)):
        ref = O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMV, S, residual=res, rows=(rb, re))
        assert_parity(y[:, rb:re], ref[:, rb:re], f"w8 long K T={T} rows {rb}:{re}")


@pytest.mark.parametrize("M,K,T", [(512, 1024, 8), (256, 2048, 16), (512, 1024, 40), (1040, 640, 300)])
def test_w8a8_gemm(M, K, T):
    # x_gemm_w8a8: one serial chain per output (forced split 1); T <= 16 runs
    # on the row-wave kernel, larger T on the general GEMM
    print(f"w8a8 gemm M={M} K={K} T={T}", flush=True)
    rng = np.random.default_rng(M * 3 + K + T)
    codes, scales, w = w8_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    y = ops.gemm(w, a, forced_splits=1).cpu().numpy()
    ref = O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMM, 1)
    assert_parity(y, ref, f"gemm {M}x{K} T={T}")
    # the heuristic split plan and packed segments (split-ordered sums)
    offsets = [0, T // 2, T] if T >= 2 else None
    y2 = ops.gemm(w, a, offsets=offsets).cpu().numpy()
    sp = O.segment_splits(T, M, K, offsets)
    ref2 = O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMM, sp)
    assert_parity(y2, ref2, f"gemm {M}x{K} T={T} segments")


@pytest.mark.parametrize("T", [3, 40])
def test_w8a8_partials(T):
    rng = np.random.default_rng(42 + T)
    M, K = 64, 512
    codes, scales, w = w8_weight(rng, M, K)
    a = ops.quantize_act(dev(rng.standard_normal((T, K)).astype(np.float32)), 32)
    P = ops.partials(w, a).cpu().numpy()
    q = ops.act_codes_natural(a).cpu().numpy().astype(np.int64)
    want = np.einsum("mkj,tkj->tmk", codes.reshape(M, K // 32, 32).astype(np.int64),
                     q.reshape(T, K // 32, 32))
    assert np.array_equal(P, want)


def test_w8a8_lm_head_shape_row_subset():
    # an lm_head-sized W8 weight (K = 5120) with the spec wave's 8 rows
    rng = np.random.default_rng(43)
    M, K, T = 65536, 5120, 8
    codes, scales, w = w8_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    y = ops.gemm(w, a, forced_splits=1).cpu().numpy()
    for rb, re in ((0, 512), (M - 512, M)):
        ref = O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMM, 1, rows=(rb, re))
        assert_parity(y[:, rb:re], ref[:, rb:re], f"lm_head rows {rb}:{re}")


def test_w8a8_argument_checks():
    rng = np.random.default_rng(44)
    M, K = 64, 256
    codes, scales, w = w8_weight(rng, M, K)
    x = dev(rng.standard_normal((17, K)).astype(np.float32))
    with pytest.raises(KxError) as e:                    # W8A8 needs block-32 activations
        ops.gemv(w, ops.quantize_act(x[:1], 0))
    assert e.value.code == -1
    with pytest.raises(KxError) as e:                    # GEMV takes at most 16 token rows
        ops.gemv(w, ops.quantize_act(x, 32))
    assert e.value.code == -2
    with pytest.raises(KxError) as e:                    # no W8 fan-out in the reference
        ops.gemv_fanout([w, w], ops.quantize_act(x[:1], 32))
    assert e.value.code == -5
