"""Parity of the K16 tier (W4 weights with one FP16|zp scale per K16 half,
kernels_dpas.cpp:287-296 and 683-760) on the GPU with the CPU oracle: the
repack bit for bit, the GEMV bit for bit and within max relative error 1e-3,
including the reference's accumulation order and split boundaries.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from knivesysl_xe_amd import ops  # noqa: E402
from knivesysl_xe_amd._lib import KxError  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests.test_oracle import k16_case, random_payload  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    O.set_num_threads(16)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def k16_weight(rng, M, K):
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    mags = (np.abs(rng.standard_normal((M, K // 16))) * 0.02).astype(np.float16).view(np.uint16)
    scales = ((mags & 0xFFF0) | (rng.integers(-8, 8, mags.shape) & 0xF)).astype(np.uint16)
    w = ops.W4Weight.from_codes(dev(codes), dev(scales.view(np.int16)), 16, O.SCALE_FP16_ZP4)
    return codes, scales, w


def assert_parity(got, ref, what):
    rel = np.max(np.abs(got.astype(np.float64) - ref) / (np.abs(ref.astype(np.float64)) + 1e-3))
    assert rel <= 1e-3, f"{what}: max rel {rel}"
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        f"{what}: within tolerance (max rel {rel:.2e}) but {np.count_nonzero(got != ref)} of {got.size} differ"


def test_repack_k16_matches_oracle():
    rng = np.random.default_rng(60)
    M, K = 256, 1024
    payload, bs, scale_cols = random_payload(rng, M, K)
    want_codes, want_scales = O.repack_e2m3(payload, bs, scale_cols, M, K, 1)
    w = ops.W4Weight.repack_e2m3(dev(payload), dev(bs), scale_cols, M, K, 1)
    assert w.group == 16
    c, s = w.unpack()
    assert np.array_equal(s.cpu().numpy().view(np.uint16), want_scales)
    assert np.array_equal(c.cpu().numpy(), want_codes)


@pytest.mark.parametrize("M,K,T", [(64, 384, 1), (1040, 5120, 1), (512, 2048, 8), (256, 1152, 16),
                                   (256, 1152, 2), (1040, 2048, 3)])
@pytest.mark.parametrize("splits", [0, 1, 8])
def test_k16_gemv(M, K, T, splits):
    print(f"k16 gemv M={M} K={K} T={T} splits={splits}", flush=True)
    rng = np.random.default_rng(M + K + T + splits)
    codes, scales, w = k16_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    S = splits or O.gemv_splits(M // 16)
    y = ops.gemv(w, a, splits=splits).cpu().numpy()
    assert_parity(y, O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, S), f"k16 {M}x{K} T={T} S={S}")
    yr = ops.gemv(w, a, residual=dev(res), splits=splits).cpu().numpy()
    assert_parity(yr, O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, S, residual=res), "k16 + res")


@pytest.mark.parametrize("M,T", [(1040, 8), (1040, 16), (5120, 16), (5120, 1), (5120, 2)])
def test_k16_gemv_long_k(M, T):
    # K = 17408 (the down projection): T tokens' activations do not fit in one
    # work-group's LDS with the scale tables, so the launcher runs the tokens
    # in chunks that do; the last chunk is shorter
    K = 17408
    print(f"k16 gemv long K M={M} K={K} T={T}", flush=True)
    rng = np.random.default_rng(620 + T + M)
    codes, scales, w = k16_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    S = O.gemv_splits(M // 16)
    y = ops.gemv(w, a, residual=dev(res)).cpu().numpy()
    ref = O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, S, residual=res, rows=(0, 272))
    assert_parity(y[:, :272], ref[:, :272], f"k16 long K T={T}")
    ref2 = O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, S, residual=res, rows=(M - 144, M))
    assert_parity(y[:, M - 144:], ref2[:, M - 144:], f"k16 long K T={T} last rows")


@pytest.mark.parametrize("case", ["splits_on_k32_tiles", "single_accumulator"])
def test_k16_order_cases(case):
    # the oracle's hand-derived order cases (tests/test_oracle.py) on the GPU
    if case == "splits_on_k32_tiles":
        terms, tiles, S, want = [2.0 ** 24, 0, 1.0, 1.0] + [0] * 20, [2.0 ** 11] + [1.0] * 11, 8, 2.0 ** 24 + 2
    else:
        terms, tiles, S, want = [1.0, 2.0 ** 24, 1.0] + [0] * 21, [2.0 ** 12] + [1.0] * 11, 1, 2.0 ** 24
    codes, scales, q, s, sm = k16_case(terms, tiles)
    w = ops.W4Weight.from_codes(dev(codes), dev(scales.view(np.int16)), 16, O.SCALE_FP16_ZP4)
    a = ops.act_from_codes(dev(q), dev(s), dev(sm), 32)
    y = ops.gemv(w, a, splits=S).cpu().numpy()
    assert y[0, 0] == np.float32(want)


def test_k16_argument_checks():
    rng = np.random.default_rng(61)
    M, K = 64, 256
    codes, scales, w = k16_weight(rng, M, K)
    x = dev(rng.standard_normal((17, K)).astype(np.float32))
    with pytest.raises(KxError) as e:                   # no K16 GEMM (kernels_dpas.cpp:1337)
        ops.gemm(w, ops.quantize_act(x, 32))
    assert e.value.code == -1
    with pytest.raises(KxError) as e:                   # no K16 fan-out (956-959)
        ops.gemv_fanout([w, w], ops.quantize_act(x[:1], 32))
    assert e.value.code == -2
    with pytest.raises(KxError) as e:                   # block-32 activations only
        ops.gemv(w, ops.quantize_act(x[:1], 0))
    assert e.value.code == -1
    with pytest.raises(KxError) as e:                   # at most 16 token rows
        ops.gemv(w, ops.quantize_act(x, 32))
    assert e.value.code == -2
