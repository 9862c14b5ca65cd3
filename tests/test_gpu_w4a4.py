"""Parity of the W4A4 path (s4 activation quantizer and W4A4 GEMM, through the
C ABI) with the CPU oracle: codes, scales and sums bit for bit, outputs within
max relative error 1e-3 (denominator |ref| + 1e-3) and, since the kernel runs
the reference's chain order with explicit fused multiply-adds, bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from knivesysl_xe_amd import ops  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests.test_oracle import gemm_check_input, rounding_boundary_rows  # noqa: E402

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


def k64_weight(rng, M, K):
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    mags = (np.abs(rng.standard_normal((M, K // 64))) * 0.02).astype(np.float16).view(np.uint16)
    scales = ((mags & 0xFFF0) | (rng.integers(-8, 8, mags.shape) & 0xF)).astype(np.uint16)
    w = ops.W4Weight.from_codes(dev(codes), dev(scales.view(np.int16)), 64, O.SCALE_FP16_ZP4)
    return codes, scales, w


def assert_parity(got, ref, what, bf16=False):
    g, r = (O.bf16_to_f32(got), O.bf16_to_f32(ref)) if bf16 else (got, ref)
    rel = np.max(np.abs(g.astype(np.float64) - r) / (np.abs(r.astype(np.float64)) + 1e-3))
    assert rel <= REL_TOL, f"{what}: max rel {rel}"
    view = np.uint16 if bf16 else np.uint32
    assert np.array_equal(got.view(view), ref.view(view)), \
        f"{what}: within tolerance (max rel {rel:.2e}) but {np.count_nonzero(got != ref)} of {got.size} differ"


def s4_layout_bytes(q, T, K):
    """include/kxw4.h: [K/128][T][64 B], dword i of lane group g holds
    k = 128kb + 32i + 8g + b (b < 4 low nibbles of bytes 0..3, b >= 4 high)."""
    n = (q.astype(np.int64) & 0xF).reshape(T, K // 128, 4, 4, 8)     # [t][kb][i][g][b]
    byte = n[..., :4] | (n[..., 4:] << 4)                             # [t][kb][i][g][byte]
    return byte.transpose(1, 0, 3, 2, 4).reshape(-1).astype(np.uint8)  # [kb][t][g][i][byte]


def edge_input(rng, T, K, inf=True):
    x = (rng.standard_normal((T, K)) * np.exp2(rng.integers(-8, 8, (T, 1)))).astype(np.float32)
    if T > 2 and K >= 256:
        x[1, 64:128] = 0.0                    # zero block: scale 1, codes 0
        x[2, 5] = np.nan                      # NaN: ignored by the max, code -7
        if inf:
            x[2, 130] = np.inf                # inf max: finite codes 0, inf -> -7
    return x


@pytest.mark.parametrize("T,K", [(1, 128), (8, 640), (37, 1024), (300, 5120), (3, 17408)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_s4_quantizer(T, K, dtype):
    rng = np.random.default_rng(T * 7 + K)
    x = edge_input(rng, T, K)
    if dtype == "bf16":
        xt = dev(x).to(torch.bfloat16)
        x = xt.float().cpu().numpy()
    else:
        xt = dev(x)
    a = ops.quantize_act_s4(xt)
    q, s, sm = O.quantize_act_s4(x)
    torch.cuda.synchronize()
    assert np.array_equal(a.q4.cpu().numpy().reshape(-1), s4_layout_bytes(q, T, K))
    assert np.array_equal(ops.s4_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.T.copy().view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm.T)


@pytest.mark.parametrize("T,K", [(1, 4096), (37, 1024)])
def test_s4_quantizer_rounding_boundaries(T, K):
    # values at and within 3 ulp of every rounding boundary of v / s per K64
    # block: the reciprocal products must give the division's codes
    rng = np.random.default_rng(T + K)
    x = rounding_boundary_rows(rng, T, K, 64, 7)
    a = ops.quantize_act_s4(dev(x))
    q, s, sm = O.quantize_act_s4(x)
    torch.cuda.synchronize()
    assert np.array_equal(ops.s4_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.T.copy().view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm.T)


def oracle_w4a4(codes, scales, x, residual=None, out_bf16=False, rows=None):
    q, s, sm = O.quantize_act_s4(x)
    return O.project(codes, scales, 64, O.SCALE_FP16_ZP4, q, s, sm, 64, O.VAR_GEMM, 1,
                     residual=residual, out_bf16=out_bf16, rows=rows)


@pytest.fixture(params=[0, 1, 2, 3, 4])
def w4a4_tile(request):
    with ops.option("w4a4_tile", request.param):
        yield request.param


@pytest.mark.parametrize("M,K,T", [(64, 128, 1), (128, 640, 37), (1040, 1024, 300), (256, 5120, 8),
                                   (2064, 2048, 129)])
def test_w4a4_gemm(M, K, T, w4a4_tile):
    print(f"w4a4 M={M} K={K} T={T} tile={w4a4_tile}", flush=True)
    rng = np.random.default_rng(M + K + T)
    codes, scales, w = k64_weight(rng, M, K)
    x = edge_input(rng, T, K, inf=False)
    a = ops.quantize_act_s4(dev(x))
    y = ops.gemm_w4a4(w, a)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), oracle_w4a4(codes, scales, x), f"w4a4 {M}x{K} T={T}")
    res = rng.standard_normal((T, M)).astype(np.float32)
    yb = ops.gemm_w4a4(w, a, dtype=torch.bfloat16, residual=dev(res))
    torch.cuda.synchronize()
    ref = oracle_w4a4(codes, scales, x, residual=res, out_bf16=True)
    assert_parity(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref, "w4a4 bf16+res", bf16=True)


def test_w4a4_all_ones_gives_K():
    # xpu/probe/w4a4_gemm_probe.cpp:13-17
    M, K, T = 64, 1024, 16
    w = ops.W4Weight.from_codes(dev(np.ones((M, K), np.int8)),
                                dev(np.full((M, K // 64), 0x3C00, np.int16)), 64, O.SCALE_FP16_ZP4)
    a = ops.quantize_act_s4(dev(np.full((T, K), 7.0, np.float32)))
    # s = 1, every code 7: y = 7K
    y = ops.gemm_w4a4(w, a)
    torch.cuda.synchronize()
    assert torch.all(y == 7 * K)


def test_w4a4_cfg2_shape_row_subset():
    # the K64 down projection of BASELINE config 2 at its GEMM size (T = 512),
    # oracle on the first and last 256 rows
    rng = np.random.default_rng(5)
    M, K, T = 5120, 17408, 512
    codes, scales, w = k64_weight(rng, M, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = ops.gemm_w4a4(w, ops.quantize_act_s4(dev(x))).cpu().numpy()
    for rb, re in ((0, 256), (M - 256, M)):
        ref = oracle_w4a4(codes, scales, x, rows=(rb, re))
        assert_parity(y[:, rb:re], ref[:, rb:re], f"cfg2 rows {rb}:{re}")


def test_w4a4_agrees_with_w4a8_gemv_gate():
    # qwn_gemm_w4a4_check (kernels_dpas.cpp:2335-2409): GPU W4A4 against the
    # GPU W4A8 GEMV on the same K64 weight, worst token-row cosine >= 0.995
    rng = np.random.default_rng(6)
    M, K, T = 1024, 5120, 16
    codes, scales, w = k64_weight(rng, M, K)
    x = dev(gemm_check_input(T, K))
    ref = ops.gemv(w, ops.quantize_act(x, 32)).double()
    got = ops.gemm_w4a4(w, ops.quantize_act_s4(x)).double()
    cos = (ref * got).sum(1) / (ref.norm(dim=1) * got.norm(dim=1))
    assert cos.min().item() >= 0.995, cos


def test_w4a4_argument_checks():
    rng = np.random.default_rng(7)
    M, K, T = 64, 256, 8
    codes, scales, w = k64_weight(rng, M, K)
    a = ops.quantize_act_s4(dev(rng.standard_normal((T, K)).astype(np.float32)))
    w128 = ops.W4Weight.from_codes(dev(codes), dev(scales[:, ::2].copy().view(np.int16)), 128,
                                   O.SCALE_FP16_ZP4)
    with pytest.raises(ops._lib.KxError) as e:
        ops.gemm_w4a4(w128, a)
    assert e.value.code == -1
    wplain = ops.W4Weight(w.M, w.K, 64, O.SCALE_FP16, w.codes, w.scales)
    with pytest.raises(ops._lib.KxError) as e:
        ops.gemm_w4a4(wplain, a)
    assert e.value.code == -1
    with pytest.raises(ops._lib.KxError) as e:
        ops.quantize_act_s4(dev(rng.standard_normal((T, 192)).astype(np.float32)))
    assert e.value.code == -2
