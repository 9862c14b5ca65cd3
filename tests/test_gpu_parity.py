"""Parity of the HIP path (libkxw4.so via its C ABI) with the CPU oracle.

Integer results (packed codes, quantized activations, int32 unit partials)
must match bit for bit. Float outputs must match within max relative error
1e-3 with denominator |ref| + 1e-3 (kernels_dpas.cpp:2320); because the
kernels run the reference's accumulation order with explicit fused
multiply-adds, they are additionally required to match the oracle bit for
bit. Shapes are the BASELINE configurations at full size (cfg4 on a row
subset) plus small edge cases.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from knivesysl_xe_amd import ops, workloads  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests.test_oracle import gemm_check_input, random_payload, rounding_boundary_rows  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_TOL = 1e-3


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    O.set_num_threads(16)


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(DEV) if dtype is None else t.to(DEV).view(dtype)


def weight(codes, scales, group, enc=0):
    return ops.W4Weight.from_codes(dev(codes), dev(scales.view(np.int16)), group, enc)


def gpu_act(q, scale, sums, block):
    return ops.act_from_codes(dev(q), dev(scale), dev(sums), block)


def to_np(y):
    if y.dtype == torch.bfloat16:
        return y.view(torch.int16).cpu().numpy().view(np.uint16)
    return y.cpu().numpy()


def assert_parity(got, ref, what, bf16=False):
    if bf16:
        g, r = O.bf16_to_f32(got), O.bf16_to_f32(ref)
    else:
        g, r = got, ref
    rel = np.max(np.abs(g.astype(np.float64) - r) / (np.abs(r.astype(np.float64)) + 1e-3))
    assert rel <= REL_TOL, f"{what}: max rel {rel}"
    same = np.array_equal(got.view(np.uint16 if bf16 else np.uint32),
                          ref.view(np.uint16 if bf16 else np.uint32))
    assert same, f"{what}: within tolerance (max rel {rel:.2e}) but not bit-exact " \
                 f"({np.count_nonzero(got != ref)} of {got.size} differ)"


def rand_weight(rng, M, K, group, enc):
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    mags = (np.abs(rng.standard_normal((M, K // group))) * 0.02).astype(np.float16).view(np.uint16)
    if enc:
        mags = ((mags & 0xFFF0) | (rng.integers(-8, 8, mags.shape) & 0xF)).astype(np.uint16)
    return codes, mags


# ------------------------------------------------------------------ weights
def test_pack_matches_documented_layout_and_roundtrips():
    rng = np.random.default_rng(0)
    M, K = 48, 384
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    scales = rng.integers(0, 65536, (M, K // 64)).astype(np.uint16)
    w = weight(codes, scales, 64)
    got = w.codes.cpu().numpy().view(np.uint32)
    # include/kxw4.h: tile (rg, kb) of 1024 bytes; lane l owns 16 bytes, row
    # l%16; dword i holds k = 32i + 8(l/16) + b, b<4 low nibbles, b>=4 high
    want = np.zeros(M * K // 8, np.uint32)
    NT = K // 128
    for rg in range(M // 16):
        for kb in range(NT):
            for lane in range(64):
                for i in range(4):
                    row, k0 = rg * 16 + lane % 16, kb * 128 + 32 * i + 8 * (lane // 16)
                    v = 0
                    for b in range(4):
                        lo = int(codes[row, k0 + b]) & 0xF
                        hi = int(codes[row, k0 + b + 4]) & 0xF
                        v |= (lo | (hi << 4)) << (8 * b)
                    want[((rg * NT + kb) * 64 + lane) * 4 + i] = v
    assert np.array_equal(got, want)
    st = w.scales.cpu().numpy().view(np.uint16).reshape(M // 16, K // 64, 16)
    assert np.array_equal(st.transpose(0, 2, 1).reshape(M, K // 64), scales)
    c2, s2 = w.unpack()
    assert np.array_equal(c2.cpu().numpy(), codes)
    assert np.array_equal(s2.cpu().numpy().view(np.uint16), scales)


@pytest.mark.parametrize("group", [32, 64])
def test_import_reference_layout(group):
    rng = np.random.default_rng(1)
    M, K = 64, 512
    codes, scales = rand_weight(rng, M, K, group, 1)
    rc, rs = O.pack_ref_layout(codes, scales, group)
    w = ops.W4Weight.from_reference_layout(dev(rc), dev(rs.view(np.int16)), M, K, group)
    c2, s2 = w.unpack()
    assert np.array_equal(c2.cpu().numpy(), codes)
    assert np.array_equal(s2.cpu().numpy().view(np.uint16), scales)


@pytest.mark.parametrize("mode", [0, 2])
def test_repack_e2m3_matches_oracle(mode):
    rng = np.random.default_rng(2 + mode)
    M, K = 256, 1024
    payload, bs, scale_cols = random_payload(rng, M, K)
    want_codes, want_scales = O.repack_e2m3(payload, bs, scale_cols, M, K, mode)
    w = ops.W4Weight.repack_e2m3(dev(payload), dev(bs), scale_cols, M, K, mode)
    c2, s2 = w.unpack()
    assert np.array_equal(s2.cpu().numpy().view(np.uint16), want_scales)
    assert np.array_equal(c2.cpu().numpy(), want_codes)


# ------------------------------------------------------------------ activations
@pytest.mark.parametrize("mode", ["finite", "exceptional"])
@pytest.mark.parametrize("block", [32, 0])
def test_quantizer_golden(golden, mode, block):
    key = f"quant_{mode}_b{block}"
    x = golden[key + "_x"]
    a = ops.quantize_act(dev(x), block)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), golden[key + "_q"])
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32),
                          golden[key + "_scale"].view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), golden[key + "_sum"])


@pytest.mark.parametrize("T,K", [(7, 5120), (260, 5120), (260, 17408)])
@pytest.mark.parametrize("block", [32, 0])
def test_quantizer_bf16_input(T, K, block):
    rng = np.random.default_rng(3)
    xb = workloads.f32_to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32) * 3)
    a = ops.quantize_act(dev(xb.view(np.int16)).view(torch.bfloat16), block)
    q, s, sm = O.quantize_act(workloads.bf16_bits_to_f32(xb), block)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("T,K", [
    # the K32-block quantizer spreads rows over ceil(K/2048) work-groups at
    # any T: one to twelve work-groups per row, few and many rows
    (1, 4096), (2, 17408), (70, 4096), (64, 8192), (65, 20480), (64, 24576)])
@pytest.mark.parametrize("bf16", [False, True])
def test_quantizer_block_shapes(T, K, bf16):
    rng = np.random.default_rng(T * 7 + K)
    x = (rng.standard_normal((T, K)) * rng.uniform(0.01, 10, (T, 1))).astype(np.float32)
    x[0, 64:96] = 0.0                                    # an all-zero block: scale 1
    if bf16:
        xb = workloads.f32_to_bf16_bits(x)
        a = ops.quantize_act(dev(xb.view(np.int16)).view(torch.bfloat16), 32)
        x = workloads.bf16_bits_to_f32(xb)
    else:
        a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("T,K,block", [
    # K32 blocks (rows spread over 2, 9 and 1 work-groups), per-token rows
    # spread over 1, 2, 3, 4, 9 and 12 work-groups (the 1, 2, 3, 5, 9 and 12
    # chunk instances), and per-token rows of one work-group each (T at
    # least the CU count: 2, 3, 4 and 10 chunks of 256 threads, 3 of 1024)
    (1, 4096, 32), (3, 17408, 32), (300, 1024, 32),
    (7, 640, 0), (1, 4096, 0), (3, 5120, 0), (4, 8192, 0), (2, 17408, 0), (5, 24576, 0),
    (300, 2048, 0), (260, 5120, 0), (260, 8192, 0), (260, 12288, 0), (260, 17408, 0)])
def test_quantizer_rounding_boundaries(T, K, block):
    # values at and within 3 ulp of every rounding boundary of v / s, scales
    # from subnormal to 2^114, and a NaN and an infinity: the quantizers'
    # reciprocal products must give the division's codes everywhere
    print(f"quant boundaries T={T} K={K} block={block}", flush=True)
    rng = np.random.default_rng(T * 13 + K + block)
    x = rounding_boundary_rows(rng, T, K, 32 if block else K, 127)
    x[0, 37] = np.nan
    if T > 1:
        x[T - 1, 70] = np.inf
    a = ops.quantize_act(dev(x), block)
    q, s, sm = O.quantize_act(x, block)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


def test_quantizer_block_unaligned_rows():
    # rows that do not start on 16 bytes take the element loop; same bits
    T, K = 3, 4096
    rng = np.random.default_rng(8)
    x = rng.standard_normal((T, K)).astype(np.float32)
    base = torch.zeros(T * K + 1, dtype=torch.float32, device=DEV)
    xu = base[1:].view(T, K)
    xu.copy_(dev(x))
    assert xu.data_ptr() % 16 != 0
    a = ops.quantize_act(xu, 32)
    q, s, sm = O.quantize_act(x, 32)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("T,K", [(70, 4096), (1, 5120), (64, 20480), (300, 1024)])
@pytest.mark.parametrize("block", [32, 0])
def test_silu_mul_quant_shapes(T, K, block):
    # the SiLU quantizers with rows spread over 2, 3 and 10 work-groups, and
    # per-token rows of one work-group each
    rng = np.random.default_rng(T + K)
    gate = (rng.uniform(-1, 1, (T, K)) * 8).astype(np.float32)
    up = (rng.uniform(-1, 1, (T, K)) * 4).astype(np.float32)
    hidden, a = ops.silu_mul_quant(dev(gate), dev(up), block)
    h = hidden.cpu().numpy()
    ref = O.silu_mul(gate, up)
    assert np.max(np.abs(h - ref) / (np.abs(ref) + 1e-30)) < 1e-5
    q, s, sm = O.quantize_act(h, block)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("block", [32, 0])
def test_silu_mul_quant(block):
    # silu_quant_bench.cpp:40-55 inputs: scaled LCG draws plus zero blocks,
    # -0, saturated +-100 gates and tiny up values
    K, T = 17408, 2
    rng = np.random.default_rng(4)
    gate = (rng.uniform(-1, 1, (T, K)) * 8).astype(np.float32)
    up = (rng.uniform(-1, 1, (T, K)) * 4).astype(np.float32)
    gate[:, :32] = 0.0
    gate[:, 0] = -0.0
    gate[:, 32], gate[:, 33] = -100.0, 100.0
    up[:, 64:96] *= np.float32(1e-20)
    hidden, a = ops.silu_mul_quant(dev(gate), dev(up), block)
    h = hidden.cpu().numpy()
    ref = O.silu_mul(gate, up)
    assert np.max(np.abs(h - ref) / (np.abs(ref) + 1e-30)) < 1e-5
    q, s, sm = O.quantize_act(h, block)      # quantization itself is bit-exact
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("block", [32, 0])
def test_rmsnorm_quant(block):
    rng = np.random.default_rng(5)
    T, H = 3, 5120
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = O.f32_to_bf16(rng.standard_normal(H).astype(np.float32) * 0.1)
    normed, a = ops.rmsnorm_quant(dev(x), dev(w.view(np.int16)), 1e-6, block)
    nv = normed.cpu().numpy()
    for t in range(T):
        ref = O.rmsnorm(x[t], w, 1e-6)
        assert np.max(np.abs(nv[t] - ref)) <= 2e-6 * np.max(np.abs(ref))
    q, s, sm = O.quantize_act(nv, block)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("T,H", [(70, 4096), (2, 17408), (1, 512), (300, 640), (260, 5120),
                                 (260, 17408)])
@pytest.mark.parametrize("block", [32, 0])
def test_rmsnorm_quant_shapes(T, H, block):
    # the RMSNorm quantizers with rows spread over 2, 9 and 1 work-groups, and
    # rows of one work-group each (T at least the CU count: 2, 3 and 10
    # chunks per thread)
    rng = np.random.default_rng(T * 3 + H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = O.f32_to_bf16(rng.standard_normal(H).astype(np.float32) * 0.1)
    normed, a = ops.rmsnorm_quant(dev(x), dev(w.view(np.int16)), 1e-6, block)
    nv = normed.cpu().numpy()
    for t in range(T):
        ref = O.rmsnorm(x[t], w, 1e-6)
        assert np.max(np.abs(nv[t] - ref)) <= 2e-6 * np.max(np.abs(ref))
    y = ops.rmsnorm(dev(x), dev(w.view(np.int16)), 1e-6).cpu().numpy()
    assert np.array_equal(nv.view(np.uint32), y.view(np.uint32))
    q, s, sm = O.quantize_act(nv, block)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q)
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(a.sum.cpu().numpy(), sm)


@pytest.mark.parametrize("T,H", [(1, 2048), (5, 5120), (300, 640), (2, 1000)])
def test_rmsnorm_chunk(T, H):
    # x_rmsnorm_chunk (kernels_dpas.cpp:1124-1144): the rows kxw4_rmsnorm_quant
    # writes, bit for bit, and the oracle's norm within 2e-6
    rng = np.random.default_rng(T + H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = O.f32_to_bf16(rng.standard_normal(H).astype(np.float32) * 0.1)
    y = ops.rmsnorm(dev(x), dev(w.view(np.int16)), 1e-6).cpu().numpy()
    for t in range(T):
        ref = O.rmsnorm(x[t], w, 1e-6)
        assert np.max(np.abs(y[t] - ref)) <= 2e-6 * np.max(np.abs(ref))
    if H % 64 == 0:
        normed, _ = ops.rmsnorm_quant(dev(x), dev(w.view(np.int16)), 1e-6, 32)
        assert np.array_equal(normed.cpu().numpy().view(np.uint32), y.view(np.uint32))


# ------------------------------------------------------------------ partials
@pytest.mark.parametrize("name", ["ref32", "ref64", "cfg128", "cfg64"])
def test_partials_golden(golden, name):
    g = lambda k: golden[f"part_{name}_{k}"]
    group, block, zp = (int(v) for v in g("meta"))
    T, K = g("q").shape
    scale = np.ones((T, K // 32) if block == 32 else T, np.float32)
    w = weight(g("codes"), g("scales"), group, zp)
    P = ops.partials(w, gpu_act(g("q"), scale, g("asum"), block))
    assert np.array_equal(P.cpu().numpy(), g("P"))


@pytest.mark.parametrize("M,K,T,group,block,enc", [
    (128, 5120, 19, 128, 0, 0), (80, 17408, 3, 64, 0, 0), (64, 1024, 70, 32, 32, 1),
    (48, 2048, 33, 64, 32, 1)])
def test_partials_random(M, K, T, group, block, enc):
    rng = np.random.default_rng(M + K + T)
    codes, scales = rand_weight(rng, M, K, group, enc)
    q, s, sm = O.quantize_act(rng.standard_normal((T, K)).astype(np.float32), block)
    P = ops.partials(weight(codes, scales, group, enc), gpu_act(q, s, sm, block))
    assert np.array_equal(P.cpu().numpy(), O.partials(codes, scales, group, enc, q, s, sm, block))


# ------------------------------------------------------------------ golden projections
@pytest.mark.parametrize("name", ["ref32", "ref64", "cfg128", "cfg64"])
def test_exact_golden(golden, name):
    g = lambda k: golden[f"exact_{name}_{k}"]
    group, block, zp = (int(v) for v in g("meta"))
    w = weight(g("codes"), g("scales"), group, zp)
    a = gpu_act(g("q"), g("ascale"), g("asum"), block)
    want = g("y").view(np.uint32)
    for S in (1, 2, 4):
        assert np.array_equal(to_np(ops.gemv(w, a, splits=S)).view(np.uint32), want)
        assert np.array_equal(to_np(ops.gemm(w, a, forced_splits=S)).view(np.uint32), want)
    assert np.array_equal(to_np(ops.gemv_fanout([w], a)[0]).view(np.uint32), want)


def test_order_golden(golden):
    g = lambda k: golden[f"order_{k}"]
    codes, scales = g("codes"), g("scales")
    a = gpu_act(g("q"), g("ascale"), g("asum"), 0)
    w = weight(codes, scales, 32)
    # fan-out needs >= 4096 row-groups for one split: replicate the row
    wide = weight(np.repeat(codes[:1], 65536, 0), np.repeat(scales[:1], 65536, 0), 32)
    for var, S, want in zip(g("variants"), g("splits"), g("expected")):
        if var == 0:
            y = ops.gemv(w, a, splits=int(S))
        elif var == 2:
            y = ops.gemm(w, a, forced_splits=int(S))
        elif S == 1:
            y = ops.gemv_fanout([wide], a)[0]
        else:
            continue
        assert np.all(to_np(y) == want), (var, S, to_np(y)[0, :4], want)


@pytest.mark.parametrize("block,group,enc", [(32, 32, 1), (32, 64, 1), (0, 128, 0), (0, 64, 0)])
def test_all_ones_gives_K(block, group, enc):
    M, K, T = 256, 2048, 5
    w = weight(np.ones((M, K), np.int8), np.full((M, K // group), 0x3C00, np.uint16), group, enc)
    a = gpu_act(np.ones((T, K), np.int8),
                np.ones((T, K // 32) if block == 32 else T, np.float32),
                np.full((T, K // 32), 32, np.int32), block)
    for y in (ops.gemv(w, a), ops.gemm(w, a), ops.gemm(w, a, forced_splits=4),
              ops.gemv_fanout([w, w], a)[1]):
        assert np.all(to_np(y) == K)
    big = gpu_act(np.ones((300, K), np.int8),
                  np.ones((300, K // 32) if block == 32 else 300, np.float32),
                  np.full((300, K // 32), 32, np.int32), block)
    assert np.all(to_np(ops.gemm(w, big)) == K)


# ------------------------------------------------------------------ BASELINE configs
def run_config(name, seed=0, rows=None):
    cfg = workloads.CONFIGS[name]
    inp = workloads.generate(cfg, seed)
    ws = [weight(c, s, cfg.group) for c, s in zip(inp.codes, inp.scales)]
    x = dev(inp.x_bf16.view(np.int16)).view(torch.bfloat16)
    a = ops.quantize_act(x, 0)
    q, s, sm = O.quantize_act(workloads.bf16_bits_to_f32(inp.x_bf16), 0)
    assert np.array_equal(ops.act_codes_natural(a).cpu().numpy(), q), "activation codes"
    assert np.array_equal(a.scale.cpu().numpy().view(np.uint32), s.view(np.uint32))
    dt = torch.bfloat16 if cfg.out_bf16 else torch.float32
    if cfg.kind == "gemv":
        ys = [ops.gemv(ws[0], a, dt)]
        variant, splits = O.VAR_GEMV, [O.gemv_splits(cfg.rows[0] // 16)]
        splits = [np.full(cfg.tokens, splits[0], np.int32)]
    else:
        ys = ops.gemm_fanout(ws, a, dt, offsets=cfg.offsets)
        variant = O.VAR_GEMM
        splits = [O.segment_splits(cfg.tokens, N, cfg.K, cfg.offsets) for N in cfg.rows]
    torch.cuda.synchronize()
    for i, (c, sc, y) in enumerate(zip(inp.codes, inp.scales, ys)):
        N = c.shape[0]
        ranges = rows or [(0, N)]
        got = to_np(y)
        for rb, re in ranges:
            ref = O.project(c, sc, cfg.group, 0, q, s, sm, 0, variant, splits[i],
                            out_bf16=cfg.out_bf16, rows=(rb, re))
            assert_parity(got[:, rb:re], ref[:, rb:re], f"{name} weight {i} rows {rb}:{re}",
                          bf16=cfg.out_bf16)


@pytest.mark.parametrize("name", ["cfg0", "cfg1", "cfg2_m1", "cfg2_m512", "cfg3"])
def test_baseline_config(name):
    run_config(name)


def test_baseline_cfg4_row_subset():
    run_config("cfg4", rows=[(0, 512), (8192, 8704), (16896, 17408)])


@pytest.fixture
def kparallel():
    # up to 16 tokens normally run on the row-wave kernel; this keeps the
    # K-parallel decode kernel covered at the decode configurations
    with ops.option("decode_kernel", 1):
        yield


@pytest.fixture
def rowwave():
    # per-token shapes with at most 8 tokens and no more row-groups than CUs
    # (cfg0, the small golden cases) normally run on the K-parallel kernel;
    # this keeps the row-wave kernel covered there
    with ops.option("decode_kernel", 2):
        yield


def test_baseline_cfg0_rowwave(rowwave):
    run_config("cfg0")


@pytest.mark.parametrize("name", ["cfg128", "cfg64"])
def test_exact_golden_rowwave(golden, name, rowwave):
    test_exact_golden(golden, name)


@pytest.mark.parametrize("name", ["cfg0", "cfg1", "cfg2_m1"])
def test_baseline_config_kparallel(name, kparallel):
    run_config(name)


@pytest.mark.parametrize("spw,ring", [(1, 4), (2, 4), (3, 8), (4, 8), (8, 4)])
def test_cfg1_rowwave_shapes(spw, ring):
    # the row-wave kernel's slicing (rows per wave, one or two 16-row
    # windows) and ring depth change only who streams which rows: every shape
    # gives the same bits
    with ops.option("rowwave_spw", spw), ops.option("rowwave_ring", ring):
        run_config("cfg1", rows=[(0, 512), (8192, 8704), (16896, 17408)])


@pytest.mark.parametrize("ring", [4, 8])
def test_cfg2_m1_rowwave_ring(ring):
    with ops.option("rowwave_ring", ring):
        run_config("cfg2_m1")


@pytest.mark.parametrize("rows,K,T,group,block,enc,variant,forced", [
    # fewer chains than CUs: row-groups spread over several work-groups
    ([64], 4096, 1, 128, 0, 0, "gemv", 0),
    ([16], 2048, 3, 64, 0, 0, "gemm", 16),
    # cut row-groups at many boundaries, mixed weights in one fan-out
    ([4096, 1024, 48, 16], 5120, 8, 128, 0, 0, "gemm", 0),
    ([17408, 17408], 5120, 5, 128, 0, 0, "gemm", 0),
    ([3072, 1040], 2048, 2, 64, 0, 0, "fanout", 0),
    # K below one work-group's worth of tiles per segment, and K = 128
    ([4096], 512, 4, 128, 0, 0, "gemv", 0),
    ([1024], 128, 1, 128, 0, 0, "gemv", 0),
    # reference mode (per-K32 activation scales, zero points)
    ([2048, 512], 4096, 2, 64, 32, 1, "gemm", 0),
    ([5120], 17408, 1, 64, 32, 1, "gemv", 0),
    ([1024], 2048, 8, 32, 32, 1, "fanout", 0),
    # one or two tokens per token scale: the short-chain instances
    ([4096, 1024], 5120, 1, 128, 0, 0, "fanout", 0),
    ([2048], 4096, 2, 64, 0, 0, "gemv", 0),
    ([512, 48], 1024, 1, 32, 0, 0, "gemm", 4),
    ([1040], 17408, 2, 64, 0, 0, "gemm", 0),
])
def test_decode_shapes(rows, K, T, group, block, enc, variant, forced):
    # decode shapes off the BASELINE grid: fewer row-groups than CUs, mixed
    # weight heights in one launch, short K, both activation modes
    rng = np.random.default_rng(sum(rows) + K + T)
    wts = [rand_weight(rng, M, K, group, enc) for M in rows]
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, rows[0])).astype(np.float32)
    a = ops.quantize_act(dev(x), block)
    q, s, sm = O.quantize_act(x, block)
    ws = [weight(c, sc, group, enc) for c, sc in wts]
    if variant == "gemv":
        S = O.gemv_splits(rows[0] // 16)
        for r in (None, res):
            got = to_np(ops.gemv(ws[0], a, residual=None if r is None else dev(r)))
            ref = O.project(*wts[0], group, enc, q, s, sm, block, O.VAR_GEMV, S, residual=r)
            assert_parity(got, ref, f"gemv rows={rows[0]} residual={r is not None}")
        return
    if variant == "fanout":
        ys = ops.gemv_fanout(ws, a)
        S = O.gemv_splits(sum(rows) // 16)
        refs = [O.project(c, sc, group, enc, q, s, sm, block, O.VAR_FANOUT, S) for c, sc in wts]
    else:
        ys = ops.gemm_fanout(ws, a, torch.float32, forced_splits=forced)
        refs = [O.project(c, sc, group, enc, q, s, sm, block, O.VAR_GEMM,
                          O.segment_splits(T, c.shape[0], K, None, forced)) for c, sc in wts]
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert_parity(to_np(y), ref, f"{variant} weight {i} rows={rows[i]}")
    # a second launch gives the same bits
    ys2 = ops.gemv_fanout(ws, a) if variant == "fanout" else \
        ops.gemm_fanout(ws, a, torch.float32, forced_splits=forced)
    for y, y2 in zip(ys, ys2):
        assert np.array_equal(to_np(y).view(np.uint32), to_np(y2).view(np.uint32))


@pytest.fixture
def gemm_general():
    # the per-token prefill shapes normally run on the large-tile GEMM
    # kernel; this keeps the general GEMM kernel covered on them
    with ops.option("gemm_kernel", 1):
        yield


@pytest.fixture(params=list(range(12)))
def gemm3_tile(request):
    # every tile configuration of the large-tile kernel
    with ops.option("gemm3_tile", request.param):
        yield request.param


@pytest.mark.parametrize("rows,K,T,group", [
    # partial token and row tiles, fan-out weights of different heights,
    # fewer K steps than ring stages, both group sizes
    ([1040], 1024, 300, 128), ([1040, 2064], 640, 257, 64), ([4096], 128, 520, 128),
    ([256], 5120, 2048, 64), ([1040, 2064], 1024, 520, 128)])
def test_gemm3_shapes(rows, K, T, group, gemm3_tile):
    rng = np.random.default_rng(sum(rows) + K + T)
    wts = [rand_weight(rng, M, K, group, 0) for M in rows]
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, rows[0])).astype(np.float32)
    a = ops.quantize_act(dev(x), 0)
    q, s, sm = O.quantize_act(x, 0)
    ws = [weight(c, sc, group, 0) for c, sc in wts]
    sps = [O.segment_splits(T, M, K) for M in rows]
    # one split per token: the shapes the large-tile kernel takes
    assert all(np.all(sp == 1) for sp in sps)
    ys = ops.gemm_fanout(ws, a, torch.float32)
    for i, ((c, sc), y, sp) in enumerate(zip(wts, ys, sps)):
        ref = O.project(c, sc, group, 0, q, s, sm, 0, O.VAR_GEMM, sp)
        assert_parity(to_np(y), ref, f"weight {i} rows={rows[i]}")
    got = to_np(ops.gemm(ws[0], a, torch.bfloat16, residual=dev(res)))
    ref = O.project(*wts[0], group, 0, q, s, sm, 0, O.VAR_GEMM, sps[0], residual=res, out_bf16=True)
    assert_parity(got, ref, "bf16 + residual", bf16=True)


@pytest.mark.parametrize("K", [128, 256, 384, 512, 768, 896, 1152, 1408])
@pytest.mark.parametrize("tile", [8, 0])
def test_gemm3_k_steps(K, tile):
    # K step counts 1..11 at group 64: the one-block tile (8) unrolls its K
    # loop over six steps (three ring stages x two slot parities) and
    # finishes the rest one step at a time, so every remainder and counts
    # below one iteration run; tile 0 is the default tracked-offset loop
    with ops.option("gemm3_tile", tile):
        test_gemm3_shapes([1040, 2064], K, 257, 64, tile)


@pytest.mark.parametrize("rows,K,T,group", [
    # the tile chooser's own pick on ragged token counts
    ([1040, 2064], 640, 300, 128), ([4096], 512, 600, 128), ([1040], 1024, 1100, 64)])
def test_gemm3_auto_tile(rows, K, T, group):
    test_gemm3_shapes(rows, K, T, group, None)


@pytest.fixture(params=list(range(10)))
def gemmr_tile(request):
    # every tile configuration of the reference-mode large-tile kernel
    with ops.option("gemmr_tile", request.param):
        yield request.param


@pytest.mark.parametrize("rows,K,T,group,enc", [
    # x_gemm_w4a8's own inputs (K32 activation blocks, FP16|zp K32 and K64
    # weights) and plain FP16 weights at every group size; partial token
    # and row tiles, fan-out weights of different heights, fewer K steps
    # than ring stages, rows that start a new scale group mid-step
    ([1040], 1024, 300, 32, 1), ([1040, 2064], 640, 257, 64, 1), ([4096], 128, 520, 32, 1),
    ([256], 5120, 2048, 64, 1), ([1040], 512, 300, 32, 0), ([528, 1040], 1024, 520, 64, 0),
    ([1024], 768, 400, 128, 0)])
def test_gemmr_shapes(rows, K, T, group, enc, gemmr_tile):
    print(f"gemmr rows={rows} K={K} T={T} group={group} enc={enc} tile={gemmr_tile}", flush=True)
    rng = np.random.default_rng(sum(rows) + K + T + enc)
    wts = [rand_weight(rng, M, K, group, enc) for M in rows]
    x = rng.standard_normal((T, K)).astype(np.float32)
    x[:, :32] = 0.0                                  # an all-zero block (scale 1)
    res = rng.standard_normal((T, rows[0])).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    ws = [weight(c, sc, group, enc) for c, sc in wts]
    sps = [O.segment_splits(T, M, K) for M in rows]
    assert all(np.all(sp == 1) for sp in sps)       # the shapes the kernel takes
    ys = ops.gemm_fanout(ws, a, torch.float32)
    for i, ((c, sc), y, sp) in enumerate(zip(wts, ys, sps)):
        ref = O.project(c, sc, group, enc, q, s, sm, 32, O.VAR_GEMM, sp)
        assert_parity(to_np(y), ref, f"weight {i} rows={rows[i]}")
    got = to_np(ops.gemm(ws[0], a, torch.bfloat16, residual=dev(res)))
    ref = O.project(*wts[0], group, enc, q, s, sm, 32, O.VAR_GEMM, sps[0], residual=res, out_bf16=True)
    assert_parity(got, ref, "bf16 + residual", bf16=True)


def test_gemmr_packed_segments(gemmr_tile):
    # packed prefill segments whose split plans are all 1 (ragged lengths):
    # rows are independent of the segments, so the packed launch equals the
    # oracle per segment
    rng = np.random.default_rng(11)
    M, K, group = 8192, 512, 32
    offs = np.array([0, 25, 89, 389, 600], np.int32)
    T = int(offs[-1])
    c, sc = rand_weight(rng, M, K, group, 1)
    x = rng.standard_normal((T, K)).astype(np.float32)
    a = ops.quantize_act(dev(x), 32)
    q, s, sm = O.quantize_act(x, 32)
    sp = O.segment_splits(T, M, K, offs)
    assert np.all(sp == 1)
    got = to_np(ops.gemm(weight(c, sc, group, 1), a, offsets=offs))
    ref = O.project(c, sc, group, 1, q, s, sm, 32, O.VAR_GEMM, sp)
    assert_parity(got, ref, "packed reference-mode segments")


@pytest.mark.parametrize("name", ["cfg2_m512", "cfg3"])
def test_baseline_config_gemm_general(name, gemm_general):
    run_config(name)


def test_baseline_cfg4_rows_gemm_general(gemm_general):
    run_config("cfg4", rows=[(0, 256), (17152, 17408)])


# ------------------------------------------------------------------ properties
@pytest.mark.parametrize("kind", ["gemm", "gemv"])
def test_row_independence_specwave(kind):
    # qwn_specwave_check (kernels_dpas.cpp:2202-2255): rows 0-3 of a T=8
    # wave must be byte-identical when rows 4-7 change
    rng = np.random.default_rng(6)
    M, K = 17408 // 4, 5120
    codes, scales = rand_weight(rng, M, K, 128, 0)
    w = weight(codes, scales, 128)
    x0 = rng.standard_normal((8, K)).astype(np.float32)
    x1 = x0.copy()
    x1[4:] = rng.standard_normal((4, K)).astype(np.float32)
    outs = []
    for x in (x0, x1):
        a = ops.quantize_act(dev(x), 0)
        outs.append(to_np(ops.gemm(w, a) if kind == "gemm" else ops.gemv(w, a)))
    assert np.array_equal(outs[0][:4].view(np.uint32), outs[1][:4].view(np.uint32))


@pytest.mark.parametrize("M,segments", [(17408, [17, 64, 300, 512]), (5120, [8, 24, 40, 200]),
                                        (1024, [3, 13, 16, 100, 7])])
def test_packed_equals_serial(M, segments):
    # prefill_batch_check semantics: a packed launch equals independent
    # per-segment launches, because each segment keeps its own split plan
    rng = np.random.default_rng(M)
    K = 5120
    codes, scales = rand_weight(rng, M, K, 128, 0)
    w = weight(codes, scales, 128)
    T = sum(segments)
    x = rng.standard_normal((T, K)).astype(np.float32)
    off = [0] + list(np.cumsum(segments))
    packed = to_np(ops.gemm(w, ops.quantize_act(dev(x), 0), offsets=off))
    for i in range(len(segments)):
        seg = to_np(ops.gemm(w, ops.quantize_act(dev(x[off[i]:off[i + 1]]), 0)))
        assert np.array_equal(packed[off[i]:off[i + 1]].view(np.uint32), seg.view(np.uint32)), i
    # and both equal the oracle with per-segment splits
    q, s, sm = O.quantize_act(x, 0)
    sp = O.segment_splits(T, M, K, off)
    ref = O.project(codes, scales, 128, 0, q, s, sm, 0, O.VAR_GEMM, sp)
    assert_parity(packed, ref, "packed")


@pytest.mark.parametrize("M,K,T,group,block,enc", [
    (4096, 4096, 1, 32, 32, 1), (5120, 17408, 1, 64, 32, 1), (512, 1024, 4, 64, 32, 1),
    (64, 512, 2, 128, 0, 0), (48, 256, 1, 32, 32, 1), (16, 128, 1, 32, 32, 1),
    (256, 2048, 50, 32, 32, 1), (128, 17408, 20, 64, 32, 1), (2048, 2048, 13, 64, 32, 1),
    (1024, 4096, 5, 128, 0, 0), (64, 512, 16, 64, 0, 0),
    # two tokens on the reference arithmetic (the two-token instance)
    (1024, 2048, 2, 32, 32, 1), (528, 4096, 2, 64, 32, 1)])
def test_gemv_reference_mode(M, K, T, group, block, enc):
    rng = np.random.default_rng(M * 3 + K)
    codes, scales = rand_weight(rng, M, K, group, enc)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), block)
    q, s, sm = O.quantize_act(x, block)
    S = O.gemv_splits(M // 16)
    w = weight(codes, scales, group, enc)
    for r in (None, res):
        got = to_np(ops.gemv(w, a, residual=None if r is None else dev(r)))
        ref = O.project(codes, scales, group, enc, q, s, sm, block, O.VAR_GEMV, S, residual=r)
        assert_parity(got, ref, f"gemv M={M} K={K} residual={r is not None}")


@pytest.mark.parametrize("rows,T,block,enc,group", [
    ([10240, 6144, 48, 48], 1, 32, 1, 32), ([17408, 17408], 1, 32, 1, 64), ([16, 48], 1, 32, 1, 32),
    ([4096, 1024], 3, 0, 0, 128)])
def test_gemv_fanout(rows, T, block, enc, group):
    # fanout_bench.cpp shapes: mlp, gdn and tiny sets
    rng = np.random.default_rng(sum(rows))
    K = 5120 if rows[0] != 16 else 384
    wts = [rand_weight(rng, M, K, group, enc) for M in rows]
    x = rng.standard_normal((T, K)).astype(np.float32)
    x[:, :32] = 0.0
    a = ops.quantize_act(dev(x), block)
    q, s, sm = O.quantize_act(x, block)
    ys = ops.gemv_fanout([weight(c, sc, group, enc) for c, sc in wts], a)
    S = O.gemv_splits(sum(rows) // 16)
    for (c, sc), y in zip(wts, ys):
        ref = O.project(c, sc, group, enc, q, s, sm, block, O.VAR_FANOUT, S)
        assert_parity(to_np(y), ref, f"fanout rows={c.shape[0]}")


def test_prepared_calls_match_the_checked_calls():
    # ops.PreparedGemv / PreparedGemmFanout marshal once and then make the
    # same C-ABI call: the oracle's bits on every call, also after the
    # activation buffer's contents change
    rng = np.random.default_rng(21)
    K, rows, T = 2048, [1024, 512], 8
    wts = [rand_weight(rng, M, K, 128, 0) for M in rows]
    ws = [weight(c, sc, 128, 0) for c, sc in wts]
    x1 = rng.standard_normal((T, K)).astype(np.float32)
    x2 = rng.standard_normal((T, K)).astype(np.float32)
    a = ops.quantize_act(dev(x1), 0)
    outs = [torch.empty(T, M, dtype=torch.bfloat16, device=DEV) for M in rows]
    fan = ops.PreparedGemmFanout(ws, a, torch.bfloat16, outs=outs)
    one = ops.PreparedGemv(ws[0], a, torch.float32)
    for x in (x1, x2, x1):
        ops.quantize_act(dev(x), 0, out=a)
        q, s, sm = O.quantize_act(x, 0)
        fan()
        y = one()
        for (c, sc), got in zip(wts, outs):
            sp = O.segment_splits(T, c.shape[0], K, None, 0)
            ref = O.project(c, sc, 128, 0, q, s, sm, 0, O.VAR_GEMM, sp, out_bf16=True)
            assert_parity(to_np(got), ref, "prepared fan-out", bf16=True)
        ref = O.project(wts[0][0], wts[0][1], 128, 0, q, s, sm, 0, O.VAR_GEMV,
                        O.gemv_splits(rows[0] // 16))
        assert_parity(to_np(y), ref, "prepared gemv")


@pytest.mark.parametrize("M,K,T,block,enc,group,forced", [
    (17408 // 4, 5120, 8, 32, 1, 32, 0), (5120, 5120, 24, 32, 1, 64, 0), (1024, 2048, 128, 32, 1, 32, 0),
    (5120, 5120, 8, 0, 0, 128, 16), (768, 4096, 200, 0, 0, 64, 0), (512, 2048, 40, 0, 0, 128, 0),
    (1024, 4096, 64, 32, 1, 32, 0), (256, 17408, 61, 0, 0, 64, 0), (4096, 5120, 16, 0, 0, 128, 0),
    (1024, 4096, 12, 32, 1, 32, 0), (2048, 2048, 5, 32, 1, 64, 4), (512, 1024, 3, 0, 0, 64, 8),
    # the group-64 folded-zero-point decode GEMM at 8 and 16 tokens
    (2048, 4096, 8, 32, 1, 64, 0), (1040, 2048, 12, 32, 1, 64, 0)])
def test_gemm_modes(M, K, T, block, enc, group, forced):
    rng = np.random.default_rng(M + T)
    codes, scales = rand_weight(rng, M, K, group, enc)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), block)
    q, s, sm = O.quantize_act(x, block)
    sp = O.segment_splits(T, M, K, None, forced)
    w = weight(codes, scales, group, enc)
    got = to_np(ops.gemm(w, a, residual=dev(res), forced_splits=forced))
    ref = O.project(codes, scales, group, enc, q, s, sm, block, O.VAR_GEMM, sp, residual=res)
    assert_parity(got, ref, f"gemm M={M} K={K} T={T}")
    gotb = to_np(ops.gemm(w, a, torch.bfloat16, forced_splits=forced))
    refb = O.project(codes, scales, group, enc, q, s, sm, block, O.VAR_GEMM, sp, out_bf16=True)
    assert_parity(gotb, refb, "gemm bf16", bf16=True)


def test_gemm_agrees_with_gemv_gate():
    # qwn_gemm_check (kernels_dpas.cpp:2264-2333) for T in {8, 32, 128, 512}
    # (tools/gemm_check.py:22): GEMM vs per-row GEMV, cos >= 0.9999
    rng = np.random.default_rng(7)
    M, K = 17408 // 4, 5120
    codes, scales = rand_weight(rng, M, K, 32, 1)
    w = weight(codes, scales, 32, 1)
    for T in (8, 32, 128, 512):
        a = ops.quantize_act(dev(gemm_check_input(T, K)), 32)
        got = to_np(ops.gemm(w, a)).astype(np.float64)
        ref = to_np(ops.gemv(w, a) if T <= 64 else torch.cat(
            [ops.gemv(w, ops.quantize_act(dev(gemm_check_input(T, K)[i:i + 64]), 32))
             for i in range(0, T, 64)])).astype(np.float64)
        for t in range(T):
            c = got[t] @ ref[t] / np.sqrt((got[t] @ got[t]) * (ref[t] @ ref[t]))
            assert c >= 0.9999, (T, t, c)


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("S", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("variant", ["gemv", "gemm"])
def test_rowwave_short_token_splits(T, S, variant):
    # the one- and two-token row-wave instances (live-register chains, split
    # partials read at once before the ordered sum) at every split count,
    # both chain variants, with and without residual, against the oracle
    print(f"short-token rowwave T={T} S={S} {variant}", flush=True)
    M, K, group = 1040, 4096, 128
    rng = np.random.default_rng(T * 100 + S)
    codes, sc = rand_weight(rng, M, K, group, 0)
    w = weight(codes, sc, group, 0)
    x = rng.standard_normal((T, K)).astype(np.float32)
    res = rng.standard_normal((T, M)).astype(np.float32)
    a = ops.quantize_act(dev(x), 0)
    q, s, sm = O.quantize_act(x, 0)
    var = O.VAR_GEMV if variant == "gemv" else O.VAR_GEMM
    with ops.option("decode_kernel", 2):
        for r in (None, res):
            if variant == "gemv":
                got = to_np(ops.gemv(w, a, residual=None if r is None else dev(r), splits=S))
            else:
                got = to_np(ops.gemm(w, a, residual=None if r is None else dev(r), forced_splits=S))
            ref = O.project(codes, sc, group, 0, q, s, sm, 0, var, np.full(T, S, np.int32) if variant == "gemm" else S,
                            residual=r)
            assert_parity(got, ref, f"T={T} S={S} {variant} residual={r is not None}")
