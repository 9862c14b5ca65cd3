"""Pins the CPU oracle (oracle/w4a8_oracle.cpp) before it is trusted as the
checker of the HIP path. Every check here is independent of the oracle's own
code: numpy's IEEE conversions and integer matmuls, exact rational
arithmetic, hand-derived order cases, closed forms and invariants. Fixtures
come from tests/golden/make_golden.py."""
import numpy as np
import pytest

from oracle import oracle as O


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint16)


# ------------------------------------------------------------------ conversions
def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000)).astype(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e6, -1e6,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2.0 ** -24, 2.0 ** -25,
                        3 * 2.0 ** -26, 2.0 ** -26, 5.9604645e-08, 6.097555e-05, 6.1035156e-05,
                        np.inf, -np.inf, 1e-30, -1e-45], np.float32)
    x = np.concatenate([x, special])
    got = O.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert O.f32_to_f16(np.array([np.nan], np.float32))[0] & 0x7C00 == 0x7C00


def test_f16_to_f32_all_codes():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_bf16_is_nearest_even():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-20, 20, 100000)).astype(np.float32)
    b = O.f32_to_bf16(x).astype(np.int64)
    for d in (-1, 1):
        other = O.bf16_to_f32((b + d).astype(np.uint16)).astype(np.float64)
        mine = O.bf16_to_f32(b.astype(np.uint16)).astype(np.float64)
        e_mine = np.abs(mine - x)
        e_other = np.abs(other - x)
        assert np.all(e_mine <= e_other)
        tie = e_mine == e_other
        assert np.all((b[tie] & 1) == 0)


def test_e2m3_table_closed_form():
    # OCP FP6 E2M3: exponent bias 1, subnormal m/8; positive codes 0..31 are
    # the 32 values {0, 1/8, ..., 7/8, 1, 9/8, ..., 15/8, 2, ..., 3.75, 4, ..., 7.5}
    pos = [O.lib().orc_e2m3(c) for c in range(32)]
    want = [m / 8 for m in range(8)] + [1 + m / 8 for m in range(8)] + \
           [2 * (1 + m / 8) for m in range(8)] + [4 * (1 + m / 8) for m in range(8)]
    assert pos == want
    assert [O.lib().orc_e2m3(c | 0x20) for c in range(32)] == [-v for v in want]


def test_e2m3_fragment_addressing_is_a_bijection():
    # one m16k32 tile holds 512 six-bit codes in 384 bytes; every (row, col)
    # must own a distinct field and all 3072 bits must be covered
    Kt = 2
    seen = set()
    for row in range(16):
        for col in range(32):
            # recover (lane, idx) through the library by planting a one-hot
            payload = np.zeros(32 * Kt * 384, np.uint8)
            hits = []
            for byte in range(384):
                for bit in range(8):
                    payload[:] = 0
                    payload[byte] = 1 << bit
                    if O.lib().orc_e2m3_code_at(payload.ctypes.data, Kt, row, col) != 0:
                        hits.append(byte * 8 + bit)
            assert len(hits) == 6 and hits == list(range(hits[0], hits[0] + 6))
            seen.add(hits[0] // 6)
    assert seen == set(range(512))


def _plant_le(payload, tile_off, lane, idx, code):
    """Write `code` as field `idx` of lane `lane`'s little-endian 96-bit
    stream of 16 six-bit codes, in the lane's own 12 bytes of the tile
    (kernels_core.cpp:55-57)."""
    base = tile_off + 12 * lane
    v = int.from_bytes(bytes(payload[base:base + 12]), "little")
    v |= code << (6 * idx)
    payload[base:base + 12] = np.frombuffer(v.to_bytes(12, "little"), np.uint8)


def _lane_stream_holds(read, Kt=2, mt=1, kt=1, code=0b100101):
    """One field at a time: the field planted as (lane, idx) of tile (mt, kt)
    must be read back, with its value, at exactly one (row, col) of that
    tile, every other position reading 0, and the 512 fields must land on
    512 distinct positions. `code` is not its own 6-bit reversal."""
    tile_off = (mt * Kt + kt) * 384
    where = set()
    for lane in range(32):
        for idx in range(16):
            payload = np.zeros(2 * Kt * 384, np.uint8)
            _plant_le(payload, tile_off, lane, idx, code)
            hits = [(r, c, read(payload, Kt, 16 * mt + r, 32 * kt + c))
                    for r in range(16) for c in range(32)]
            nz = [h for h in hits if h[2] != 0]
            if len(nz) != 1 or nz[0][2] != code:
                return False
            where.add(nz[0][:2])
    return len(where) == 512


def _oracle_read(payload, Kt, row, col):
    return O.lib().orc_e2m3_code_at(payload.ctypes.data, Kt, row, col)


def _mutant_read(big_endian, stride):
    # the oracle's (row, col) -> (lane, idx) map, read from another stream
    # convention: most significant field first, or a 16-byte lane stride
    def read(payload, Kt, row, col):
        lane = (((row & 15) >> 1) << 2) | ((col & 31) >> 3)
        idx = (((col >> 2) & 1) << 3) | ((row & 1) << 2) | (col & 3)
        base = ((row >> 4) * Kt + (col >> 5)) * 384 + lane * stride
        v = int.from_bytes(bytes(payload[base:base + 12]), "big" if big_endian else "little")
        return (v >> (6 * (15 - idx) if big_endian else 6 * idx)) & 0x3F
    return read


def test_e2m3_lanes_are_little_endian_12_byte_streams():
    assert _lane_stream_holds(_oracle_read)
    # the check discriminates: a big-endian stream or a 16-byte lane stride
    # (the other plausible readings of the payload) fail it
    assert _lane_stream_holds(_mutant_read(False, 12))
    assert not _lane_stream_holds(_mutant_read(True, 12))
    assert not _lane_stream_holds(_mutant_read(False, 16))


# ------------------------------------------------------------------ quantizer
@pytest.mark.parametrize("mode", ["finite", "exceptional"])
@pytest.mark.parametrize("block", [32, 0])
def test_quantizer_matches_golden(golden, mode, block):
    key = f"quant_{mode}_b{block}"
    q, s, sm = O.quantize_act(golden[key + "_x"], block)
    assert np.array_equal(q, golden[key + "_q"])
    assert np.array_equal(bits(s), bits(golden[key + "_scale"]))
    assert np.array_equal(sm, golden[key + "_sum"])


def test_quantizer_round_half_even(golden):
    q, s, _ = O.quantize_act(golden["quant_ties_x"], 32)
    assert s[0, 0] == 1.0
    assert np.array_equal(q, golden["quant_ties_q"])


def test_quantizer_invariants():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 512)) * rng.uniform(1e-3, 1e3, (16, 1))).astype(np.float32)
    for block in (32, 0):
        q, s, sm = O.quantize_act(x, block)
        w = 32 if block == 32 else 512
        sb = np.repeat(s.reshape(16, -1), w, axis=1)
        xb = x.reshape(16, -1, w)
        # the block's absmax element lands on +-127; error within half a step
        idx = np.abs(xb).argmax(axis=2)
        qa = np.take_along_axis(q.reshape(16, -1, w), idx[..., None], 2)[..., 0]
        assert np.all(np.abs(qa) == 127)
        assert np.all(np.abs(x - q * sb) <= sb * (0.5 + 1e-6))
        assert np.array_equal(sm, q.reshape(16, -1, 32).astype(np.int32).sum(axis=2))


def test_quantizer_divides_rather_than_multiplies_by_reciprocal():
    # find inputs where rint(x/s) and rint(x*(1/s)) differ in fp32; the
    # reference divides (kernels_dpas.cpp:205, 1181)
    rng = np.random.default_rng(4)
    for _ in range(2000):
        mx = np.float32(rng.uniform(0.5, 100.0))
        s = mx / np.float32(127.0)
        x = (np.arange(-126, 127, dtype=np.float32) + np.float32(0.5)) * s
        x = np.nextafter(x, np.float32(0), dtype=np.float32)
        div = np.rint(x / s)
        mul = np.rint(x * (np.float32(1.0) / s))
        diff = np.nonzero(div != mul)[0]
        if diff.size:
            blk = np.zeros((1, 32), np.float32)
            blk[0, 0] = mx
            blk[0, 1] = x[diff[0]]
            q, sc, _ = O.quantize_act(blk, 32)
            assert sc[0, 0] == s
            assert q[0, 1] == div[diff[0]] != mul[diff[0]]
            return
    pytest.skip("no distinguishing case found")


def rounding_boundary_rows(rng, T, K, group, limit):
    """x[T][K] fp32 whose groups of `group` values (a K32 block, a K64 s4
    block, or the whole row for per-token scales) hold their maximum m in
    element 0 and otherwise values at or within 3 ulp of a half-integer
    multiple of s = fl(m / limit): the values where multiplying by a
    reciprocal can round differently from the division. Group maxima run from
    2^-140 (subnormal, and s below 2^-120) to 2^121."""
    ng = K // group
    e = rng.integers(-140, 121, (T, ng, 1)).astype(np.float64)
    mx = (rng.uniform(1, 2, (T, ng, 1)) * np.exp2(e)).astype(np.float32)
    s = mx / np.float32(limit)
    h = rng.integers(-limit, limit, (T, ng, group)) + 0.5
    v = (h * s.astype(np.float64)).astype(np.float32)
    d = rng.integers(-3, 4, (T, ng, group))
    for k in range(3):
        v = np.where(d > k, np.nextafter(v, np.float32(np.inf)), v)
        v = np.where(d < -k, np.nextafter(v, np.float32(-np.inf)), v)
    v = np.clip(v, -mx, mx)
    v[..., 0] = mx[..., 0] * np.where(rng.integers(0, 2, (T, ng)) == 1, 1, -1).astype(np.float32)
    return v.reshape(T, K)


@pytest.mark.parametrize("group,limit", [(32, 127), (4096, 127), (64, 7)])
def test_rounding_boundary_rows_separate_division_from_reciprocal(group, limit):
    # The GPU quantizers multiply by a reciprocal and divide only near a
    # rounding boundary. Their tests use these rows, which must hold values
    # where the two round differently, or a quantizer that skipped the
    # division would pass them.
    rng = np.random.default_rng(group + limit)
    x = rounding_boundary_rows(rng, 2, 4096, group, limit)
    if limit == 7:
        q, s, _ = O.quantize_act_s4(x)
    else:
        q, s, _ = O.quantize_act(x, 32 if group == 32 else 0)
    sb = np.repeat(s.reshape(2, -1), group, axis=1)
    with np.errstate(all="ignore"):
        div = np.clip(np.rint(x / sb), -limit, limit)
        mul = np.clip(np.rint(x * (np.float32(1) / sb)), -limit, limit)
    assert np.array_equal(div, q)                        # the oracle divides
    assert np.count_nonzero(mul != q) > 0


def test_silu_mul_and_rmsnorm_close_to_float64():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    got = O.silu_mul(g, u)
    g64 = g.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-30)) < 4e-7
    x = rng.standard_normal(5120).astype(np.float32)
    w = O.f32_to_bf16(rng.standard_normal(5120).astype(np.float32) * 0.1)
    got = O.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * (1 + O.bf16_to_f32(w).astype(np.float64))
    assert np.max(np.abs(got - want)) < 1e-5 * np.max(np.abs(want))


# ------------------------------------------------------------------ weights
def test_fit_int4_asym_known_answer():
    # w = 0.25 * [0..15]: lo=0, hi=3.75 -> s=0.25, zi=-8, q=j-8, centered=j;
    # least squares keeps s=0.25 exactly; z=-8; fp16(0.25)=0x3400
    sh, z = O.fit_int4_asym(np.arange(16, dtype=np.float32) * 0.25)
    assert (sh, z) == (0x3400, -8)
    # all-zero group: s falls back to 1.0, z = -8, and w=0 reconstructs to 0
    sh, z = O.fit_int4_asym(np.zeros(32, np.float32))
    assert (sh, z) == (0x3C00, -8)


@pytest.mark.parametrize("contract", [True, False])
def test_fit_int4_asym_nibble_reserve_rounds_up(contract):
    # fit_int4_asym stores (sh + 8) & 0xFFF0 (kernels_dpas.cpp:254-255): the
    # scale's low nibble is rounded half up into the next 16-ulp step, not
    # truncated and not rounded to even. Groups on an exact grid
    # w_j = s*(j-8), j = 0..15, keep s through the fit: lo = -8s, hi = 7s,
    # (hi-lo)/15 = s exactly; zi = rint(8s/s) - 8 = 0; codes q_j = j-8, so
    # num = 344*s and den = 344 (sum of c^2 over c = -8..7) are exact and
    # num/den = s in every refinement; z = 0.
    def grid(step):
        return (np.float32(step) * (np.arange(16) - 8)).astype(np.float32)
    # s = 1033/1024: fp16 0x3C09, nibble 9 -> 0x3C11 & 0xFFF0 = 0x3C10
    # (truncation would give 0x3C00)
    assert O.fit_int4_asym(grid(1033 / 1024), contract=contract) == (0x3C10, 0)
    # s = 129/128: fp16 0x3C08, nibble 8 (a tie) -> 0x3C10 (rounding the
    # nibble to even would keep 0x3C00)
    assert O.fit_int4_asym(grid(129 / 128), contract=contract) == (0x3C10, 0)
    # s = 1031/1024: fp16 0x3C07, nibble 7 -> 0x3C0F & 0xFFF0 = 0x3C00
    assert O.fit_int4_asym(grid(1031 / 1024), contract=contract) == (0x3C00, 0)
    # without the reservation the FP16 bits are returned as they are
    assert O.fit_int4_asym(grid(1033 / 1024), reserve_nibble=False, contract=contract) == (0x3C09, 0)


@pytest.mark.parametrize("contract", [True, False])
def test_fit_int4_asym_three_refinements(contract):
    # A group whose scale moves in each of the three least-squares
    # refinements (kernels_dpas.cpp:239-251). Integer weights keep every num
    # and den an exact integer (so the FMA contraction cannot matter); only
    # the divisions round, and no rint below is within 0.05 of a tie.
    #   w = [5,0,0,-4,7,7,7,0,0,0,-4,0,0,0,0,0]: lo = -4, hi = 7
    #   s0 = 11/15 = 0.73333335
    #   refinement 1: zi = rint(4/s0) - 8 = rint(5.4545) - 8 = -3
    #     w/s0 + zi: 5 -> 3.818 -> q 4, c 7; -4 -> -8.455 -> q -8, c -5;
    #     7 -> 6.545 -> q 7, c 10; 0 -> q -3, c 0
    #     num = 5*7 + 2*(-4)(-5) + 3*7*10 = 285, den = 49 + 2*25 + 3*100 = 399
    #     s1 = 285/399 = 0.71428573
    #   refinement 2: zi = rint(4/s1) - 8 = rint(5.6) - 8 = -2
    #     5 -> 7.0 - 2 = 5 -> c 7; -4 -> -7.6 -> q -8, c -6; 7 -> 7.8 -> q 7, c 9
    #     num = 35 + 2*24 + 3*63 = 272, den = 49 + 2*36 + 3*81 = 364
    #     s2 = 272/364 = 0.74725276
    #   refinement 3: zi = rint(4/s2) - 8 = rint(5.353) - 8 = -3
    #     5 -> 3.691 -> q 4, c 7; -4 -> -8.353 -> q -8, c -5; 7 -> 6.368 -> q 6, c 9
    #     num = 35 + 40 + 189 = 264, den = 49 + 50 + 243 = 342
    #     s3 = 264/342 = 0.7719298
    #   z = rint(4/s3) - 8 = rint(5.182) - 8 = -3
    #   fp16(s3) = 0x3A2D (1.5439 * 2^-1, mantissa rint(556.9) = 557)
    #   -> (0x3A2D + 8) & 0xFFF0 = 0x3A30
    # Two refinements would store fp16(s2) = 0x39FA -> 0x3A00; four would
    # give 0x3A50.
    w = np.array([5, 0, 0, -4, 7, 7, 7, 0, 0, 0, -4, 0, 0, 0, 0, 0], np.float32)
    assert O.fit_int4_asym(w, contract=contract) == (0x3A30, -3)
    assert O.fit_int4_asym(w, reserve_nibble=False, contract=contract) == (0x3A2D, -3)
    # the same group inside K32 and K64 groups (zeros do not change num, den,
    # lo or hi)
    for n in (32, 64):
        wn = np.zeros(n, np.float32)
        wn[:16] = w
        assert O.fit_int4_asym(wn, contract=contract) == (0x3A30, -3)


def test_fit_int4_asym_range_includes_zero():
    # lo and hi start at 0, so the fitted range always includes 0
    # (kernels_dpas.cpp:231-236); a range seeded from the data would differ.
    # All +2: lo = 0, hi = 2, s0 = 2/15 = 0.13333334; zi = rint(0/s0) - 8 = -8;
    # every w/s0 - 8 = 7 -> q 7, c 15; num = 16*2*15 = 480, den = 16*225 =
    # 3600, s = 480/3600 = 0.13333334 again (three times); z = -8;
    # fp16(s) = 0x3044 -> 0x3040. (A range seeded from the data, lo = hi = 2,
    # gives s = 0 -> 1 and stays there: 0x3C00.)
    assert O.fit_int4_asym(np.full(16, 2.0, np.float32)) == (0x3040, -8)
    # All -2: lo = -2, hi = 0, s0 = 2/15; zi = rint(2/s0) - 8 = rint(15) - 8 =
    # 7; w/s0 + 7 = -8 -> q -8, c -15; num = 480, den = 3600; z = 7 -> 0x3040.
    assert O.fit_int4_asym(np.full(16, -2.0, np.float32)) == (0x3040, 7)


def test_fit_int4_asym_reserves_nibble_and_keeps_zero():
    rng = np.random.default_rng(6)
    for _ in range(200):
        wf = (rng.standard_normal(32) * rng.uniform(0.01, 2)).astype(np.float32)
        wf[rng.integers(0, 32)] = 0.0
        sh, z = O.fit_int4_asym(wf)
        assert sh & 0xF == 0 and -8 <= z <= 7
        s = O.f16_to_f32(np.array([sh], np.uint16))[0]
        q = np.clip(np.rint(wf / s + z), -8, 7)
        assert np.all((q - z)[wf == 0] == 0)
        # at most one clamped code at each end of a fitted range; all others
        # within half a step of the weight
        inside = (q > -8) & (q < 7)
        assert np.all(np.abs(wf - s * (q - z))[inside] <= s * 0.5 * (1 + 1e-5))


def random_payload(rng, M, K):
    Kt = K // 32
    payload = rng.integers(0, 256, size=(M // 16) * Kt * 384, dtype=np.uint8)
    scale_cols = Kt // 4
    bs = rng.uniform(0.001, 0.05, size=((M + 127) // 128) * scale_cols).astype(np.float32)
    return payload, bs, scale_cols


def decode_payload(payload, bs, scale_cols, M, K):
    Kt = K // 32
    L = O.lib()
    wf = np.empty((M, K), np.float32)
    for r in range(M):
        for k in range(K):
            kt = k // 32
            sc = kt if scale_cols == Kt else kt >> 2
            b = bs[(r >> 4 >> 3) * scale_cols + sc]
            wf[r, k] = np.float32(L.orc_e2m3(L.orc_e2m3_code_at(payload.ctypes.data, Kt, r, k))) * b
    return wf


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_repack_e2m3_quantizes_against_stored_scale(mode):
    rng = np.random.default_rng(7 + mode)
    M, K = 32, 256
    payload, bs, scale_cols = random_payload(rng, M, K)
    codes, scales = O.repack_e2m3(payload, bs, scale_cols, M, K, mode)
    group = {0: 32, 1: 16, 2: 64}[mode]
    wf = decode_payload(payload, bs, scale_cols, M, K)
    ws = O.f16_to_f32(scales & 0xFFF0)
    z = (scales & 0xF).astype(np.int32)
    z = np.where(z >= 8, z - 16, z)
    wsk = np.repeat(ws, group, axis=1)
    zk = np.repeat(z, group, axis=1)
    assert np.array_equal(codes, np.clip(np.rint(wf / wsk + zk), -8, 7).astype(np.int8))
    for r in range(M):
        for g in range(K // group):
            sh, zz = O.fit_int4_asym(wf[r, g * group:(g + 1) * group])
            assert scales[r, g] == (sh | (zz & 0xF))


def test_ref_layout_roundtrip_and_dpas_contract():
    rng = np.random.default_rng(8)
    M, K = 32, 128
    for group in (32, 64):
        codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
        scales = rng.integers(0, 65536, (M, K // group)).astype(np.uint16)
        rc, rs = O.pack_ref_layout(codes, scales, group)
        c2, s2 = O.unpack_ref_layout(rc, rs, M, K, group)
        assert np.array_equal(codes, c2) and np.array_equal(scales, s2)
    # one-hot: the B-operand contract (kernels_dpas.cpp:13-15, lane-major
    # 331-337): row n of a row-group owns dwords n*4..n*4+3 of its 256-byte
    # (row-group, K32) tile; k sits in dword (k%32)/8 at nibble k%8.
    Kt = K // 32
    for row, k in [(0, 0), (5, 9), (17, 63), (31, 127), (16, 32)]:
        codes = np.zeros((M, K), np.int8)
        codes[row, k] = -1          # nibble 0xF
        rc, _ = O.pack_ref_layout(codes, np.zeros((M, K // 32), np.uint16), 32)
        dword = ((row // 16) * Kt + k // 32) * 64 + (row % 16) * 4 + (k % 32) // 8
        words = rc.view(np.uint32)
        assert np.count_nonzero(words) == 1
        assert words[dword] == 0xF << (4 * (k % 8))


# ------------------------------------------------------------------ split plans
def test_split_heuristics_known_values():
    # derived by reading kernels_dpas.cpp:170-173 and 1226-1250 at the
    # BASELINE shapes (row-groups = rows/16, t-groups = tokens/8, K32 tiles)
    assert [O.gemv_splits(g) for g in (1, 4, 5, 256, 320, 2176, 4095, 4096, 9999)] == \
        [16, 16, 8, 8, 8, 8, 8, 1, 1]
    assert O.gemm_splits(1088, 1, 160) == 2       # cfg1, one gate/up weight at T=8
    assert O.gemm_splits(2176, 1, 160) == 1       # cfg1 if the two were concatenated
    assert O.gemm_splits(320, 64, 544) == 1       # cfg2, M=512
    assert O.gemm_splits(320, 256, 160) == 1      # cfg3
    assert O.gemm_splits(320, 1, 160) == 8        # one 8-row segment at N=5120
    assert O.gemm_splits(3, 1, 4) == 4            # capped by the K32 tile count
    assert O.gemm_splits(1, 1, 160) == 16
    assert O.gemm_splits(2048, 1, 160) == 1
    assert O.gemm_splits(320, 1, 160, forced=4) == 4
    assert O.gemm_splits(320, 1, 2, forced=16) == 2
    assert O.gemm_splits(320, 1, 160, forced=3) == 8   # invalid override ignored


def test_segment_splits():
    seg = [0, 17, 81, 381, 893, 1917, 3965]          # cfg4 token counts
    sp = O.segment_splits(3965, 17408, 5120, seg)
    assert np.all(sp == 1)
    sp = O.segment_splits(24, 5120, 5120, [0, 8, 24])
    assert np.all(sp[:8] == 8) and np.all(sp[8:] == 4)
    for bad in ([1, 8, 24], [0, 8, 8, 24], [0, 8, 23]):
        with pytest.raises(ValueError):
            O.segment_splits(24, 5120, 5120, bad)


@pytest.mark.parametrize("K,unit,S", [(4096, 128, 8), (5120, 128, 2), (17408, 64, 8),
                                      (5120, 128, 1), (17408, 64, 1)])
def test_config_split_boundaries_fall_on_units(K, unit, S):
    # the reference splits in K32 tiles, [Kt*s/S, Kt*(s+1)/S); at every
    # BASELINE config the boundary is also a weight-group boundary, so the
    # unit-based split of the oracle is the same partition
    Kt, Nu = K // 32, K // unit
    for s in range(S + 1):
        assert (Kt * s // S) * 32 == (Nu * s // S) * unit


# ------------------------------------------------------------------ projection
@pytest.mark.parametrize("name", ["ref32", "ref64", "cfg128", "cfg64"])
def test_partials_match_numpy_matmul(golden, name):
    g = lambda k: golden[f"part_{name}_{k}"]
    group, block, zp = g("meta")
    P = O.partials(g("codes"), g("scales"), int(group), int(zp), g("q"), np.zeros(1, np.float32),
                   g("asum"), int(block))
    assert np.array_equal(P, g("P"))


@pytest.mark.parametrize("name", ["ref32", "ref64", "cfg128", "cfg64"])
@pytest.mark.parametrize("variant", [O.VAR_GEMV, O.VAR_FANOUT, O.VAR_GEMM])
@pytest.mark.parametrize("splits", [1, 2, 4])
def test_exact_cases(golden, name, variant, splits):
    g = lambda k: golden[f"exact_{name}_{k}"]
    group, block, zp = (int(v) for v in g("meta"))
    y = O.project(g("codes"), g("scales"), group, zp, g("q"), g("ascale"), g("asum"), block,
                  variant, splits)
    assert np.array_equal(bits(y), bits(g("y")))


def test_order_cases(golden):
    g = lambda k: golden[f"order_{k}"]
    for var, S, want in zip(g("variants"), g("splits"), g("expected")):
        variant = [O.VAR_GEMV, O.VAR_FANOUT, O.VAR_GEMM][int(var)]
        y = O.project(g("codes"), g("scales"), 32, O.SCALE_FP16, g("q"), g("ascale"), g("asum"),
                      0, variant, int(S))
        assert np.all(y == want), (var, S, y[0, 0], want)


@pytest.mark.parametrize("block,group,enc", [(32, 32, 1), (32, 64, 1), (0, 128, 0), (0, 64, 0)])
def test_all_ones_gives_K(block, group, enc):
    # xpu/probe/w4a4_gemm_probe.cpp:13-17: every code 1, every scale 1.0 with
    # zero point 0 -> each output equals K
    M, K, T = 32, 512, 3
    codes = np.ones((M, K), np.int8)
    scales = np.full((M, K // group), 0x3C00, np.uint16)
    q = np.ones((T, K), np.int8)
    asum = np.full((T, K // 32), 32, np.int32)
    ascale = np.ones((T, K // 32) if block == 32 else T, np.float32)
    for variant in (O.VAR_GEMV, O.VAR_FANOUT, O.VAR_GEMM):
        for S in (1, 2, 8, 16):
            y = O.project(codes, scales, group, enc, q, ascale, asum, block, variant, S)
            assert np.all(y == K)


def test_bf16_output_and_residual():
    rng = np.random.default_rng(9)
    M, K, T = 64, 256, 2
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    scales = (np.abs(rng.standard_normal((M, K // 128))) * 0.02).astype(np.float16).view(np.uint16)
    q, s, sm = O.quantize_act(rng.standard_normal((T, K)).astype(np.float32), 0)
    res = rng.standard_normal((T, M)).astype(np.float32)
    for variant in (O.VAR_GEMV, O.VAR_GEMM):
        y = O.project(codes, scales, 128, 0, q, s, sm, 0, variant, 2)
        yb = O.project(codes, scales, 128, 0, q, s, sm, 0, variant, 2, out_bf16=True)
        assert np.array_equal(yb, O.f32_to_bf16(y))
        yr = O.project(codes, scales, 128, 0, q, s, sm, 0, variant, 2, residual=res)
        assert np.array_equal(bits(yr), bits((y + res).astype(np.float32)))


def gemm_check_input(T, K):
    """qwn_gemm_check's deterministic activations (kernels_dpas.cpp:2280-2286)."""
    k = np.arange(K, dtype=np.int64)[None, :]
    t = np.arange(T, dtype=np.int64)[:, None]
    mag = np.exp2((((k * 7) + t * 3) % 13) - 6.0)
    sgn = np.where((((k * 2654435761 + t) & 0xFFFFFFFF) >> 31) != 0, -1.0, 1.0)
    return np.where(k % 97 == 0, 0.0, sgn * mag).astype(np.float32)


def test_gemm_agrees_with_gemv_reference_gate():
    # the reference's own gate: RC8 GEMM vs per-row GEMV, cos >= 0.9999 per
    # token row (kernels_dpas.cpp:2264-2333), here on asymmetric K32 weights
    rng = np.random.default_rng(10)
    M, K, T = 256, 1024, 8
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    mags = (np.abs(rng.standard_normal((M, K // 32))) * 0.02).astype(np.float16).view(np.uint16)
    scales = ((mags & 0xFFF0) | (rng.integers(-8, 8, mags.shape) & 0xF)).astype(np.uint16)
    q, s, sm = O.quantize_act(gemm_check_input(T, K), 32)
    ref = O.project(codes, scales, 32, 1, q, s, sm, 32, O.VAR_GEMV, O.gemv_splits(M // 16))
    got = O.project(codes, scales, 32, 1, q, s, sm, 32, O.VAR_GEMM,
                    O.gemm_splits(M // 16, T // 8, K // 32))
    for t in range(T):
        a, b = ref[t].astype(np.float64), got[t].astype(np.float64)
        assert a @ b / np.sqrt((a @ a) * (b @ b)) >= 0.9999
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3)) < 1e-3


# ---- W4A4: s4 activation quantizer and the W4A4 GEMM arithmetic -------------

def test_s4_quantizer_known_answers():
    # x_quantize_act_chunk_s4 (kernels_dpas.cpp:1149-1197, S4): per (token, K64)
    # s = absmax/7, q = clamp(rint(v/s), -7, 7). With absmax 7 the scale is 1 and
    # the codes are rint of the values themselves: ties go to even.
    x = np.zeros((2, 128), np.float32)
    x[0, :8] = [7.0, 0.5, 1.5, 2.5, -2.5, -0.5, 3.49, -6.51]
    x[0, 64:66] = [-14.0, 5.0]          # block 1: s = 2, 5/2 = 2.5 -> 2
    x[1, 3] = np.nan                     # block 0 of token 1: NaN beside zeros
    x[1, 64 + 9] = 1e-30                 # tiny absmax, s = 1e-30/7
    q, s, sm = O.quantize_act_s4(x)
    assert s[0, 0] == 1.0 and s[0, 1] == 2.0
    assert list(q[0, :8]) == [7, 0, 2, 2, -2, 0, 3, -7]
    assert list(q[0, 64:66]) == [-7, 2] and not q[0, 66:].any()
    assert sm[0, 0] == 7 + 0 + 2 + 2 - 2 + 0 + 3 - 7 and sm[0, 1] == -5
    # NaN is ignored by the max (fmax) and lands on the low clamp bound (sycl
    # clamp = fmin(fmax(x, lo), hi)); an all-zero max gives scale 1
    assert s[1, 0] == 1.0 and q[1, 3] == -7 and sm[1, 0] == -7
    assert s[1, 1] == np.float32(1e-30) / np.float32(7) and q[1, 64 + 9] == 7


def test_s4_quantizer_invariants():
    rng = np.random.default_rng(21)
    T, K = 5, 640
    x = (rng.standard_normal((T, K)) * np.exp2(rng.integers(-20, 20, (T, 1)))).astype(np.float32)
    x[2, 64:128] = 0.0
    q, s, sm = O.quantize_act_s4(x)
    assert np.abs(q).max() <= 7
    xb = x.reshape(T, K // 64, 64)
    qb = q.reshape(T, K // 64, 64).astype(np.int64)
    mx = np.abs(xb).max(axis=2)
    want_s = np.where(mx > 0, mx / np.float32(7), np.float32(1)).astype(np.float32)
    assert np.array_equal(s, want_s)
    assert np.array_equal(sm, qb.sum(axis=2))
    # the absmax element maps to +-7; every code is within half a step
    arg = np.abs(xb).argmax(axis=2)
    top = np.take_along_axis(qb, arg[..., None], axis=2)[..., 0]
    assert np.all((np.abs(top) == 7) | (mx == 0))
    err = np.abs(xb.astype(np.float64) - qb * s[..., None].astype(np.float64))
    assert np.all(err <= 0.5 * s[..., None] * (1 + 1e-6))
    assert not q[2, 64:128].any() and s[2, 1] == 1.0


def w4a4_weight(rng, M, K):
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    mags = (np.abs(rng.standard_normal((M, K // 64))) * 0.02).astype(np.float16).view(np.uint16)
    scales = ((mags & 0xFFF0) | (rng.integers(-8, 8, mags.shape) & 0xF)).astype(np.uint16)
    return codes, scales


def test_w4a4_all_ones_gives_K():
    # xpu/probe/w4a4_gemm_probe.cpp:13-17 (s4 x s4 arm)
    M, K, T = 32, 512, 8
    codes = np.ones((M, K), np.int8)
    scales = np.full((M, K // 64), 0x3C00, np.uint16)
    q, s, sm = O.quantize_act_s4(np.ones((T, K), np.float32) * 7)
    assert np.all(q == 7) and np.all(s == 1.0)
    y = O.project(codes, scales, 64, O.SCALE_FP16_ZP4, q // 7, s, sm // 7, 64, O.VAR_GEMM, 1)
    assert np.all(y == K)


def test_w4a4_zero_point_exact_case():
    # exact-rational case: scales 2^-k and codes small enough that every FP32
    # step is exact, so y must equal the int64 product sum_u (w - zp_u) . a_u
    # * ws_u * as_u, pinning the zero-point sign and the per-K64 sum indexing
    rng = np.random.default_rng(22)
    M, K, T = 48, 384, 8
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    zp = rng.integers(-8, 8, (M, K // 64))
    ws_exp = rng.integers(-4, 2, (M, K // 64))
    scales = ((np.exp2(ws_exp).astype(np.float16).view(np.uint16) & 0xFFF0) | (zp & 0xF)).astype(np.uint16)
    q = rng.integers(-7, 8, (T, K)).astype(np.int8)
    sm = q.reshape(T, K // 64, 64).sum(axis=2).astype(np.int32)
    s = np.exp2(rng.integers(-3, 3, (T, K // 64))).astype(np.float32)
    y = O.project(codes, scales, 64, O.SCALE_FP16_ZP4, q, s, sm, 64, O.VAR_GEMM, 1)
    w = codes.reshape(M, K // 64, 64).astype(np.int64) - zp[..., None]
    a = q.reshape(T, K // 64, 64).astype(np.int64)
    d = np.einsum("muk,tuk->tmu", w, a)
    want = (d * np.exp2(ws_exp)[None] * s[:, None, :]).sum(axis=2)
    assert np.array_equal(y, want.astype(np.float32))


def test_w4a4_agrees_with_w4a8_gemv_gate():
    # the reference's gate qwn_gemm_w4a4_check (kernels_dpas.cpp:2335-2409): the
    # W4A4 GEMM against the W4A8 GEMV on the same K64 weight, worst token-row
    # cosine >= 0.995 on the deterministic gate input, at the gate's K = 5120
    # (the s4 noise it is sized for; the reference measured 0.9962-0.9963)
    rng = np.random.default_rng(23)
    M, K, T = 256, 5120, 8
    codes, scales = w4a4_weight(rng, M, K)
    x = gemm_check_input(T, K)
    q8, s8, sm8 = O.quantize_act(x, 32)
    ref = O.project(codes, scales, 64, 1, q8, s8, sm8, 32, O.VAR_GEMV, O.gemv_splits(M // 16))
    q4, s4, sm4 = O.quantize_act_s4(x)
    got = O.project(codes, scales, 64, 1, q4, s4, sm4, 64, O.VAR_GEMM, 1)
    cos = [ref[t].astype(np.float64) @ got[t] /
           np.sqrt((ref[t].astype(np.float64) @ ref[t]) * (got[t].astype(np.float64) @ got[t]))
           for t in range(T)]
    assert min(cos) >= 0.995 and min(cos) < 0.99999, cos


def test_w4a4_rejects_other_tiers_and_variants():
    rng = np.random.default_rng(24)
    M, K, T = 32, 256, 8
    codes, scales = w4a4_weight(rng, M, K)
    q, s, sm = O.quantize_act_s4(rng.standard_normal((T, K)).astype(np.float32))
    with pytest.raises(ValueError, match="rc=-2"):
        O.project(codes, scales, 64, 1, q, s, sm, 64, O.VAR_GEMV, 1)
    with pytest.raises(ValueError, match="rc=-1"):
        O.project(codes, scales[:, ::2].copy(), 128, 1, q, s, sm, 64, O.VAR_GEMM, 1)
    with pytest.raises(ValueError, match="rc=-1"):
        O.project(codes, scales & 0xFFF0, 64, 0, q, s, sm, 64, O.VAR_GEMM, 1)


# ---- W8A8 tier: int8 fit and projection -------------------------------------

def test_fit_int8_known_answers():
    # w8_repack_kernel (kernels_dpas.cpp:346-399): a group on an exact grid of
    # step 1/16 keeps that step through both refinements
    wf = (0.5 * (np.arange(32) - 16)).astype(np.float32)
    assert O.fit_int8(wf) == 0x2C00                              # fp16(0.0625)
    # the negative side divides by 128: a lone -1 with grid-aligned positives
    # gives s = 1/128 and code -128 (the positive side's 127 would not reach)
    wf = (np.arange(32) % 5 / 128.0).astype(np.float32)
    wf[7] = -1.0
    assert O.fit_int8(wf) == 0x2000                              # fp16(1/128)
    assert O.fit_int8(np.zeros(32, np.float32)) == 0x3C00        # scale 1


@pytest.mark.parametrize("contract", [True, False])
def test_fit_int8_two_refinements_and_negative_side(contract):
    # w8_repack_kernel's fit (kernels_dpas.cpp:358-380) on a K32 group of
    # integers (num and den exact; only the divisions round, no rint within
    # 0.01 of a tie):
    #   w: -16 at 6 and 7, 23 at 10, 26 and 30, -39 at 29, 0 elsewhere
    #   hi = 23, neg = 39: s0 = max(23/127, 39/128) = 39/128 = 0.3046875
    #   refinement 1: -16/s0 = -52.513 -> -53; 23/s0 = 75.487 -> 75; -39 -> -128
    #     num = 2*16*53 + 3*23*75 + 39*128 = 11863
    #     den = 2*53^2 + 3*75^2 + 128^2 = 38877; s1 = 0.30514187
    #   refinement 2: -16/s1 = -52.435 -> -52; 23/s1 = 75.375 -> 75;
    #     -39/s1 = -127.81 -> -128
    #     num = 2*16*52 + 5175 + 4992 = 11831, den = 5408 + 16875 + 16384 = 38667
    #     s2 = 11831/38667 = 0.3059715
    #   fp16(s2) = 1.22389 * 2^-2: mantissa rint(229.26) = 229 -> 0x34E5
    # One refinement would store fp16(s1) = 0x34E2, three 0x34E9; the
    # negative side divided by 127 instead of 128 also ends at 0x34E9.
    w = np.zeros(32, np.float32)
    w[[6, 7]] = -16
    w[[10, 26, 30]] = 23
    w[29] = -39
    assert O.fit_int8(w, contract=contract) == 0x34E5


def test_fit_int8_invariants():
    rng = np.random.default_rng(31)
    for _ in range(200):
        wf = (rng.standard_normal(32) * np.exp2(rng.integers(-12, 4))).astype(np.float32)
        sh = O.fit_int8(wf)
        st = np.float32(np.uint16(sh).view(np.float16))
        assert st > 0
        q = np.clip(np.rint(wf / st), -128, 127)
        inside = (q > -128) & (q < 127)
        assert np.all(np.abs(wf[inside] - q[inside] * st) <= 0.5 * st * (1 + 1e-6))
        # the fit lands within a few percent of the absmax step
        s0 = max(wf.max() / 127, -wf.min() / 128)
        assert 0.9 * s0 <= st <= 1.1 * s0


def test_repack_e2m3_s8_uses_the_fit_per_k32():
    rng = np.random.default_rng(32)
    M, K = 32, 256
    payload, bs, scale_cols = random_payload(rng, M, K)
    codes, scales = O.repack_e2m3_s8(payload, bs, scale_cols, M, K)
    wf = decode_payload(payload, bs, scale_cols, M, K)
    for row in (0, 17, 31):
        for kt in range(K // 32):
            g = wf[row, kt * 32:(kt + 1) * 32]
            assert scales[row, kt] == O.fit_int8(g)
            st = np.float32(np.uint16(scales[row, kt]).view(np.float16))
            assert np.array_equal(codes[row, kt * 32:(kt + 1) * 32],
                                  np.clip(np.rint(g / st), -128, 127).astype(np.int8))


def w8_weight(rng, M, K):
    codes = rng.integers(-128, 128, (M, K)).astype(np.int8)
    scales = (np.abs(rng.standard_normal((M, K // 32))) * 0.002).astype(np.float16).view(np.uint16)
    return codes, scales


def test_w8a8_exact_case():
    # exact-rational: power-of-two scales and small activation codes keep every
    # FP32 step exact, so GEMV (alternating chains) and GEMM agree with the
    # int64 product sum_kt d_kt * ws_kt * as_kt
    rng = np.random.default_rng(33)
    M, K, T = 32, 512, 3
    codes = rng.integers(-128, 128, (M, K)).astype(np.int8)
    e = rng.integers(-6, 0, (M, K // 32))
    scales = np.exp2(e).astype(np.float16).view(np.uint16)
    q = rng.integers(-3, 4, (T, K)).astype(np.int8)
    sm = q.reshape(T, K // 32, 32).sum(axis=2).astype(np.int32)
    s = np.exp2(rng.integers(-4, 2, (T, K // 32))).astype(np.float32)
    d = np.einsum("mkj,tkj->tmk", codes.reshape(M, K // 32, 32).astype(np.int64),
                  q.reshape(T, K // 32, 32).astype(np.int64))
    want = (d * np.exp2(e)[None] * s[:, None, :]).sum(axis=2).astype(np.float32)
    for variant, S in ((O.VAR_GEMV, 1), (O.VAR_GEMV, 4), (O.VAR_GEMM, 1)):
        y = O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, variant, S)
        assert np.array_equal(y, want), (variant, S)


def test_w8a8_all_ones_gives_K_and_tier_checks():
    M, K, T = 32, 256, 2
    codes = np.ones((M, K), np.int8)
    scales = np.full((M, K // 32), 0x3C00, np.uint16)
    q = np.ones((T, K), np.int8)
    s = np.ones((T, K // 32), np.float32)
    sm = np.full((T, K // 32), 32, np.int32)
    for variant in (O.VAR_GEMV, O.VAR_GEMM):
        assert np.all(O.project(codes, scales, 32, O.SCALE_S8, q, s, sm, 32, variant, 2) == K)
    with pytest.raises(ValueError, match="rc=-1"):          # W8 needs block-32 activations
        O.project(codes, scales, 32, O.SCALE_S8, q, np.ones(T, np.float32), sm, 0, O.VAR_GEMV, 1)
    with pytest.raises(ValueError, match="rc=-1"):          # and K32 scales
        O.project(codes, scales[:, ::2].copy(), 64, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMV, 1)


# ---- K16 tier: GEMV over K16 halves -----------------------------------------

def k16_case(terms, as_tiles, K=384):
    """One weight row whose K16 unit u contributes exactly terms[u] (code w at
    the unit's first element, activation code 1 there and 0 elsewhere, zero
    point 0): terms[u] = w * ws_u * as_{u/2}. Returns oracle inputs for T = 1."""
    Nu = K // 16
    codes = np.zeros((16, K), np.int8)
    ws = np.ones((16, Nu), np.float32)
    q = np.zeros((1, K), np.int8)
    for u, v in enumerate(terms):
        if v == 0:
            continue
        w = 4 if v / as_tiles[u // 2] >= 4 else 1
        codes[0, 16 * u] = w
        ws[0, u] = v / as_tiles[u // 2] / w
        q[0, 16 * u] = 1
    scales = (ws.astype(np.float16).view(np.uint16) & 0xFFF0).astype(np.uint16)
    assert np.all(O.f16_to_f32(scales[0]) == ws[0])
    s = np.repeat(np.asarray(as_tiles, np.float32)[None, :K // 32], 1, axis=0)
    sm = q.reshape(1, K // 32, 32).sum(axis=2).astype(np.int32)
    return codes, scales, q, s, sm


def test_k16_splits_fall_on_k32_tiles():
    # x_gemv_w4a8_core_k16 (kernels_dpas.cpp:712-713) splits K32 tiles: K = 384
    # (12 tiles) in 8 splits gives tile boundaries 0,1,3,4,...; split 0 holds
    # units 0-1 (2^24) and split 1 units 2-5 (1 + 1), so the ordered sum is
    # 2^24 + 2 exactly. Boundaries taken on K16 units (0,3,6,...) would put the
    # first 1 in split 0, where 2^24 + 1 rounds back to 2^24.
    terms = [2.0 ** 24, 0, 1.0, 1.0] + [0] * 20
    codes, scales, q, s, sm = k16_case(terms, [2.0 ** 11, 1.0] + [1.0] * 10)
    y = O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, 8)
    assert y[0, 0] == np.float32(2.0 ** 24 + 2)


def test_k16_single_serial_accumulator():
    # one accumulator per split (kernels_dpas.cpp:704, 733-739): units 1, 2^24,
    # 1 give (1 + 2^24) + 1 = 2^24; the W4A8 GEMV's alternating pair would
    # give (1 + 1) + 2^24 = 2^24 + 2
    terms = [1.0, 2.0 ** 24, 1.0] + [0] * 21
    codes, scales, q, s, sm = k16_case(terms, [2.0 ** 12, 1.0] + [1.0] * 10)
    y = O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, 1)
    assert y[0, 0] == np.float32(2.0 ** 24)


def test_k16_zero_points_per_half_and_tier_checks():
    # exact-rational: each K16 half subtracts its own zero point times its own
    # code sum, then scales by ws_half * as_tile
    rng = np.random.default_rng(51)
    M, K, T = 32, 256, 2
    codes = rng.integers(-8, 8, (M, K)).astype(np.int8)
    zp = rng.integers(-8, 8, (M, K // 16))
    e = rng.integers(-4, 1, (M, K // 16))
    scales = ((np.exp2(e).astype(np.float16).view(np.uint16) & 0xFFF0) | (zp & 0xF)).astype(np.uint16)
    q = rng.integers(-3, 4, (T, K)).astype(np.int8)
    s = np.exp2(rng.integers(-3, 2, (T, K // 32))).astype(np.float32)
    sm = q.reshape(T, K // 32, 32).sum(axis=2).astype(np.int32)
    w = codes.reshape(M, K // 16, 16).astype(np.int64) - zp[..., None]
    d = np.einsum("muk,tuk->tmu", w, q.reshape(T, K // 16, 16).astype(np.int64))
    want = (d * np.exp2(e)[None] * np.repeat(s, 2, axis=1)[:, None, :]).sum(axis=2).astype(np.float32)
    for S in (1, 2, 4):
        y = O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMV, S)
        assert np.array_equal(y, want), S
    with pytest.raises(ValueError, match="rc=-1"):        # GEMV only
        O.project(codes, scales, 16, 1, q, s, sm, 32, O.VAR_GEMM, 1)
    with pytest.raises(ValueError, match="rc=-1"):        # block-32 activations only
        O.project(codes, scales, 16, 1, q, np.ones(T, np.float32), sm, 0, O.VAR_GEMV, 1)
