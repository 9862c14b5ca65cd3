"""Writes the golden fixtures in tests/golden/*.npz.

The reference holds no golden vectors for the W4A8 path (its snapshots are
generated, not committed) and cannot run here, so every expected value below
is derived WITHOUT the oracle:
  * quantizer edges: the input pattern of the reference's chunk_quant_bench
    (xpu/probe/chunk_quant_bench.cpp:54-99), expected codes from numpy's IEEE
    float32 division and round-half-even, written independently of the oracle;
  * integer partials: numpy int64 matrix products;
  * "exact" projections: inputs chosen so every float operation is exact, the
    expected output is an exact rational (fractions.Fraction);
  * "order" projections: hand-built unit partials whose fp32 result depends
    on the accumulation order, with the expected value derived by hand from
    the reference's chain rules (kernels_dpas.cpp:644-652, 1030-1074,
    1313-1321, 1477-1486);
  * all-ones: y == K for every variant (xpu/probe/w4a4_gemm_probe.cpp:13-17).

Run: python tests/golden/make_golden.py   (writes next to this file)
"""
from __future__ import annotations

import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


# ---------------------------------------------------------------- quantizer
def lcg_input(K: int, T: int, exceptional: bool) -> np.ndarray:
    """chunk_quant_bench.cpp:54-99 input pattern (seed 391), as float32 [T][K]."""
    n = K * T
    out = np.empty(n, np.float32)
    seed = 391
    for i in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(((seed >> 8) - 8388608) / 1048576.0)
    fmax = np.finfo(np.float32).max
    dmin = np.float32(np.finfo(np.float32).smallest_subnormal)
    for block in range(n // 64):
        p = out[block * 64:(block + 1) * 64]
        c = block % 16
        if c == 0:
            p[:] = 0.0
            p[0] = -0.0
        elif c == 1:
            for j in range(64):
                p[j] = np.float32((-1.0 if j & 1 else 1.0) * 1.0e-20 * (j + 1))
        elif c == 2:
            for j in range(64):
                p[j] = np.float32(j - 32) + np.float32(0.5)
            p[0] = p[32] = 127.0
        elif c == 3:
            p[:] = dmin
            p[0] = -dmin
        elif c == 4:
            p[0] = fmax
            p[32] = -fmax
        if exceptional:
            p[block % 64] = np.nan
            if block % 67 == 0:
                p[:] = np.nan
            elif block % 67 == 1:
                p[(block + 17) % 64] = np.inf
            elif block % 67 == 2:
                p[(block + 31) % 64] = -np.inf
    return out.reshape(T, K)


def np_quantize(x: np.ndarray, block: int):
    """Symmetric int8: s = absmax/127 (1 if absmax <= 0 or all NaN),
    q = clamp(rint(x/s), -127, 127) where a NaN quotient lands on -127."""
    T, K = x.shape
    width = 32 if block == 32 else K
    q = np.empty((T, K), np.int8)
    scale = np.empty((T, K // width), np.float32)
    with np.errstate(all="ignore"):
        for t in range(T):
            for b in range(K // width):
                v = x[t, b * width:(b + 1) * width]
                a = np.abs(v)
                a = a[~np.isnan(a)]
                mx = np.float32(a.max()) if a.size else np.float32(-np.inf)
                s = (mx / np.float32(127.0)) if mx > 0 else np.float32(1.0)
                r = np.rint(v / s)
                r = np.where(np.isnan(r), np.float32(-127), np.clip(r, -127, 127))
                q[t, b * width:(b + 1) * width] = r.astype(np.int8)
                scale[t, b] = s
    sums = q.reshape(T, K // 32, 32).astype(np.int32).sum(axis=2).astype(np.int32)
    return q, (scale if block == 32 else scale[:, 0].copy()), sums


def quant_ties():
    """Absmax 127 makes the scale exactly 1, so x/s = x and rint's
    round-half-even shows directly: 2.5 -> 2, 3.5 -> 4, -2.5 -> -2."""
    x = np.zeros((1, 32), np.float32)
    vals = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5, -126.5, 200.0 / 2.0]
    x[0, :len(vals)] = vals
    expect = np.zeros((1, 32), np.int8)
    expect[0, :len(vals)] = [127, 2, 4, -2, -4, 0, 2, 0, 126, -126, 100]
    return x, expect


# ---------------------------------------------------------------- partials
def np_partials(codes, scales, group, zp_enc, q, asum, block):
    M, K = codes.shape
    T = q.shape[0]
    unit = 32 if block == 32 else group
    Nu = K // unit
    w = codes.astype(np.int64).reshape(M, Nu, unit)
    a = q.astype(np.int64).reshape(T, Nu, unit)
    P = np.einsum("nuj,tuj->tnu", w, a)
    if zp_enc:
        z = (scales.astype(np.int64) & 0xF)
        z = np.where(z >= 8, z - 16, z)                     # [M][K/group]
        zu = np.repeat(z, group // unit, axis=1) if group > unit else z[:, (np.arange(Nu) * unit) // group]
        su = asum.astype(np.int64).reshape(T, Nu, unit // 32).sum(axis=2)   # [T][Nu]
        P = P - zu[None, :, :] * su[:, None, :]
    return P.astype(np.int32)


def random_weight(rng, M, K, group, zp_enc):
    codes = rng.integers(-8, 8, size=(M, K)).astype(np.int8)
    mags = (np.abs(rng.standard_normal((M, K // group))) * 0.02).astype(np.float16).view(np.uint16)
    if zp_enc:
        zs = rng.integers(-8, 8, size=(M, K // group))
        mags = ((mags & 0xFFF0) | (zs & 0xF)).astype(np.uint16)
    return codes, mags


# ---------------------------------------------------------------- exact floats
def exact_case(rng, M, K, T, group, block, zp_enc):
    """Powers-of-two scales and small codes: every fp32 operation is exact."""
    codes = rng.integers(-8, 8, size=(M, K)).astype(np.int8)
    G = K // group
    exps = rng.integers(-3, 2, size=(M, G))
    scales = np.array([[np.float16(2.0 ** int(e)).view(np.uint16) for e in row] for row in exps],
                      np.uint16)
    if zp_enc:
        zs = rng.integers(-8, 8, size=(M, G))
        scales = ((scales & 0xFFF0) | (zs & 0xF)).astype(np.uint16)
    q = rng.integers(-3, 4, size=(T, K)).astype(np.int8)
    asum = q.reshape(T, K // 32, 32).astype(np.int32).sum(axis=2).astype(np.int32)
    if block == 32:
        aexp = rng.integers(-5, -1, size=(T, K // 32))
        ascale = (2.0 ** aexp).astype(np.float32)
    else:
        ascale = (2.0 ** rng.integers(-5, -1, size=T)).astype(np.float32)
    P = np_partials(codes, scales, group, zp_enc, q, asum, block)
    unit = 32 if block == 32 else group
    Nu = K // unit
    y = np.zeros((T, M), np.float32)
    for t in range(T):
        for n in range(M):
            acc = Fraction(0)
            for u in range(Nu):
                g = (u * unit) // group
                raw = int(scales[n, g])
                ws = Fraction(float(np.uint16(raw & 0xFFF0 if zp_enc else raw).view(np.float16)))
                term = Fraction(int(P[t, n, u])) * ws
                if block == 32:
                    term *= Fraction(float(ascale[t, u]))
                acc += term
            if block != 32:
                acc *= Fraction(float(ascale[t]))
            y[t, n] = np.float32(float(acc))
            assert Fraction(float(y[t, n])) == acc, "case is not exact in fp32"
    return codes, scales, q, ascale, asum, y


# ---------------------------------------------------------------- order cases
def order_case():
    """Four config-mode units (group 32, per-token scale 1, plain FP16 scales
    1024, 1, 1, 1024) whose terms are +2^24, +1, +1, -2^24.

    Hand-derived expected outputs (fp32, round-half-even, fma chains):
      GEMV S=1 : acc0 takes units 0, 2: 2^24 + 1 -> 2^24 (tie to even);
                 acc1 takes 1, 3: 1 - 2^24 = -(2^24-1) exact;
                 y = 2^24 - (2^24-1) = 1
      GEMM/fan-out S=1 : serial 2^24, +1 -> 2^24, +1 -> 2^24, -2^24 -> 0
      GEMM/fan-out S=2 : p0 = 2^24 + 1 -> 2^24; p1 = 1 - 2^24 exact;
                 y = (0 + p0) + p1 = 1
      GEMV S=2 : p0 = acc0 + acc1 = 2^24 + 1 -> 2^24; p1 = 1 + (-2^24)
                 = -(2^24-1); y = 1
    """
    K = 128
    group = 32
    codes = np.zeros((16, K), np.int8)
    q = np.zeros((1, K), np.int8)
    # unit 0: 32 x (-8)(-64) = 16384; units 1 and 2: one element 1*1;
    # unit 3: 32 x (-8)(64) = -16384.
    codes[:, 0:32] = -8
    q[0, 0:32] = -64
    codes[:, 32] = 1
    q[0, 32] = 1
    codes[:, 64] = 1
    q[0, 64] = 1
    codes[:, 96:128] = -8
    q[0, 96:128] = 64
    # ws = 1024 for units 0 and 3 and 1.0 for units 1 and 2: terms 2^24, 1, 1, -2^24.
    scales = np.zeros((16, K // group), np.uint16)
    scales[:, 0] = np.float16(1024.0).view(np.uint16)
    scales[:, 1] = np.float16(1.0).view(np.uint16)
    scales[:, 2] = np.float16(1.0).view(np.uint16)
    scales[:, 3] = np.float16(1024.0).view(np.uint16)
    ascale = np.ones(1, np.float32)
    asum = q.reshape(1, K // 32, 32).astype(np.int32).sum(axis=2).astype(np.int32)
    expected = {  # (variant, splits) -> y
        ("gemv", 1): 1.0, ("gemm", 1): 0.0, ("fanout", 1): 0.0,
        ("gemm", 2): 1.0, ("fanout", 2): 1.0, ("gemv", 2): 1.0,
    }
    return codes, scales, q, ascale, asum, expected


def main():
    rng = np.random.default_rng(20261201)
    out = {}

    # quantizer edge cases (finite + exceptional), both block modes
    for mode in ("finite", "exceptional"):
        x = lcg_input(128, 4, mode == "exceptional")
        for block in (32, 0):
            q, s, sm = np_quantize(x, block)
            key = f"quant_{mode}_b{block}"
            out[key + "_x"] = x
            out[key + "_q"] = q
            out[key + "_scale"] = s
            out[key + "_sum"] = sm
    x, expect = quant_ties()
    out["quant_ties_x"] = x
    out["quant_ties_q"] = expect

    # integer partials, reference mode and config mode
    for name, (M, K, T, group, block, zp) in {
        "ref32": (32, 256, 5, 32, 32, True),
        "ref64": (32, 256, 3, 64, 32, True),
        "cfg128": (48, 512, 4, 128, 0, False),
        "cfg64": (32, 256, 2, 64, 0, False),
    }.items():
        codes, scales = random_weight(rng, M, K, group, zp)
        xa = rng.standard_normal((T, K)).astype(np.float32)
        q, s, sm = np_quantize(xa, block)
        out[f"part_{name}_codes"] = codes
        out[f"part_{name}_scales"] = scales
        out[f"part_{name}_q"] = q
        out[f"part_{name}_asum"] = sm
        out[f"part_{name}_meta"] = np.array([group, block, int(zp)], np.int32)
        out[f"part_{name}_P"] = np_partials(codes, scales, group, zp, q, sm, block)

    # exact projections
    for name, (M, K, T, group, block, zp) in {
        "ref32": (32, 256, 3, 32, 32, True),
        "ref64": (16, 256, 2, 64, 32, True),
        "cfg128": (32, 512, 3, 128, 0, False),
        "cfg64": (16, 256, 2, 64, 0, False),
    }.items():
        codes, scales, q, ascale, asum, y = exact_case(rng, M, K, T, group, block, zp)
        for k, v in dict(codes=codes, scales=scales, q=q, ascale=ascale, asum=asum, y=y).items():
            out[f"exact_{name}_{k}"] = v
        out[f"exact_{name}_meta"] = np.array([group, block, int(zp)], np.int32)

    # accumulation-order cases
    codes, scales, q, ascale, asum, expected = order_case()
    out["order_codes"] = codes
    out["order_scales"] = scales
    out["order_q"] = q
    out["order_ascale"] = ascale
    out["order_asum"] = asum
    keys = sorted(expected)
    out["order_variants"] = np.array([["gemv", "fanout", "gemm"].index(v) for v, _ in keys], np.int32)
    out["order_splits"] = np.array([s for _, s in keys], np.int32)
    out["order_expected"] = np.array([expected[k] for k in keys], np.float32)

    np.savez_compressed(os.path.join(HERE, "w4a8_golden.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
