// kxw4_skinny.hip — decode-shaped projections (T <= 64 tokens): the GEMV
// (kernels_dpas.cpp:586-675), the fan-out GEMV (945-1102) and the batched
// GEMM at small T with a uniform split count (1379-1488).
//
// Work decomposition (HBM-bound: every weight byte is read once):
//   * a work-group is 8 waves; a row-group (16 output rows) is served by
//     wrg = min(S, 8) waves, so a work-group holds 8/wrg row-groups;
//   * wave j of a row-group runs splits [j*S/wrg, (j+1)*S/wrg) one after the
//     other; split s covers units [Nu*s/S, Nu*(s+1)/S) and runs the
//     reference chain for its variant (two alternating accumulators for the
//     GEMV, one serial accumulator otherwise);
//   * with S > 1 the split partials meet in LDS and one wave adds them in
//     split order starting from 0.0f, as the fused reduction does
//     (kernels_dpas.cpp:663-672, 1092-1101, 1477-1486).
// Per 128-K step a lane issues one 16-byte weight load (a whole 1 KB tile per
// wave) and two 16-byte activation loads per 16-token block, unpacks nibbles
// to int8 in registers and runs the int8 MFMAs; PF steps are kept in flight.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

namespace kxw4 {

constexpr int kSkWaves = 8;

template <int TB, int UNIT>
struct SkStage {
    v4u wd;                  // packed weight dwords of this lane
    v4i A[TB][2];            // activation slots, 16-token blocks x 64-K chunks
    uint16_t sraw[kTileK / UNIT];
};

template <int TB, int UNIT, int MODE, bool DEBUG>
__global__ __launch_bounds__(64 * kSkWaves) void skinny_kernel(const SkinnyArgs a) {
    constexpr int UPS = kTileK / UNIT;                  // units per 128-K step
    constexpr int PF = TB == 1 ? 4 : (TB == 2 || MODE == 0) ? 2 : 1;   // steps in flight
    extern __shared__ float lds[];

    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if ((int)blockIdx.x >= a.w[i].wg_begin) wi = i;
    const SkinnyWeight W = a.w[wi];

    const int K = a.K, T = a.T, M = W.M;
    const int NT = K / kTileK, Nu = K / UNIT, G = K / a.group;
    const int S = W.S, wrg = W.wrg;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int R = kSkWaves / wrg;
    const int rgl = wave / wrg, wj = wave % wrg;
    const int rg = ((int)blockIdx.x - W.wg_begin) * R + rgl;
    const bool active = rg < M / 16;
    const int n = lane & 15, g4 = lane >> 4;
    const bool alt2 = a.variant == kVarGemv;

    const uint8_t *wbase = W.codes + (size_t)rg * NT * kTileBytes + lane * 16;
    const uint16_t *sbase = W.scales + (size_t)rg * G * 16 + n;
    const int8_t *abase[TB];
    bool tvalid[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int t = tb * 16 + n;
        tvalid[tb] = t < T;
        abase[tb] = a.q + (size_t)(tvalid[tb] ? t : 0) * K + 16 * g4;
    }

    auto load_stage = [&](SkStage<TB, UNIT> &st, int kb) {
        st.wd = *reinterpret_cast<const v4u *>(wbase + (size_t)kb * kTileBytes);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            v4i z0 = {0, 0, 0, 0}, z1 = {0, 0, 0, 0};
            if (tvalid[tb]) {
                z0 = *reinterpret_cast<const v4i *>(abase[tb] + (size_t)kb * kTileK);
                z1 = *reinterpret_cast<const v4i *>(abase[tb] + (size_t)kb * kTileK + 64);
            }
            st.A[tb][0] = z0;
            st.A[tb][1] = z1;
        }
#pragma unroll
        for (int j = 0; j < UPS; ++j) st.sraw[j] = sbase[(size_t)(((kb * UPS + j) * UNIT) / a.group) * 16];
    };

    float part[TB][4];
    int split_begin = wj * S / wrg, split_end = (wj + 1) * S / wrg;
    if (!active) split_end = split_begin;

    for (int s = split_begin; s < split_end; ++s) {
        const int u0 = (int)((long long)Nu * s / S), u1 = (int)((long long)Nu * (s + 1) / S);
        float f0[TB][4], f1[TB][4];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) f0[tb][r] = f1[tb][r] = 0.0f;

        // One unit's epilogue into accumulator set f (fp32, 16x scaled).
        auto epilogue = [&](float (&f)[TB][4], const v4i (&acc)[TB], int u, uint16_t raw) {
            float ws;
            int z = 0;
            if (MODE == 0) {
                ws = half_bits_to_float(raw);
            } else {
                const bool zp = a.scale_enc == 1;
                ws = half_bits_to_float(zp ? (uint16_t)(raw & 0xFFF0u) : raw);
                z = zp ? sext4(raw) : 0;
            }
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int p = acc[tb][r];
                    if (MODE == 0) {
                        f[tb][r] = __builtin_fmaf((float)p, ws, f[tb][r]);
                        continue;
                    }
                    const int t = tb * 16 + 4 * g4 + r;
                    const int tc = t < T ? t : 0;
                    if (z != 0) {
                        int sm = 0;
                        for (int b = (u * UNIT) / 32; b < ((u + 1) * UNIT) / 32; ++b)
                            sm += a.asum[(size_t)tc * (K / 32) + b];
                        p -= (z * sm) << 4;
                    }
                    if (DEBUG && t < T)
                        a.dbg[((size_t)t * M + rg * 16 + n) * Nu + u] = p >> 4;
                    const float pf = (float)p;
                    if (a.block == 0) {
                        f[tb][r] = __builtin_fmaf(pf, ws, f[tb][r]);
                    } else {
                        const float as = a.ascale[(size_t)tc * (K / 32) + u];
                        if (a.variant == kVarGemm) f[tb][r] = __builtin_fmaf(pf, ws * as, f[tb][r]);
                        else f[tb][r] = __builtin_fmaf(pf * ws, as, f[tb][r]);
                    }
                }
        };

        auto process = [&](const SkStage<TB, UNIT> &st, int kb) {
#pragma unroll
            for (int j = 0; j < UPS; ++j) {
                const int u = kb * UPS + j;
                if (u < u0 || u >= u1) continue;
                v4i acc[TB];
                if constexpr (UNIT == 128) {
                    const v4i b0 = unpack_k64(st.wd.x, st.wd.y), b1 = unpack_k64(st.wd.z, st.wd.w);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) {
                        const v4i zero = {0, 0, 0, 0};
                        acc[tb] = mfma_k64(st.A[tb][0], b0, zero);
                        acc[tb] = mfma_k64(st.A[tb][1], b1, acc[tb]);
                    }
                } else if constexpr (UNIT == 64) {
                    const v4i b = j == 0 ? unpack_k64(st.wd.x, st.wd.y) : unpack_k64(st.wd.z, st.wd.w);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) {
                        const v4i zero = {0, 0, 0, 0};
                        acc[tb] = mfma_k64(st.A[tb][j], b, zero);
                    }
                } else {
                    const uint32_t d = j == 0 ? st.wd.x : j == 1 ? st.wd.y : j == 2 ? st.wd.z : st.wd.w;
                    const long b = unpack_k32(d);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) {
                        const v4i c = st.A[tb][j >> 1];
                        const long av = (j & 1) ? (long)(((uint64_t)(uint32_t)c.w << 32) | (uint32_t)c.z)
                                                : (long)(((uint64_t)(uint32_t)c.y << 32) | (uint32_t)c.x);
                        const v4i zero = {0, 0, 0, 0};
                        acc[tb] = mfma_k32(av, b, zero);
                    }
                }
                if (alt2 && ((u - u0) & 1)) epilogue(f1, acc, u, st.sraw[j]);
                else epilogue(f0, acc, u, st.sraw[j]);
            }
        };

        const int st0 = u0 / UPS, st1 = (u1 + UPS - 1) / UPS;
        SkStage<TB, UNIT> stg[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i)
            if (st0 + i < st1) load_stage(stg[i], st0 + i);
        for (int sb = st0; sb < st1; sb += PF) {
#pragma unroll
            for (int i = 0; i < PF; ++i) {
                const int kb = sb + i;
                if (kb < st1) {
                    process(stg[i], kb);
                    if (kb + PF < st1) load_stage(stg[i], kb + PF);
                }
            }
        }
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[tb][r] = alt2 ? f0[tb][r] + f1[tb][r] : f0[tb][r];
        if (S > 1) {
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    lds[(((size_t)(rgl * S + s) * TB + tb) * 4 + r) * 64 + lane] = part[tb][r];
        }
    }

    if (S > 1) {
        __syncthreads();
        if (wj != 0 || !active) return;
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float sum = 0.0f;
                for (int s = 0; s < S; ++s)
                    sum = sum + lds[(((size_t)(rgl * S + s) * TB + tb) * 4 + r) * 64 + lane];
                part[tb][r] = sum;
            }
    } else if (!active) {
        return;
    }

    const int row = rg * 16 + n;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = tb * 16 + 4 * g4 + r;
            if (t >= T) continue;
            const float v = a.block == 0 ? part[tb][r] * (a.ascale[t] * 0.0625f)
                                         : part[tb][r] * 0.0625f;
            float out;
            if (a.residual) out = v + a.residual[(size_t)t * M + row];
            else if (alt2 && S > 1) out = v + 0.0f;
            else out = v;
            if (a.y_bf16) static_cast<uint16_t *>(W.y)[(size_t)t * M + row] = float_to_bf16(out);
            else static_cast<float *>(W.y)[(size_t)t * M + row] = out;
        }
}

template <int TB, int UNIT>
static void launch_tb_unit(const SkinnyArgs &a, int mode, bool debug, dim3 grid, size_t lds,
                           hipStream_t st) {
    const dim3 block(64 * kSkWaves);
    if (debug)
        hipLaunchKernelGGL((skinny_kernel<TB, UNIT, 1, true>), grid, block, lds, st, a);
    else if (mode == 0)
        hipLaunchKernelGGL((skinny_kernel<TB, UNIT, 0, false>), grid, block, lds, st, a);
    else
        hipLaunchKernelGGL((skinny_kernel<TB, UNIT, 1, false>), grid, block, lds, st, a);
}

template <int TB>
static void launch_tb(const SkinnyArgs &a, int unit, int mode, bool debug, dim3 grid, size_t lds,
                      hipStream_t st) {
    if (unit == 128) launch_tb_unit<TB, 128>(a, mode, debug, grid, lds, st);
    else if (unit == 64) launch_tb_unit<TB, 64>(a, mode, debug, grid, lds, st);
    else launch_tb_unit<TB, 32>(a, mode, debug, grid, lds, st);
}

int launch_skinny(SkinnyArgs &a, bool debug, hipStream_t st) {
    const int unit = a.block == 32 ? 32 : a.group;
    const int TB = a.T <= 16 ? 1 : a.T <= 32 ? 2 : 4;
    int wg = 0;
    size_t lds = 0;
    for (int i = 0; i < a.count; ++i) {
        SkinnyWeight &w = a.w[i];
        w.wrg = w.S < kSkWaves ? w.S : kSkWaves;
        const int R = kSkWaves / w.wrg;
        w.wg_begin = wg;
        wg += (w.M / 16 + R - 1) / R;
        if (w.S > 1) {
            const size_t need = (size_t)R * w.S * TB * 256 * sizeof(float);
            if (need > lds) lds = need;
        }
    }
    const int mode = (a.block == 0 && a.scale_enc == 0) ? 0 : 1;
    const dim3 grid(wg);
    if (TB == 1) launch_tb<1>(a, unit, mode, debug, grid, lds, st);
    else if (TB == 2) launch_tb<2>(a, unit, mode, debug, grid, lds, st);
    else launch_tb<4>(a, unit, mode, debug, grid, lds, st);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace kxw4
