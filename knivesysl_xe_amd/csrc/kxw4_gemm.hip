// kxw4_gemm.hip — prefill-shaped projections (x_gemm_w4a8 / gemm_rc16,
// kernels_dpas.cpp:1255-1490) on int8 MFMA.
//
// Block tile: BM tokens x 128 output rows, 4 waves in a 2 x 2 grid; each wave
// owns WM 16-token sub-tiles x 4 row-groups. The K loop walks 128-K weight
// tiles; activations (BM x 128 int8) and packed weights (8 row-groups x 1 KB)
// are staged through double-buffered LDS, weights stay packed in LDS and are
// unpacked to int8 in registers right before the MFMAs.
//
// Per unit (weight group, or K32 in reference mode) the int32 MFMA result is
// folded into an fp32 accumulator: acc = fma((float)P, ws, acc) with the token
// scale applied once at the end (per-token mode), or the reference's
// acc += (float)P * (ws * as) per K32 (reference mode). That is the serial
// K-order chain of the reference GEMM. Packed segments with a split count
// S > 1 (kernels_dpas.cpp:1343-1367, 1413-1420) keep their order by flushing
// each row's chain into a running sum at its split boundaries:
// sum = 0 + partial_0 + ... + partial_{S-1}; S == 1 rows store the chain
// directly (1477-1486).
//
// W8 (x_gemm_w8a8, kernels_dpas.cpp:1578-1629): 2 KB int8 weight tiles
// staged the same way and fed to the K32 MFMA without an unpack; the unit
// partial carries no factor 16.
//
// Block order is XCD-aware: consecutive logical tiles land on one XCD (blocks
// are dealt round-robin to the 8 XCDs) and are rastered in groups of 4 token
// tiles so the tiles running together share activation and weight tiles in
// that XCD's L2.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"


namespace kxw4 {

constexpr int kGemmThreads = 256;
constexpr int kApitch = 144;      // LDS row pitch of the activation tile (bytes)
constexpr int kGroupTT = 4;       // token tiles per raster group

__device__ __forceinline__ int seg_of(const GemmArgs &a, int t) {
    int s = 0;
    while (s + 1 < a.seg_count && t >= a.seg_end[s]) ++s;
    return s;
}

template <int WM, int UNIT, int MODE, bool SPLITS, bool DEBUG, bool W8>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(const GemmArgs a) {
    constexpr int BM = 2 * 16 * WM;
    constexpr int UPS = kTileK / UNIT;
    static_assert(!W8 || (UNIT == 32 && MODE == 1), "W8: K32 units, reference mode");
    constexpr int TB = W8 ? 2 : 1;             // 1 KB halves per weight tile
    constexpr int TILE = kTileBytes * TB;
    __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * kApitch];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][8 * TILE];

    // ---- block -> (token tile, weight, n-tile) ----
    const int nblk = gridDim.x, id = blockIdx.x;
    const int q8 = nblk / 8, r8 = nblk % 8, xcd = id % 8, j8 = id / 8;
    const int L = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int nnt = a.n_tiles, ntt = a.t_tiles;
    const int group = L / (kGroupTT * nnt);
    const int first = group * kGroupTT;
    const int gsz = min(ntt - first, kGroupTT);
    const int within = L % (kGroupTT * nnt);
    const int tt = first + within % gsz;
    const int ntg = within / gsz;
    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (ntg >= a.w[i].nt_begin) wi = i;
    const GemmWeight &W = a.w[wi];
    const int M = W.M;
    const int rg0 = (ntg - W.nt_begin) * 8;
    const int t0 = tt * BM;

    const int K = a.K, T = a.T, NT = K / kTileK, Nu = K / UNIT, G = K / a.group;
    const int gsh = __builtin_ctz(a.group / UNIT);       // unit -> scale group shift
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int n = lane & 15, g4 = lane >> 4;

    // ---- global -> register staging ----
    constexpr int ACH = BM * 8 / kGemmThreads;   // 16-byte activation chunks per thread
    v4i ra[ACH];
    v4u rb[2 * TB];
    // The loads go out unconditionally, at token and row-group indices
    // clamped into range, and the rows past T or M are zeroed when staged:
    // a load under its own bounds branch is waited for inside the branch,
    // which would hold every step's loads back until they arrive instead of
    // leaving them in flight across the step.
    auto gload = [&](int kb) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + kGemmThreads * i;
            const int row = c >> 3, col = c & 7;
            const int t = min(t0 + row, T - 1);
            ra[i] = *reinterpret_cast<const v4i *>(a.q + (size_t)t * K + kb * kTileK + col * 16);
        }
#pragma unroll
        for (int i = 0; i < 2 * TB; ++i) {
            const int c = tid + kGemmThreads * i;
            const int rgl = c / (64 * TB), l = c % (64 * TB);
            const int rg = min(rg0 + rgl, M / 16 - 1);
            rb[i] = *reinterpret_cast<const v4u *>(W.codes + ((size_t)rg * NT + kb) * TILE + l * 16);
        }
    };
    auto sstore = [&](int stage) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + kGemmThreads * i;
            const v4i zero = {0, 0, 0, 0};
            *reinterpret_cast<v4i *>(&As[stage][(c >> 3) * kApitch + (c & 7) * 16]) =
                t0 + (c >> 3) < T ? ra[i] : zero;
        }
#pragma unroll
        for (int i = 0; i < 2 * TB; ++i) {
            const int c = tid + kGemmThreads * i;
            const v4u zero = {0u, 0u, 0u, 0u};
            *reinterpret_cast<v4u *>(&Bs[stage][(c / (64 * TB)) * TILE + (c % (64 * TB)) * 16]) =
                rg0 + c / (64 * TB) < M / 16 ? rb[i] : zero;
        }
    };

    // ---- per-lane constants ----
    const int wrg0 = rg0 + wn * 4;          // first row-group of this wave
    const uint16_t *sb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int rg = wrg0 + j < M / 16 ? wrg0 + j : 0;
        sb[j] = W.scales + (size_t)rg * G * 16 + n;
    }
    const int tw0 = t0 + wm * 16 * WM;      // first token of this wave

    float f[WM][4][4];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) f[i][j][r] = 0.0f;

    // per-row split state (packed segments with S > 1)
    float sum[SPLITS ? WM : 1][4][4];
    int rS[SPLITS ? WM : 1][4], rsi[SPLITS ? WM : 1][4], rnb[SPLITS ? WM : 1][4];
    if constexpr (SPLITS) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = tw0 + i * 16 + 4 * g4 + r;
                const int S = t < T ? W.seg_split[seg_of(a, t)] : 1;
                rS[i][r] = S;
                int si = 1, nb = S > 1 ? (int)((long long)Nu / S) : Nu;
                while (si < S && nb == 0) { ++si; nb = si < S ? (int)((long long)Nu * si / S) : Nu; }
                rsi[i][r] = si;
                rnb[i][r] = si < S ? nb : Nu;
#pragma unroll
                for (int j = 0; j < 4; ++j) sum[i][j][r] = 0.0f;
            }
    }

    auto unit_epilogue = [&](const v4i (&acc)[WM][4], int u, const uint16_t (&raw)[4]) {
        if constexpr (SPLITS) {
            bool hit = false;
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) hit |= (u == rnb[i][r]);
            if (__any(hit)) {
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (u == rnb[i][r]) {
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                sum[i][j][r] = sum[i][j][r] + f[i][j][r];
                                f[i][j][r] = 0.0f;
                            }
                            int si = rsi[i][r] + 1;
                            int nb = si < rS[i][r] ? (int)((long long)Nu * si / rS[i][r]) : Nu;
                            while (si < rS[i][r] && nb == u) {
                                ++si;
                                nb = si < rS[i][r] ? (int)((long long)Nu * si / rS[i][r]) : Nu;
                            }
                            rsi[i][r] = si;
                            rnb[i][r] = si < rS[i][r] ? nb : Nu;
                        }
            }
        }
        float ws[4];
        int z[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (MODE == 0) {
                ws[j] = half_bits_to_float(raw[j]);
                z[j] = 0;
            } else {
                const bool zp = a.scale_enc == 1;
                ws[j] = half_bits_to_float(zp ? (uint16_t)(raw[j] & 0xFFF0u) : raw[j]);
                z[j] = zp ? sext4(raw[j]) : 0;
            }
        }
        // Reference mode: the unit's activation scale and code sum of each of
        // this lane's tokens, all loaded before any is used (a load under
        // its own branch would be waited for before the next one went out,
        // a memory round trip per token and unit). Every address is valid
        // whichever the mode: the per-token scale index without K32 blocks,
        // and the scale array (of the same [T][K/32] shape) standing in for
        // the sums when the weights have no zero points; the values those
        // modes do not use are replaced after the loads.
        float asv[WM][4];
        int smv[WM][4];
        if constexpr (MODE != 0) {
            const bool blk = a.block != 0, zps = a.scale_enc == 1;
            const int32_t *sp = zps ? a.asum : reinterpret_cast<const int32_t *>(a.ascale);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = tw0 + i * 16 + 4 * g4 + r;
                    const int tc = t < T ? t : 0;
                    asv[i][r] = a.ascale[blk ? (size_t)tc * (K / 32) + u : (size_t)tc];
                    int sm = 0;
#pragma unroll
                    for (int b = (u * UNIT) / 32; b < ((u + 1) * UNIT) / 32; ++b)
                        sm += sp[(size_t)tc * (K / 32) + b];
                    smv[i][r] = sm;
                }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    asv[i][r] = blk ? asv[i][r] : 1.0f;
                    smv[i][r] = zps ? smv[i][r] : 0;
                }
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = tw0 + i * 16 + 4 * g4 + r;
                float as = 1.0f;
                int sm = 0;
                if constexpr (MODE != 0) {
                    as = asv[i][r];
                    sm = smv[i][r];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int p = acc[i][j][r];
                    if (MODE == 0) {
                        f[i][j][r] = __builtin_fmaf((float)p, ws[j], f[i][j][r]);
                        continue;
                    }
                    p -= (z[j] * sm) << 4;
                    if (DEBUG && t < T && wrg0 + j < M / 16)
                        a.dbg[((size_t)t * M + (wrg0 + j) * 16 + n) * Nu + u] = W8 ? p : p >> 4;
                    if (a.block == 0) f[i][j][r] = __builtin_fmaf((float)p, ws[j], f[i][j][r]);
                    else f[i][j][r] = __builtin_fmaf((float)p, ws[j] * as, f[i][j][r]);
                }
            }
    };

    auto compute = [&](int stage, int kb, const uint16_t (&raw)[UPS][4]) {
        v4u wd[4][TB];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int h = 0; h < TB; ++h)
                wd[j][h] = *reinterpret_cast<const v4u *>(&Bs[stage][(wn * 4 + j) * TILE + h * 1024 + lane * 16]);
        v4i A[WM][2];
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                A[i][c] = *reinterpret_cast<const v4i *>(
                    &As[stage][(wm * 16 * WM + i * 16 + n) * kApitch + c * 64 + 16 * g4]);
#pragma unroll
        for (int jj = 0; jj < UPS; ++jj) {
            v4i acc[WM][4];
            const v4i zero = {0, 0, 0, 0};
            if constexpr (UNIT == 128) {
                v4i b0[4], b1[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    b0[j] = unpack_k64(wd[j][0].x, wd[j][0].y);
                    b1[j] = unpack_k64(wd[j][0].z, wd[j][0].w);
                }
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma_k64(A[i][0], b0[j], zero);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma_k64(A[i][1], b1[j], acc[i][j]);
            } else if constexpr (UNIT == 64) {
                v4i b[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    b[j] = jj == 0 ? unpack_k64(wd[j][0].x, wd[j][0].y) : unpack_k64(wd[j][0].z, wd[j][0].w);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma_k64(A[i][jj], b[j], zero);
            } else {
                long b[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (W8) {
                        const v4u h = wd[j][jj >> 1];
                        b[j] = (jj & 1) ? (long)(((uint64_t)h.w << 32) | h.z) : (long)(((uint64_t)h.y << 32) | h.x);
                    } else {
                        const v4u h = wd[j][0];
                        b[j] = unpack_k32(jj == 0 ? h.x : jj == 1 ? h.y : jj == 2 ? h.z : h.w);
                    }
                }
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    const v4i c = A[i][jj >> 1];
                    const long av = (jj & 1) ? (long)(((uint64_t)(uint32_t)c.w << 32) | (uint32_t)c.z)
                                             : (long)(((uint64_t)(uint32_t)c.y << 32) | (uint32_t)c.x);
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma_k32(av, b[j], zero);
                }
            }
            unit_epilogue(acc, kb * UPS + jj, raw[jj]);
        }
    };

    auto load_scales = [&](int kb, uint16_t (&raw)[UPS][4]) {
#pragma unroll
        for (int jj = 0; jj < UPS; ++jj)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                raw[jj][j] = sb[j][(size_t)((kb * UPS + jj) >> gsh) * 16];
    };

    uint16_t raw_cur[UPS][4], raw_nxt[UPS][4];
    gload(0);
    load_scales(0, raw_cur);
    sstore(0);
    __syncthreads();
    for (int kb = 0; kb < NT; ++kb) {
        const int stage = kb & 1;
        if (kb + 1 < NT) {
            // (the scales first: a wait for them then leaves the tile
            // loads issued after them in flight)
            load_scales(kb + 1, raw_nxt);
            gload(kb + 1);
        }
        compute(stage, kb, raw_cur);
        if (kb + 1 < NT) {
            sstore(stage ^ 1);
#pragma unroll
            for (int jj = 0; jj < UPS; ++jj)
#pragma unroll
                for (int j = 0; j < 4; ++j) raw_cur[jj][j] = raw_nxt[jj][j];
        }
        __syncthreads();
    }

    // ---- output (the debug run only records partials) ----
    if constexpr (DEBUG) return;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = tw0 + i * 16 + 4 * g4 + r;
            if (t >= T) continue;
            constexpr float kInv16 = W8 ? 1.0f : 0.0625f;   // the nibble unpack's factor 16
            const float sc = a.block == 0 ? a.ascale[t] * kInv16 : kInv16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rg = wrg0 + j;
                if (rg >= M / 16) continue;
                float val = f[i][j][r];
                if constexpr (SPLITS) {
                    if (rS[i][r] > 1) val = sum[i][j][r] + val;
                }
                const int row = rg * 16 + n;
                float out = val * sc;
                if (a.residual) out = out + a.residual[(size_t)t * M + row];
                if (a.y_bf16) static_cast<uint16_t *>(W.y)[(size_t)t * M + row] = float_to_bf16(out);
                else static_cast<float *>(W.y)[(size_t)t * M + row] = out;
            }
        }
}

template <int WM, int UNIT>
static void launch_wm_unit(const GemmArgs &a, int mode, bool splits, bool debug, dim3 grid,
                           hipStream_t st) {
    const dim3 block(kGemmThreads);
    // (split rows and debug runs always take the narrow tile: the wide one
    // is built for the plain chain only)
    if constexpr (WM == 2) {
        if (debug) {
            hipLaunchKernelGGL((gemm_kernel<WM, UNIT, 1, true, true, false>), grid, block, 0, st, a);
            return;
        }
        if (splits) {
            if (mode == 0) hipLaunchKernelGGL((gemm_kernel<WM, UNIT, 0, true, false, false>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((gemm_kernel<WM, UNIT, 1, true, false, false>), grid, block, 0, st, a);
            return;
        }
    }
    {
        if (mode == 0) hipLaunchKernelGGL((gemm_kernel<WM, UNIT, 0, false, false, false>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((gemm_kernel<WM, UNIT, 1, false, false, false>), grid, block, 0, st, a);
    }
}

// W8: K32 units in reference mode, the narrow tile
static void launch_w8(const GemmArgs &a, bool splits, bool debug, dim3 grid, hipStream_t st) {
    const dim3 block(kGemmThreads);
    if (debug) hipLaunchKernelGGL((gemm_kernel<2, 32, 1, true, true, true>), grid, block, 0, st, a);
    else if (splits) hipLaunchKernelGGL((gemm_kernel<2, 32, 1, true, false, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((gemm_kernel<2, 32, 1, false, false, true>), grid, block, 0, st, a);
}

int launch_gemm(GemmArgs &a, bool debug, hipStream_t st) {
    // The one-split modes go to the large-tile kernels (per-token: gemm3;
    // K32 activation blocks: gemmr); the gemm_kernel option keeps them here
    // (the tests cover both).
    if (!debug && options().gemm_kernel != kGemmGeneral && !a.w8) {
        int r = launch_gemm3(a, st);
        if (r != 1) return r;
        r = launch_gemmr(a, st);
        if (r != 1) return r;
    }
    bool splits = false;
    int nt = 0;
    for (int i = 0; i < a.count; ++i) {
        a.w[i].nt_begin = nt;
        nt += (a.w[i].M / 16 + 7) / 8;
        for (int s = 0; s < a.seg_count; ++s) splits |= a.w[i].seg_split[s] > 1;
    }
    // Split rows, debug runs and K32 units take the narrower wave tile (fewer
    // live registers).
    const int unit = a.block == 32 ? 32 : a.group;
    const bool narrow = splits || debug || unit == 32;
    const int BM = narrow ? 64 : 128;
    a.n_tiles = nt;
    a.t_tiles = (a.T + BM - 1) / BM;
    const dim3 grid(a.n_tiles * a.t_tiles);
    const int mode = (a.block == 0 && a.scale_enc == 0) ? 0 : 1;
    if (a.w8) {
        if (unit != 32 || mode != 1) return -2;
        launch_w8(a, splits, debug, grid, st);
    } else if (narrow) {
        if (unit == 128) launch_wm_unit<2, 128>(a, mode, splits, debug, grid, st);
        else if (unit == 64) launch_wm_unit<2, 64>(a, mode, splits, debug, grid, st);
        else launch_wm_unit<2, 32>(a, mode, splits, debug, grid, st);
    } else {
        if (unit == 128) launch_wm_unit<4, 128>(a, mode, false, false, grid, st);
        else launch_wm_unit<4, 64>(a, mode, false, false, grid, st);
    }
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace kxw4
