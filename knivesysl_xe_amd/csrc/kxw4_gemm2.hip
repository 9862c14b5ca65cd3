// kxw4_gemm2.hip — prefill projections in the per-token mode (the BASELINE
// configurations): x_gemm_w4a8 / gemm_rc16 arithmetic (kernels_dpas.cpp:
// 1255-1332, 1334-1490) with one split per token, on int8 MFMA.
//
// Block tile BM tokens x 128 output rows (8 row-groups), 4 waves in a 2 x 2
// grid, wave tile BM/2 tokens x 64 rows. Per 128-K step the activation tile,
// the weight tiles and each wave's FP16 scales reach LDS through direct
// global->LDS loads (no staging registers, no LDS store instructions) into a
// ring of NST stages: the loads of step k+NST-1 are issued right after the
// barrier that opens step k, and step k waits only for its own stage (every
// wave issues the same number of loads per stage, so one vmcnt covers it).
// Two stages keep three work-groups per CU, which measured faster than a
// deeper ring at two.
// Activation rows are XOR-swizzled on the load side so a 16-lane quarter of
// an MFMA operand read hits 16 distinct 16-byte bank groups; packed weight
// tiles keep their lane order.
//
// Per row-block the wave unpacks one weight tile to 16*q int8, runs the
// MFMAs of its token blocks and folds each unit's int32 result into the FP32
// chain, f = fma((float)P, ws, f), in K order, then moves to the next
// row-block; the int32 results therefore live only briefly in VGPRs. The
// token scale and the 1/16 of the nibble unpack are applied once at the end.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

namespace kxw4 {

constexpr int kG2Threads = 256;
constexpr int kG2GroupTT = 4;      // token tiles per raster group

// LDS destination of a direct global->LDS load
#define KXW4_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// Granule (16 bytes) of activation row t, 16-byte chunk c16 (0..7), inside a
// stage: two rows share a 256-byte block; row parity is granule bit 3 and the
// chunk is XOR-ed with (t/2) & 7 in bits 0..2.
__device__ __forceinline__ int a_granule(int t, int c16) {
    return (t >> 1) * 16 + (((t & 1) << 3) | (c16 ^ ((t >> 1) & 7)));
}

template <int WM, int UNIT, int NST>
__global__ __launch_bounds__(kG2Threads) void gemm2_kernel(const GemmArgs a) {
    constexpr int BM = 2 * 16 * WM;
    constexpr int UPS = kTileK / UNIT;
    constexpr int A_BYTES = BM * kTileK;
    constexpr int B_BYTES = 8 * kTileBytes;
    constexpr int S_BYTES = 4 * 4 * UPS * 32;    // per wave: 4 row-groups x UPS units x 16 FP16
    constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // ---- block -> (token tile, weight, n-tile), XCD-aware raster ----
    const int nblk = gridDim.x, id = blockIdx.x;
    const int q8 = nblk / 8, r8 = nblk % 8, xcd = id % 8, j8 = id / 8;
    const int L = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int nnt = a.n_tiles, ntt = a.t_tiles;
    const int group = L / (kG2GroupTT * nnt);
    const int first = group * kG2GroupTT;
    const int gsz = min(ntt - first, kG2GroupTT);
    const int within = L % (kG2GroupTT * nnt);
    const int tt = first + within % gsz;
    const int ntg = within / gsz;
    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (ntg >= a.w[i].nt_begin) wi = i;
    const GemmWeight &W = a.w[wi];
    const int M = W.M, RG = M / 16;
    const int rg0 = (ntg - W.nt_begin) * 8;
    const int t0 = tt * BM;
    const int K = a.K, T = a.T, NT = K / kTileK, G = K / a.group;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int n = lane & 15, g4 = lane >> 4;

    // ---- stage issue: A (BM/8 wave loads), B (8 wave loads), 1/4 of each per wave ----
    // per-lane 32-bit source offsets that do not depend on the K step; the
    // per-step part is a uniform base, so the loads take a scalar base
    // (the launcher guarantees T*K and M*K/2 below 2^31)
    uint32_t aoffs[BM / 32];
#pragma unroll
    for (int i = 0; i < BM / 32; ++i) {
        const int p = (wave + 4 * i) * 64 + lane;            // granule this lane fills
        const int t = 2 * (p >> 4) + ((p >> 3) & 1);
        const int c16 = (p & 7) ^ ((t >> 1) & 7);
        const int tg = min(t0 + t, T - 1);                    // rows past T: never stored
        aoffs[i] = (uint32_t)tg * K + c16 * 16;
    }
    uint32_t boffs[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rg = min(rg0 + wave + 4 * i, RG - 1);       // row-groups past M: never stored
        boffs[i] = (uint32_t)rg * NT * kTileBytes + lane * 16;
    }
    // scales: lane l < 8*UPS of each wave fetches 16 bytes (half of one
    // row-group's 16 scales for one unit) of its 4 row-groups; LDS holds them
    // as [j][u][16] FP16 per wave
    const int sj = (lane >> 1) / UPS, su = (lane >> 1) % UPS;
    const uint32_t soff =
        ((uint32_t)min(rg0 + wn * 4 + min(sj, 3), RG - 1) * G + su) * 16 + (lane & 1) * 8;
    // (the DMA builtin takes a generic void pointer: with a typed pointer the
    // host compilation pass drops the kernel without a diagnostic)
    auto issue = [&](int kb, int st) {
        uint8_t *base = smem + st * STAGE;
        const int8_t *qk = a.q + (size_t)kb * kTileK;
        const uint8_t *wk = W.codes + (size_t)kb * kTileBytes;
#pragma unroll
        for (int i = 0; i < BM / 32; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(qk + aoffs[i]),
                                             KXW4_LDS(base + (wave + 4 * i) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(wk + boffs[i]),
                                             KXW4_LDS(base + A_BYTES + (wave + 4 * i) * 1024), 16, 0, 0);
        // lanes past 8*UPS are masked off; the load still counts once in vmcnt
        if (lane < 8 * UPS)
            __builtin_amdgcn_global_load_lds((const void *)(W.scales + (size_t)kb * UPS * 16 + soff),
                                             KXW4_LDS(base + A_BYTES + B_BYTES + wave * (S_BYTES / 4)), 16, 0, 0);
    };

    // ---- per-lane read offsets ----
    const int tw = wm * 16 * WM;                               // first token of this wave in the tile
    const int h = ((n >> 1) + (tw >> 1)) & 7;                  // XOR of this lane's rows
    int aoff[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
        aoff[c] = (((tw >> 1) + (n >> 1)) * 16 + (((n & 1) << 3) | ((c * 4 + g4) ^ h))) * 16;
    const int boff = A_BYTES + wn * 4 * kTileBytes + lane * 16;

    float f[WM][4][4];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) f[i][j][r] = 0.0f;

    const int soff_lds = A_BYTES + B_BYTES + wave * (S_BYTES / 4) + n * 2;

    // Ring of NST stages. Stage k % NST is issued at the top of step
    // k - (NST - 1). At the top of step k this wave's loads of steps k ..
    // k + NST - 2 may be outstanding (7 per stage): with three stages vmcnt(7)
    // retires step k's, with two (or at the last step) vmcnt(0). The barrier
    // then makes every wave's loads visible and guarantees that stage
    // (k - 1) % NST, refilled next, is no longer read.
    static_assert(NST == 2 || NST == 3, "two or three stages");
    constexpr int kLoadsPerStage = BM / 32 + 2 + 1;
    static_assert(kLoadsPerStage == 7, "vmcnt below assumes seven loads per stage");
    issue(0, 0);
    if (NST == 3 && NT > 1) issue(1, 1);
    int st = 0;
    for (int kb = 0; kb < NT; ++kb) {
        if (NST == 3 && kb + 1 < NT) __builtin_amdgcn_s_waitcnt(0x0F70 | 7);   // vmcnt(7)
        else __builtin_amdgcn_s_waitcnt(0x0F70);                              // vmcnt(0)
        lds_sync_after_dma();
        if (kb + NST - 1 < NT) issue(kb + NST - 1, st == 0 ? NST - 1 : st - 1);
        const uint8_t *sb = smem + st * STAGE;
        v4i A[WM][2];
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                A[i][c] = *reinterpret_cast<const v4i *>(sb + aoff[c] + i * 2048);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4u wd = *reinterpret_cast<const v4u *>(sb + boff + j * kTileBytes);
            const v4i zero = {0, 0, 0, 0};
            if constexpr (UNIT == 128) {
                const v4i b0 = unpack_k64(wd.x, wd.y), b1 = unpack_k64(wd.z, wd.w);
                const float w = half_bits_to_float(*reinterpret_cast<const uint16_t *>(sb + soff_lds + j * UPS * 32));
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    v4i acc = mfma_k64(A[i][0], b0, zero);
                    acc = mfma_k64(A[i][1], b1, acc);
#pragma unroll
                    for (int r = 0; r < 4; ++r) f[i][j][r] = __builtin_fmaf((float)acc[r], w, f[i][j][r]);
                }
            } else {
                static_assert(UNIT == 64, "per-token mode has unit = group in {64, 128}");
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const v4i b = u == 0 ? unpack_k64(wd.x, wd.y) : unpack_k64(wd.z, wd.w);
                    const float w = half_bits_to_float(
                        *reinterpret_cast<const uint16_t *>(sb + soff_lds + (j * UPS + u) * 32));
#pragma unroll
                    for (int i = 0; i < WM; ++i) {
                        const v4i acc = mfma_k64(A[i][u], b, zero);
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            f[i][j][r] = __builtin_fmaf((float)acc[r], w, f[i][j][r]);
                    }
                }
            }
        }
        st = st == NST - 1 ? 0 : st + 1;
    }

    // ---- output ----
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + tw + i * 16 + 4 * g4 + r;
            if (t >= T) continue;
            const float sc = a.ascale[t] * 0.0625f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rg = rg0 + wn * 4 + j;
                if (rg >= RG) continue;
                const int row = rg * 16 + n;
                float out = f[i][j][r] * sc;
                if (a.residual) out = out + a.residual[(size_t)t * M + row];
                if (a.y_bf16) static_cast<uint16_t *>(W.y)[(size_t)t * M + row] = float_to_bf16(out);
                else static_cast<float *>(W.y)[(size_t)t * M + row] = out;
            }
        }
}

int launch_gemm2(GemmArgs &a, hipStream_t st) {
    // per-token activation scale, plain FP16 weight scales, one split per token
    if (a.block != 0 || a.scale_enc != 0 || (a.group != 64 && a.group != 128)) return 1;
    if ((long long)a.T * a.K >= (1ll << 31)) return 1;          // 32-bit activation offsets
    for (int i = 0; i < a.count; ++i)
        if ((long long)a.w[i].M * a.K / 2 >= (1ll << 31)) return 1;
    int nt = 0;
    for (int i = 0; i < a.count; ++i) {
        for (int s = 0; s < a.seg_count; ++s)
            if (a.w[i].seg_split[s] != 1) return 1;
        a.w[i].nt_begin = nt;
        nt += (a.w[i].M / 16 + 7) / 8;
    }
    constexpr int WM = 4, BM = 2 * 16 * WM;
    a.n_tiles = nt;
    a.t_tiles = (a.T + BM - 1) / BM;
    const dim3 grid(a.n_tiles * a.t_tiles), block(kG2Threads);
    constexpr int NST = 2;
    const int ups = kTileK / a.group;
    const size_t lds = NST * ((size_t)BM * kTileK + 8 * kTileBytes + 4 * 4 * ups * 32);
    if (a.group == 128) hipLaunchKernelGGL((gemm2_kernel<WM, 128, NST>), grid, block, lds, st, a);
    else hipLaunchKernelGGL((gemm2_kernel<WM, 64, NST>), grid, block, lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace kxw4
