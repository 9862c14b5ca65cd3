// kxw4_gemmr.hip — prefill projections in the reference mode on the
// 32x32x32 int8 MFMA: x_gemm_w4a8 / gemm_rc16 with activation scales per
// (token, K32 block) and FP16|zp weight scales (kernels_dpas.cpp:1255-1332,
// 1334-1490), one split per token.
//
// Arithmetic: per output and K32 unit u, in K order from 0,
//   acc = fma((float)(d_u - z_u * asum_u), ws_u * as_u, acc)
// (kernels_dpas.cpp:1313-1321: the product ws * as rounded first). Each MFMA
// covers exactly one K32 unit, so its int32 result is the unit partial. The
// weight operand is unpacked to the bytes w - z with the unit's zero point
// folded in (range [-15, 15]), so the MFMA returns d - z * asum directly and
// the activation code sums are never read. Weights with plain FP16 scales
// unpack to 16 w (the nibble in the high half of a byte) and the output is
// scaled by 1/16 (exact: every chain value is 16x the reference's).
//
// Cost model: the chain is three VALU operations per output and unit (the
// conversion, ws * as, the FMA), 192 per 32x32 block and 128-K step against
// four 32-cycle MFMAs. About 16 VALU instructions issue under a block's
// MFMAs for free and each one beyond costs its full issue time (measured on
// the MI355X), so the kernel is VALU-bound and is laid out to add as little
// as possible to the chain:
//   * weights are the MFMA's A operand and activations its B operand, so a
//     lane holds one token and 16 rows of a block: the activation scale is
//     one value per lane and unit, and the 16 weight scales (and the weight
//     unpack) are shared by the wave's NT token blocks;
//   * a wave owns 32 rows x 32*NT tokens; a work-group WR x WT waves;
//   * per 128-K step the activation tile (XOR-swizzled rows), the packed
//     weight tiles, the FP16|zp scales and the activation scales of the
//     step's four units reach LDS through direct global->LDS loads into a
//     ring of NST stages, one barrier per step.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace kxw4 {

constexpr int kGrGroupTT = 4;      // token tiles per raster group

#define KXW4_GR_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// A operand of one K32 unit: dword d0 of lane group 2kg (K slots 0..7) and
// d1 of lane group 2kg + 1 (slots 8..15), unpacked to the bytes w - z (ZP)
// or 16 w. With zero points: each nibble n (two's complement w) becomes the
// byte 0x80 | (n ^ 8) = 128 + w + 8 (one bit operation); subtracting
// zz = (z + 8) * 0x01010101 leaves 128 + w - z in [113, 143] per byte, so no
// borrow crosses a byte, and the XOR turns the excess-128 bytes into two's
// complement.
__device__ __forceinline__ uint32_t gr_zp_bytes(uint32_t nib, uint32_t zz) {
    const uint32_t e = ((nib ^ 0x08080808u) & 0x0F0F0F0Fu) | 0x80808080u;
    return (e - zz) ^ 0x80808080u;
}

template <bool ZP>
__device__ __forceinline__ v4i gr_unpack(uint32_t d0, uint32_t d1, uint32_t zz) {
    v4i b;
    if constexpr (ZP) {
        b.x = (int)gr_zp_bytes(d0, zz);
        b.y = (int)gr_zp_bytes(d0 >> 4, zz);
        b.z = (int)gr_zp_bytes(d1, zz);
        b.w = (int)gr_zp_bytes(d1 >> 4, zz);
    } else {
        (void)zz;
        b.x = (int)nib_lo16(d0);
        b.y = (int)nib_hi16(d0);
        b.z = (int)nib_lo16(d1);
        b.w = (int)nib_hi16(d1);
    }
    return b;
}

template <int NT, int WR, int WT, int GROUP>
struct GrShape {
    static constexpr int NW = WR * WT;
    static constexpr int NTH = 64 * NW;
    static constexpr int BN = 32 * WR;                   // rows per tile
    static constexpr int RGS = BN / 16;                  // row-groups per tile
    static constexpr int BM = 32 * NT * WT;              // tokens per tile
    static constexpr int GPS = kTileK / GROUP;           // weight scale groups per step
    static constexpr int A_BYTES = BM * kTileK;
    static constexpr int W_BYTES = RGS * kTileBytes;
    static constexpr int S_BYTES = RGS * GPS * 32;       // [row-group][group][16] FP16|zp
    static constexpr int AS_BYTES = BM * 16;             // [token][4 units] FP32
    static constexpr int W_OFF = A_BYTES;
    static constexpr int S_OFF = W_OFF + W_BYTES;
    static constexpr int AS_OFF = (S_OFF + S_BYTES + 15) / 16 * 16;
    // prepared once per stage by the waves that loaded the scales: the FP16
    // scales with the zero-point nibble cleared ([row-group][group][16]
    // u16) and the zero-point bytes z + 8 ([row-group][group][16] u8)
    static constexpr int MS_OFF = AS_OFF + AS_BYTES;
    static constexpr int ZZ_OFF = MS_OFF + S_BYTES;
    static constexpr int STAGE = (ZZ_OFF + S_BYTES / 2 + 1023) / 1024 * 1024;
    // loads per wave and stage, equal for every wave (one vmcnt retires a
    // stage); chunk indices wrap when the waves do not divide them, and a
    // few chunks are then loaded twice (same bytes to the same LDS address)
    static constexpr int A_CHUNKS = A_BYTES / 1024;
    static constexpr int A_LOADS = (A_CHUNKS + NW - 1) / NW;
    static constexpr int W_LOADS = (RGS + NW - 1) / NW;
    static constexpr int S_TOTAL = RGS * GPS * 2;        // 16-byte scale granules per stage
    static constexpr int s_lanes() {                     // a divisor of S_TOTAL: no range straddles the wrap
        int d = (S_TOTAL + NW - 1) / NW;
        while (S_TOTAL % d) ++d;
        return d;
    }
    static constexpr int S_LANES = s_lanes();
    static constexpr int AS_LANES = BM < 64 ? BM : 64;   // tokens (16 bytes each) per load
    static constexpr int AS_CHUNKS = BM / AS_LANES;
    static constexpr int AS_LOADS = (AS_CHUNKS + NW - 1) / NW;
    static constexpr int LOADS = A_LOADS + W_LOADS + 1 + AS_LOADS;
    // output staging: one token block of a wave at a time, [token][row]
    // FP32 with a row stride of EPS floats, inside the ring
    static constexpr int EPS = 36;
    static constexpr int SLAB = 32 * EPS * 4;
    template <int NST>
    static constexpr int lds_bytes() { return NST * STAGE > NW * SLAB ? NST * STAGE : NW * SLAB; }
    static_assert(A_BYTES % 1024 == 0 && BM % AS_LANES == 0, "activation tile in whole 1 KB chunks");
    static_assert(S_LANES <= 64, "one scale load per wave and stage");
};

// OCC: waves per SIMD the register budget is sized for
template <int NT, int WR, int WT, int GROUP, bool ZP, int NST, int OCC>
__global__ __launch_bounds__(64 * WR * WT)
__attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemmr_kernel(const GemmArgs a) {
    using S = GrShape<NT, WR, WT, GROUP>;
    constexpr int NW = S::NW, BM = S::BM, RGS = S::RGS, GPS = S::GPS, STAGE = S::STAGE;
    // five or more waves per SIMD: the lean pipeline (one MFMA result live)
    constexpr bool LEAN = OCC >= 5;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // ---- block -> (token tile, weight, n-tile), XCD-aware raster: the
    // work-groups of one XCD (blockIdx % 8) take consecutive tiles, grouped
    // kGrGroupTT token tiles at a time so they share tiles in that XCD's L2 ----
    const int nblk = gridDim.x, id = blockIdx.x;
    const int q8 = nblk / 8, r8 = nblk % 8, xcd = id % 8, j8 = id / 8;
    const int L = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int nnt = a.n_tiles, ntt = a.t_tiles;
    const int grp = L / (kGrGroupTT * nnt);
    const int first = grp * kGrGroupTT;
    const int gsz = min(ntt - first, kGrGroupTT);
    const int within = L % (kGrGroupTT * nnt);
    const int tt = first + within % gsz;
    const int ntg = within / gsz;
    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (ntg >= a.w[i].nt_begin) wi = i;
    const GemmWeight &W = a.w[wi];
    const int M = W.M, RG = M / 16;
    const int rg0 = (ntg - W.nt_begin) * RGS;
    const int t0 = tt * BM;
    const int K = a.K, T = a.T, NTK = K / kTileK, G = K / GROUP, KB = K / 32;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave % WR, wt = wave / WR;

    // ---- load issue: per-lane 32-bit source offsets that do not depend on
    // the K step (the launcher keeps T*K, M*K/2 and T*K/8 below 2^31); rows
    // past T or M read the last row (never stored). They are recomputed at
    // each issue (a few VALU operations per step) rather than held across
    // the K loop, where the registers are short. ----
    auto a_off = [&](int ln, int i) {
        const int ch = (wave + NW * i) % S::A_CHUNKS;
        const int t = 8 * ch + (ln >> 3);                    // token of the tile this lane fills
        const int p = (ln & 7) ^ ((t >> 1) & 7);             // 16-byte piece of the row stored at slot lane % 8
        return (uint32_t)min(t0 + t, T - 1) * K + p * 16;
    };
    auto w_off = [&](int ln, int i) {
        const int rg = min(rg0 + (wave + NW * i) % RGS, RG - 1);
        return (uint32_t)rg * NTK * kTileBytes + ln * 16;
    };
    auto s_off = [&](int ln) {
        const int gi = (wave * S::S_LANES + min(ln, S::S_LANES - 1)) % S::S_TOTAL;
        const int j = gi / (2 * GPS), g = (gi >> 1) % GPS, half = gi & 1;
        const int rg = min(rg0 + j, RG - 1);
        return ((uint32_t)rg * G + g) * 32 + half * 16;      // bytes
    };
    auto as_off = [&](int ln, int i) {
        const int t = ((wave + NW * i) % S::AS_CHUNKS) * S::AS_LANES + min(ln, S::AS_LANES - 1);
        return (uint32_t)min(t0 + t, T - 1) * KB * 4;        // bytes
    };
    const uint8_t *qg = reinterpret_cast<const uint8_t *>(a.q);
    const uint8_t *cg = W.codes;
    const uint8_t *sg = reinterpret_cast<const uint8_t *>(W.scales);
    const uint8_t *ag = reinterpret_cast<const uint8_t *>(a.ascale);
    auto issue = [&](int kb, int st) {
        int ln = lane;
        asm volatile("" : "+v"(ln));                         // (not loop-invariant, so not hoisted)
        uint8_t *base = smem + st * STAGE;
#pragma unroll
        for (int i = 0; i < S::A_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(qg + (size_t)kb * kTileK + a_off(ln, i)),
                                             KXW4_GR_LDS(base + ((wave + NW * i) % S::A_CHUNKS) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < S::W_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(cg + (size_t)kb * kTileBytes + w_off(ln, i)),
                                             KXW4_GR_LDS(base + S::W_OFF + ((wave + NW * i) % RGS) * 1024), 16, 0, 0);
        // lanes past the wave's granules are masked off; the load still
        // counts once in vmcnt
        if (lane < S::S_LANES)
            __builtin_amdgcn_global_load_lds((const void *)(sg + (size_t)kb * GPS * 32 + s_off(ln)),
                                             KXW4_GR_LDS(base + S::S_OFF + (wave * S::S_LANES) % S::S_TOTAL * 16),
                                             16, 0, 0);
        // (lanes past a partial load's tokens are masked off; the load
        // still counts once in vmcnt)
#pragma unroll
        for (int i = 0; i < S::AS_LOADS; ++i)
            if (S::AS_LANES == 64 || lane < S::AS_LANES)
                __builtin_amdgcn_global_load_lds((const void *)(ag + (size_t)kb * 16 + as_off(ln, i)),
                                                 KXW4_GR_LDS(base + S::AS_OFF + ((wave + NW * i) % S::AS_CHUNKS) * S::AS_LANES * 16),
                                                 16, 0, 0);
    };

    // ---- per-lane read offsets: lane = weight row / token m of a block,
    // K group kg (lane groups 2kg and 2kg + 1 of the packed layout) ----
    const int m = lane & 31, kg = lane >> 5;
    const int rgl = 2 * wr + (m >> 4);                       // tile row-group of this lane's operand row
    const int w_lds = S::W_OFF + rgl * kTileBytes + (32 * kg + (m & 15)) * 16;
    const int zz_lds = S::ZZ_OFF + rgl * GPS * 16 + (m & 15);
    // weight scales of this lane's output rows 8q + 4kg + e (e = 0..3) of
    // the wave's row block: row-group 2wr + q/2, rows 8(q%2) + 4kg + e
    const int ws_lds = (ZP ? S::MS_OFF : S::S_OFF) + 2 * wr * GPS * 32 + 8 * kg;   // + (q/2) GPS 32 + (q%2) 16
    // activation pieces of token block j: row tb + m, pieces 4c + 2kg + {0,1}
    const int tb = wt * NT * 32;                             // first token of this wave in the tile
    const int tsw = ((tb + m) >> 1) & 7;                     // the row's swizzle (tb is a multiple of 32)
    const int a_row = (tb + m) * kTileK;
    const int as_lds = S::AS_OFF + (tb + m) * 16;

    float f[NT][16];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) f[j][r] = 0.0f;

    static_assert(NST >= 2 && NST <= 4, "two to four stages");
    constexpr int LD = S::LOADS;
    static_assert(LD * (NST - 2) <= 63, "vmcnt field");
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < NTK) issue(s, s);
    // Step kb reads stage kb % NST. (Unrolling the K loop over the ring, so
    // that the stage is a compile-time index, makes every instance with a
    // ring under 64 KB spill.)
    int st = 0;
    for (int kb = 0; kb < NTK; ++kb) {
        const int later = min(NST - 2, NTK - 1 - kb);
        if (NST >= 4 && later >= 2) KXW4_WAIT_VMCNT(2 * LD);
        else if (NST >= 3 && later >= 1) KXW4_WAIT_VMCNT(LD);
        else KXW4_WAIT_VMCNT(0);
        const uint8_t *sb = smem + st * STAGE;
        if constexpr (ZP) {
            // the scale granules this wave loaded into the stage (8 rows of
            // one row-group and scale group each): masked scales and
            // zero-point bytes, published by the barrier below (written to
            // their own regions, so a granule two waves loaded is prepared
            // twice with the same values)
            if (lane < S::S_LANES) {
                const int gi = (wave * S::S_LANES) % S::S_TOTAL + lane;
                const v4u p = *reinterpret_cast<const v4u *>(sb + S::S_OFF + gi * 16);
                v4u ms;
                ms.x = p.x & 0xFFF0FFF0u;
                ms.y = p.y & 0xFFF0FFF0u;
                ms.z = p.z & 0xFFF0FFF0u;
                ms.w = p.w & 0xFFF0FFF0u;
                *reinterpret_cast<v4u *>(const_cast<uint8_t *>(sb) + S::MS_OFF + gi * 16) = ms;
                // z + 8 = (p & 15) ^ 8 of each row, one byte per row: bytes
                // 0 and 2 of each dword pair up with the two rows it holds
                uint2 zb;
                zb.x = __builtin_amdgcn_perm(p.y, p.x, 0x06040200u) & 0x0F0F0F0Fu;
                zb.y = __builtin_amdgcn_perm(p.w, p.z, 0x06040200u) & 0x0F0F0F0Fu;
                zb.x ^= 0x08080808u;
                zb.y ^= 0x08080808u;
                *reinterpret_cast<uint2 *>(const_cast<uint8_t *>(sb) + S::ZZ_OFF + gi * 8) = zb;
            }
        }
        lds_sync_after_dma();
        if (kb + NST - 1 < NTK) issue(kb + NST - 1, st == 0 ? NST - 1 : st - 1);
        // The step is I = 4 NT items (unit u, token block j), j fastest, run
        // as a software pipeline: item i + 2's operands are read from LDS
        // and item i + 1's MFMA issued before item i's chain updates, so the
        // chain runs while the matrix core works and only two MFMA results
        // are live.
        constexpr int I = 4 * NT;
        // zero-point bytes (z + 8) * 0x01010101 of the operand row for
        // scale group g
        auto zc_of = [&](int g) -> uint32_t {
            if constexpr (ZP) return __builtin_amdgcn_perm(0u, (uint32_t)*(sb + zz_lds + g * 16), 0u);
            else return 0u;
        };
        // the step's packed weight dwords of this lane's operand row: dword
        // u of lane groups 2kg (wd0) and 2kg + 1 (wd1) is unit u (the lean
        // pipeline reads each unit's two dwords when it unpacks them)
        v4u wd0 = {}, wd1 = {};
        uint32_t zc[GPS];
        if constexpr (!LEAN) {
            wd0 = *reinterpret_cast<const v4u *>(sb + w_lds);
            wd1 = *reinterpret_cast<const v4u *>(sb + w_lds + 256);
#pragma unroll
            for (int g = 0; g < GPS; ++g) zc[g] = zc_of(g);
        }
        // FP16 scales of the 16 output rows of scale group g (the zero-point
        // nibble cleared): dword r/2, half r%2 is register r's row
        auto read_ws = [&](int g, uint32_t (&w)[8]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint2 v = *reinterpret_cast<const uint2 *>(sb + ws_lds + (q >> 1) * GPS * 32 + (q & 1) * 16 + g * 32);
                w[2 * q] = v.x;
                w[2 * q + 1] = v.y;
            }
        };
        // item i's activation operand (this unit's 8 bytes of pieces
        // 4c + 2kg and 4c + 2kg + 1 of the lane's token) and scale
        auto read_b = [&](int i, v4i &B, float &as) {
            const int u = i / NT, j = i % NT, c = u >> 1, h = u & 1;
            const int s0 = ((4 * c + 2 * kg) ^ tsw) * 16 + 8 * h;
            const int s1 = ((4 * c + 2 * kg + 1) ^ tsw) * 16 + 8 * h;
            const uint2 b0 = *reinterpret_cast<const uint2 *>(sb + a_row + j * 32 * kTileK + s0);
            const uint2 b1 = *reinterpret_cast<const uint2 *>(sb + a_row + j * 32 * kTileK + s1);
            B.x = (int)b0.x;
            B.y = (int)b0.y;
            B.z = (int)b1.x;
            B.w = (int)b1.y;
            as = *reinterpret_cast<const float *>(sb + as_lds + j * 32 * 16 + u * 4);
        };
        auto unpack = [&](int u) {
            if constexpr (LEAN) {
                const uint32_t d0 = *reinterpret_cast<const uint32_t *>(sb + w_lds + 4 * u);
                const uint32_t d1 = *reinterpret_cast<const uint32_t *>(sb + w_lds + 256 + 4 * u);
                return gr_unpack<ZP>(d0, d1, zc_of((u * 32) / GROUP));
            } else {
                return gr_unpack<ZP>(wd0[u], wd1[u], zc[(u * 32) / GROUP]);
            }
        };
        // item i's chain updates: four outputs at a time, their products,
        // conversions, then the FMAs (a product read by the very next
        // instruction costs a wait state)
        // (two at a time in the lean pipeline, whose registers are short)
        constexpr int CHK = LEAN ? 2 : 4;
        auto chain = [&](int j, const v16i &d, const uint32_t (&wsr)[8], float as) {
#pragma unroll
            for (int r0 = 0; r0 < 16; r0 += CHK) {
                float wa[CHK], pv[CHK];
#pragma unroll
                for (int e = 0; e < CHK; ++e) {
                    const int r = r0 + e;
                    const uint32_t wv = wsr[r >> 1];
                    const float wsv = (float)__builtin_bit_cast(_Float16, (uint16_t)((r & 1) ? (wv >> 16) : wv));
                    // ws * as rounded once: fma(ws, as, +0) equals the
                    // product except for its zero sign, which the chain's
                    // fma ignores (the accumulator is never -0)
                    wa[e] = __builtin_fmaf(wsv, as, 0.0f);
                }
#pragma unroll
                for (int e = 0; e < CHK; ++e) pv[e] = (float)d[r0 + e];
#pragma unroll
                for (int e = 0; e < CHK; ++e) f[j][r0 + e] = __builtin_fmaf(pv[e], wa[e], f[j][r0 + e]);
            }
        };
        constexpr int UPG = GROUP / 32;                      // units per scale group
        const v16i zero = {};
        if constexpr (LEAN) {
            // Few registers (more waves per SIMD hide the latencies): item
            // i + 1's operands are read during item i, and each item's
            // chain follows its own MFMA.
            uint32_t wsr[8];
            v4i Bq[2];
            float asq[2];
            read_b(0, Bq[0], asq[0]);
            v4i A;
#pragma unroll
            for (int i = 0; i < I; ++i) {
                const int u = i / NT, j = i % NT;
                if (i + 1 < I) read_b(i + 1, Bq[(i + 1) & 1], asq[(i + 1) & 1]);
                if (j == 0) {
                    if (u % UPG == 0) read_ws(u / UPG, wsr);
                    A = unpack(u);
                }
                const v16i d = mfma32(A, Bq[i & 1], zero);
                chain(j, d, wsr, asq[i & 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            uint32_t wsr[8], wsn[8];
            v4i Bq[3];
            float asq[3];
            v16i dq[2];
            read_ws(0, wsr);
            read_b(0, Bq[0], asq[0]);
            read_b(1, Bq[1], asq[1]);
            v4i A = unpack(0);
            dq[0] = mfma32(A, Bq[0], zero);
            // (the scheduling barriers keep each iteration's MFMA ahead of
            // the previous item's chain; otherwise the MFMA that follows a
            // unit's weight unpack drifts below the chain and the next
            // item's chain waits for it)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < I; ++i) {
                const int u = i / NT, j = i % NT;
                // a unit after this one that starts a new scale group
                const bool next_group = u + 1 < 4 && (u + 1) % UPG == 0;
                if (i + 2 < I) read_b(i + 2, Bq[(i + 2) % 3], asq[(i + 2) % 3]);
                if (j == 0 && next_group) read_ws((u + 1) / UPG, wsn);
                if (i + 1 < I) {
                    if ((i + 1) % NT == 0) A = unpack(u + 1);
                    dq[(i + 1) & 1] = mfma32(A, Bq[(i + 1) % 3], zero);
                }
                __builtin_amdgcn_sched_barrier(0);
                chain(j, dq[i & 1], wsr, asq[i % 3]);
                if (j == NT - 1 && next_group) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) wsr[e] = wsn[e];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        st = st == NST - 1 ? 0 : st + 1;
    }

    // ---- output: one token block at a time through the wave's LDS slab
    // [token][row], read back as 16-byte row runs of one token ----
    lds_sync();
    float *slab = reinterpret_cast<float *>(smem + wave * S::SLAB);
    constexpr float kScale = ZP ? 1.0f : 0.0625f;            // the 16 w unpack's factor
    const int row0 = (rg0 + 2 * wr) * 16;                    // first row of the wave's block
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r) slab[m * S::EPS + 8 * (r >> 2) + 4 * kg + (r & 3)] = f[j][r];
        // (the slab is this wave's own and its LDS accesses complete in order)
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int qi = it * 64 + lane;
            const int tl = qi >> 3, rl = (qi & 7) * 4;
            const int t = t0 + tb + 32 * j + tl;
            const int row = row0 + rl;
            if (t >= T || row >= M) continue;
            const float4 x = *reinterpret_cast<const float4 *>(slab + tl * S::EPS + rl);
            float v0 = x.x * kScale, v1 = x.y * kScale, v2 = x.z * kScale, v3 = x.w * kScale;
            if (a.residual) {
                const float4 rr = *reinterpret_cast<const float4 *>(a.residual + (size_t)t * M + row);
                v0 = v0 + rr.x;
                v1 = v1 + rr.y;
                v2 = v2 + rr.z;
                v3 = v3 + rr.w;
            }
            if (a.y_bf16) {
                uint2 o;
                o.x = (uint32_t)float_to_bf16(v0) | ((uint32_t)float_to_bf16(v1) << 16);
                o.y = (uint32_t)float_to_bf16(v2) | ((uint32_t)float_to_bf16(v3) << 16);
                *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(W.y) + (size_t)t * M + row) = o;
            } else {
                *reinterpret_cast<float4 *>(static_cast<float *>(W.y) + (size_t)t * M + row) = make_float4(v0, v1, v2, v3);
            }
        }
    }
}

template <int NT, int WR, int WT, int GROUP, bool ZP, int NST, int OCC>
static int launch_gr(GemmArgs &a, hipStream_t st) {
    using S = GrShape<NT, WR, WT, GROUP>;
    int nt = 0;
    for (int i = 0; i < a.count; ++i) {
        a.w[i].nt_begin = nt;
        nt += (a.w[i].M / 16 + S::RGS - 1) / S::RGS;
    }
    a.n_tiles = nt;
    a.t_tiles = (a.T + S::BM - 1) / S::BM;
    const dim3 grid(a.n_tiles * a.t_tiles), block(S::NTH);
    auto k = gemmr_kernel<NT, WR, WT, GROUP, ZP, NST, OCC>;
    const size_t lds = (size_t)S::template lds_bytes<NST>();
    static_assert(S::template lds_bytes<NST>() <= 160 * 1024, "LDS");
    // the attribute is per device
    static bool attr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -6;
    if (!attr[dev]) {
        if (hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return -6;
        attr[dev] = true;
    }
    hipLaunchKernelGGL(k, grid, block, lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Tiles (wave tile 32 rows x 32*NT tokens). The kernel is bound by each
// SIMD's VALU issue, so what decides is how evenly the 32x32 blocks spread
// over the SIMDs and how many waves share a SIMD (graph replay, bit-exact,
// T=2048 K=N=5120 group 32 / T=512 K=17408 N=5120 group 64):
//   4: 128 x 64, 4 waves of 2 token blocks, four work-groups per CU:
//     205 / 315 us (the default while its grid gives every CU at least
//     three work-groups);
//   9: 128 x 32, 4 waves of one token block, five work-groups per CU:
//     226 / 277 us (the default for smaller grids);
//   0: 160 x 256, 10 waves of 4 token blocks (3, 3, 2, 2 per SIMD), one
//     work-group per CU: 230 / 760 us;
//   5: 160 x 64, 10 waves of one token block: 374 / 310 us;
//   1, 2, 3, 6, 7, 8: 4- and 5-wave tiles with 4 token blocks, and lean
//     (one MFMA result live) tiles at 5 or 6 waves per SIMD: all slower.
template <int GROUP, bool ZP>
static int launch_gr_tile(GemmArgs &a, int sel, hipStream_t st) {
    switch (sel) {
    case 0: return launch_gr<4, 5, 2, GROUP, ZP, 3, 3>(a, st);    // 160 rows x 256 tokens, 10 waves
    case 1: return launch_gr<4, 4, 1, GROUP, ZP, 2, 3>(a, st);    // 128 rows x 128 tokens, 4 waves
    case 2: return launch_gr<4, 5, 1, GROUP, ZP, 2, 3>(a, st);    // 160 rows x 128 tokens, 5 waves
    case 3: return launch_gr<2, 5, 2, GROUP, ZP, 3, 3>(a, st);    // 160 rows x 128 tokens, 10 waves
    case 5: return launch_gr<1, 5, 2, GROUP, ZP, 3, 3>(a, st);    // 160 rows x 64 tokens, 10 waves
    case 6: return launch_gr<2, 5, 1, GROUP, ZP, 2, 5>(a, st);    // 160 rows x 64 tokens, 5 waves, lean
    case 7: return launch_gr<1, 4, 2, GROUP, ZP, 2, 6>(a, st);    // 128 rows x 64 tokens, 8 waves, lean
    case 8: return launch_gr<2, 4, 1, GROUP, ZP, 2, 5>(a, st);    // 128 rows x 64 tokens, 4 waves, lean
    case 9: return launch_gr<1, 4, 1, GROUP, ZP, 2, 4>(a, st);    // 128 rows x 32 tokens, 4 waves
    default: return launch_gr<2, 4, 1, GROUP, ZP, 2, 3>(a, st);   // 128 rows x 64 tokens, 4 waves (4)
    }
}

int launch_gemmr(GemmArgs &a, hipStream_t st) {
    // activation scales per (token, K32 block), one split per token, W4 codes
    if (a.block != 32 || a.w8 || (a.group != 32 && a.group != 64 && a.group != 128)) return 1;
    if (a.scale_enc == 1 && a.group == 128) return 1;
    if ((long long)a.T * a.K >= (1ll << 31)) return 1;               // 32-bit activation offsets
    for (int i = 0; i < a.count; ++i) {
        if ((long long)a.w[i].M * a.K / 2 >= (1ll << 31)) return 1;
        for (int s = 0; s < a.seg_count; ++s)
            if (a.w[i].seg_split[s] != 1) return 1;
    }
    int sel = options().gemmr_tile;
    if (sel < 0) {
        long long tiles = 0;
        for (int i = 0; i < a.count; ++i) tiles += (a.w[i].M / 16 + 7) / 8;
        tiles *= (a.T + 63) / 64;
        sel = tiles >= 3LL * device_cus() ? 4 : 9;
    }
    const bool zp = a.scale_enc == 1;
    switch (a.group) {
    case 32: return zp ? launch_gr_tile<32, true>(a, sel, st) : launch_gr_tile<32, false>(a, sel, st);
    case 64: return zp ? launch_gr_tile<64, true>(a, sel, st) : launch_gr_tile<64, false>(a, sel, st);
    default: return launch_gr_tile<128, false>(a, sel, st);
    }
}

}  // namespace kxw4
