// kxw4_gemm3.hip — prefill projections in the per-token mode (the BASELINE
// configurations) on the 32x32x32 int8 MFMA: x_gemm_w4a8 / gemm_rc16
// arithmetic (kernels_dpas.cpp:1255-1332, 1334-1490) with one split per
// token.
//
// Cost model (measured on the MI355X): the FP32 chain needs one int->float
// conversion and one FMA per output and weight group, as many VALU cycles as
// the MFMA cycles of a 16x16x64 product over a 128-K group. A 16x16x64 int8
// MFMA leaves the VALU about one free issue slot, so with it the two simply
// add up; a 32x32x32 int8 MFMA (twice the work, twice the cycles) leaves
// about five, so most of the chain runs under the matrix core. Hence:
//   * each wave owns a 32*TA token x 32*TB row tile of 32x32 blocks; a block
//     is four dependent MFMAs over a 128-K step followed by its 16 chain
//     updates per lane, and the scheduler overlaps one block's updates with
//     the next block's MFMAs;
//   * the unpacked weight operands of a step stay in registers, the
//     activation operands stream one 32-token block at a time;
//   * the work-group is WMW x WNW waves; each packed weight tile is unpacked
//     by one wave only;
//   * per 128-K step the activation tile, the packed weight tiles and the
//     FP16 scales reach LDS through direct global->LDS loads into a ring of
//     NST stages; every wave issues the same number of loads per stage, so
//     one vmcnt retires a stage, and one barrier per step both publishes the
//     stage and frees the one refilled next.
//
// Operand K sets: the packed tile keeps the 16x16x64 lane order (lane n+16g
// holds row n, K slots of lane group g of both 64-K halves). MFMA c of a step
// gives K group kg (lanes 32kg..) the 16-slot set of 16x16 lane group
// g = kg + 2*(c/2) in half c%2; its activation bytes are 16-byte chunk
// 4*(c%2) + g of the row. Activation rows are XOR-swizzled on the load side
// (chunk c of row t lands at chunk c ^ ((t/2) & 7) of a 256-byte row pair),
// so the 16-byte reads of each 16-lane quarter hit distinct bank groups.
//
// The FP32 chain of each output is f = fma((float)P_u, ws_u, f) over the
// weight groups u in K order; the token scale and the 1/16 of the nibble
// unpack (every MFMA result is 16 P_u exactly) are applied once at the end.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace kxw4 {

constexpr int kG3GroupTT = 4;      // token tiles per raster group

#define KXW4_G3_LDS(p) ((__attribute__((address_space(3))) void *)(p))

template <int TA, int TB, int WMW, int WNW, int UNIT>
struct G3Shape {
    static constexpr int NW = WMW * WNW;
    static constexpr int NTH = 64 * NW;
    static constexpr int BM = WMW * 32 * TA;             // tokens per tile
    static constexpr int BNG = WNW * 2 * TB;             // row-groups per tile
    static constexpr int UPS = kTileK / UNIT;
    static constexpr int A_BYTES = BM * kTileK;
    static constexpr int B_BYTES = BNG * kTileBytes;
    static constexpr int S_BYTES = BNG * UPS * 32;       // [row-group][unit][16] FP16
    static constexpr int STAGE = (A_BYTES + B_BYTES + S_BYTES + 1023) / 1024 * 1024;
    // Loads per wave and stage. Every wave issues the same number (one vmcnt
    // retires a stage); when the waves do not divide the 1 KB chunks, the
    // chunk index wraps and a few chunks are loaded twice (same bytes to the
    // same LDS address).
    static constexpr int A_CHUNKS = A_BYTES / 1024;
    static constexpr int A_LOADS = (A_CHUNKS + NW - 1) / NW;
    static constexpr int B_LOADS = (BNG + NW - 1) / NW;
    static constexpr int S_TOTAL = BNG * UPS * 2;        // 16-byte scale granules per stage
    // granules per wave: the smallest divisor of S_TOTAL that covers it with
    // NW waves, so a wave's wrapped range never straddles the wrap point
    static constexpr int s_lanes() {
        int d = (S_TOTAL + NW - 1) / NW;
        while (S_TOTAL % d) ++d;
        return d;
    }
    static constexpr int S_LANES = s_lanes();
    static constexpr int LOADS = A_LOADS + B_LOADS + 1;
    // output staging: a wave's slab of SB token blocks x 32*TB rows of FP32,
    // token stride EPS floats (EPS = 8 mod 16, so the two K groups of one
    // LDS write land in opposite halves of the banks), inside the ring
    static constexpr int EPS = 32 * TB + 8;
    static constexpr int slab_bytes(int sb) { return 32 * sb * EPS * 4; }
    template <int NST>
    static constexpr int slab_blocks() {
        return NW * slab_bytes(TA) <= NST * STAGE ? TA
             : (TA % 2 == 0 && NW * slab_bytes(TA / 2) <= NST * STAGE) ? TA / 2 : 1;
    }
    // the ring, or the output slabs where they need more, then the per-token
    // activation scales of the tile
    template <int NST>
    static constexpr int body_bytes() {
        return NST * STAGE > NW * slab_bytes(slab_blocks<NST>()) ? NST * STAGE : NW * slab_bytes(slab_blocks<NST>());
    }
    template <int NST>
    static constexpr int lds_bytes() { return body_bytes<NST>() + BM * 4; }
    static_assert(A_BYTES % 1024 == 0, "activation tile in whole 1 KB chunks");
    static_assert(S_LANES <= 64, "one scale load per wave and stage");
};

// OCC: waves per SIMD the register budget is sized for
template <int TA, int TB, int WMW, int WNW, int UNIT, int NST, int OCC>
__global__ __launch_bounds__(64 * WMW * WNW)
__attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm3_kernel(const GemmArgs a) {
    using S = G3Shape<TA, TB, WMW, WNW, UNIT>;
    constexpr int NW = S::NW, BM = S::BM, BNG = S::BNG, UPS = S::UPS;
    constexpr int A_BYTES = S::A_BYTES, B_BYTES = S::B_BYTES, STAGE = S::STAGE;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // ---- block -> (token tile, weight, n-tile), XCD-aware raster: the
    // work-groups of one XCD (blockIdx % 8) take consecutive tiles, grouped
    // kG3GroupTT token tiles at a time so they share activation and weight
    // tiles in that XCD's L2 ----
    const int nblk = gridDim.x, id = blockIdx.x;
    const int q8 = nblk / 8, r8 = nblk % 8, xcd = id % 8, j8 = id / 8;
    const int L = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int nnt = a.n_tiles, ntt = a.t_tiles;
    const int group = L / (kG3GroupTT * nnt);
    const int first = group * kG3GroupTT;
    const int gsz = min(ntt - first, kG3GroupTT);
    const int within = L % (kG3GroupTT * nnt);
    const int tt = first + within % gsz;
    const int ntg = within / gsz;
    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (ntg >= a.w[i].nt_begin) wi = i;
    const GemmWeight &W = a.w[wi];
    const int M = W.M, RG = M / 16;
    const int rg0 = (ntg - W.nt_begin) * BNG;
    const int t0 = tt * BM;
    const int K = a.K, T = a.T, NT = K / kTileK, G = K / UNIT;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;

    // ---- load issue: per-lane 32-bit source offsets that do not depend on
    // the K step (the launcher keeps T*K and M*K/2 below 2^31) ----
    uint32_t aoffs[S::A_LOADS];
#pragma unroll
    for (int i = 0; i < S::A_LOADS; ++i) {
        const int p = ((wave + NW * i) % S::A_CHUNKS) * 64 + lane;            // granule this lane fills
        const int t = 2 * (p >> 4) + ((p >> 3) & 1);
        const int c16 = (p & 7) ^ ((t >> 1) & 7);
        const int tg = min(t0 + t, T - 1);                    // rows past T: never stored
        aoffs[i] = (uint32_t)tg * K + c16 * 16;
    }
    uint32_t boffs[S::B_LOADS];
#pragma unroll
    for (int i = 0; i < S::B_LOADS; ++i) {
        const int rg = min(rg0 + (wave + NW * i) % BNG, RG - 1);      // row-groups past M: never stored
        boffs[i] = (uint32_t)rg * NT * kTileBytes + lane * 16;
    }
    // scale granule gi = (j * UPS + u) * 2 + half of this wave's slice
    uint32_t soff;
    {
        const int gi = (wave * S::S_LANES + min(lane, S::S_LANES - 1)) % S::S_TOTAL;
        const int j = gi / (2 * UPS), u = (gi >> 1) % UPS, half = gi & 1;
        const int rg = min(rg0 + j, RG - 1);
        soff = ((uint32_t)rg * G + u) * 16 + half * 8;
    }
    // (the DMA builtin takes a generic void pointer: with a typed pointer the
    // host compilation pass drops the kernel without a diagnostic)
    auto issue = [&](int kb, int st) {
        uint8_t *base = smem + st * STAGE;
        const int8_t *qk = a.q + (size_t)kb * kTileK;
        const uint8_t *wk = W.codes + (size_t)kb * kTileBytes;
#pragma unroll
        for (int i = 0; i < S::A_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(qk + aoffs[i]),
                                             KXW4_G3_LDS(base + ((wave + NW * i) % S::A_CHUNKS) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < S::B_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(wk + boffs[i]),
                                             KXW4_G3_LDS(base + A_BYTES + ((wave + NW * i) % BNG) * 1024), 16, 0, 0);
        // lanes past the wave's granules are masked off; the load still
        // counts once in vmcnt
        if (lane < S::S_LANES)
            __builtin_amdgcn_global_load_lds((const void *)(W.scales + (size_t)kb * UPS * 16 + soff),
                                             KXW4_G3_LDS(base + A_BYTES + B_BYTES + (wave * S::S_LANES) % S::S_TOTAL * 16),
                                             16, 0, 0);
        // with the first stage, the tile's token scales (64 per wave); the
        // later stages' loads are all younger, so the first wait retires it
        if (kb == 0 && wave * 64 < BM)
            __builtin_amdgcn_global_load_lds((const void *)(a.ascale + min(t0 + wave * 64 + lane, T - 1)),
                                             KXW4_G3_LDS(smem + S::template body_bytes<NST>() + wave * 256), 4, 0, 0);
    };

    // ---- per-lane read offsets (lane = row/column l%32, K group l/32) ----
    const int m32 = lane & 31, kg = lane >> 5;
    const int tw = wm * 32 * TA;                               // first token of this wave in the tile
    const int hx = (m32 >> 1) & 7;                             // XOR of this lane's rows (tw/2 is a multiple of 16)
    int aoff[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int c16 = 4 * (c & 1) + kg + 2 * (c >> 1);
        aoff[c] = (((tw >> 1) + (m32 >> 1)) * 16 + (((m32 & 1) << 3) | (c16 ^ hx))) * 16;
    }
    // row-group (relative to the tile) of this lane's column in 32-row block jb
    const int jrel0 = wn * 2 * TB + (m32 >> 4);
    const int boff = A_BYTES + jrel0 * kTileBytes + (kg * 16 + (m32 & 15)) * 16;
    const int soff_lds = A_BYTES + B_BYTES + (jrel0 * UPS * 16 + (m32 & 15)) * 2;

    float f[TA][TB][16];
#pragma unroll
    for (int i = 0; i < TA; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) f[i][j][r] = 0.0f;

    // Ring of NST stages; stage k % NST is issued at the top of step
    // k - (NST - 1). At the top of step k this wave's loads of steps
    // k .. k + NST - 2 may be outstanding; vmcnt(LOADS * later) retires step
    // k's, where `later` counts the stages issued after it. The barrier then
    // publishes every wave's loads and guarantees that stage (k - 1) % NST,
    // refilled next, is no longer read.
    static_assert(NST >= 2 && NST <= 4, "two to four stages");
    constexpr int LD = S::LOADS;
    static_assert(LD * (NST - 2) <= 63, "vmcnt field");
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < NT) issue(s, s);
    int st = 0;
    for (int kb = 0; kb < NT; ++kb) {
        const int later = min(NST - 2, NT - 1 - kb);
        if (NST >= 4 && later >= 2) KXW4_WAIT_VMCNT(2 * LD);
        else if (NST >= 3 && later >= 1) KXW4_WAIT_VMCNT(LD);
        else KXW4_WAIT_VMCNT(0);
        lds_sync_after_dma();
        if (kb + NST - 1 < NT) issue(kb + NST - 1, st == 0 ? NST - 1 : st - 1);
        const uint8_t *sb = smem + st * STAGE;
        // weight operands of the step: block jb, MFMA c = 2h + half
        v4i B[TB][4];
        float w[TB][UPS];
#pragma unroll
        for (int jb = 0; jb < TB; ++jb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const v4u wd = *reinterpret_cast<const v4u *>(sb + boff + jb * 2 * kTileBytes + h * 512);
                B[jb][2 * h] = unpack_k64(wd.x, wd.y);
                B[jb][2 * h + 1] = unpack_k64(wd.z, wd.w);
            }
#pragma unroll
            for (int u = 0; u < UPS; ++u)
                w[jb][u] = half_bits_to_float(
                    *reinterpret_cast<const uint16_t *>(sb + soff_lds + (jb * 2 * UPS + u) * 32));
        }
        // Software pipeline over the step's TA*TB blocks (row block jb
        // fastest): stage b issues block b's MFMAs interleaved with block
        // b-1's chain updates, so the updates run while the matrix core
        // works. The activation operands of the next token block are read
        // during the last stage of the current one.
        constexpr int NB = TA * TB;
        v4i Acur[4], Anext[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) Acur[c] = *reinterpret_cast<const v4i *>(sb + aoff[c]);
        // acc[slot][u]: the 64-K group u of a block (one group per block
        // at group 128, where MFMAs 0-3 chain into acc[.][0]; at group 64
        // the first 64-K half is MFMAs 0 and 2, the second 1 and 3)
        v16i acc[2][UPS];
        const v16i zero = {};
        auto update = [&](int b) {
            const int ib = b / TB, jb = b % TB;
#pragma unroll
            for (int u = 0; u < UPS; ++u) {
                const v16i &p = acc[b & 1][u];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    f[ib][jb][r] = __builtin_fmaf((float)p[r], w[jb][u], f[ib][jb][r]);
            }
        };
#pragma unroll
        for (int b = 0; b <= NB; ++b) {
            if (b < NB) {
                const int ib = b / TB, jb = b % TB;
                if (jb == 0 && ib > 0) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) Acur[c] = Anext[c];
                }
                if (jb == TB - 1 && ib + 1 < TA) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        Anext[c] = *reinterpret_cast<const v4i *>(sb + aoff[c] + (ib + 1) * 4096);
                }
                if constexpr (UNIT == 128) {
                    v16i &p = acc[b & 1][0];
                    p = mfma32(Acur[0], B[jb][0], zero);
                    p = mfma32(Acur[1], B[jb][1], p);
                    p = mfma32(Acur[2], B[jb][2], p);
                    p = mfma32(Acur[3], B[jb][3], p);
                } else {
                    static_assert(UNIT == 64, "per-token mode has unit = group in {64, 128}");
                    v16i &p0 = acc[b & 1][0];
                    v16i &p1 = acc[b & 1][UPS - 1];
                    p0 = mfma32(Acur[0], B[jb][0], zero);
                    p1 = mfma32(Acur[1], B[jb][1], zero);
                    p0 = mfma32(Acur[2], B[jb][2], p0);
                    p1 = mfma32(Acur[3], B[jb][3], p1);
                }
            }
            if (b > 0) update(b - 1);
            if (b > 0 && b < NB) {
                // one MFMA, then the VALU share of the previous block's
                // updates, four times
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 8 * UPS, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        st = st == NST - 1 ? 0 : st + 1;
    }

    // ---- output ----
    // Each wave stages SB token blocks at a time in its own LDS slab (the
    // ring is free once every wave is past its last step) and writes whole
    // 16-byte row runs: register r of block (ib, jb) is token
    // 8(r/4) + 4kg + r%4 and row m32 of the block.
    constexpr int EPS = S::EPS, SB = S::template slab_blocks<NST>();
    static_assert(TA % SB == 0, "slabs cover the wave tile");
    static_assert(S::template lds_bytes<NST>() <= 160 * 1024, "LDS");
    lds_sync();
    float *slab = reinterpret_cast<float *>(smem) + wave * (32 * SB * EPS);
    const float *tsc = reinterpret_cast<const float *>(smem + S::template body_bytes<NST>());
#pragma unroll
    for (int s0 = 0; s0 < TA; s0 += SB) {
#pragma unroll
        for (int ib = s0; ib < s0 + SB; ++ib)
#pragma unroll
            for (int jb = 0; jb < TB; ++jb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    slab[(32 * (ib - s0) + 8 * (r >> 2) + 4 * kg + (r & 3)) * EPS + 32 * jb + m32] = f[ib][jb][r];
        // read back runs of CH rows of one token (CH = 8 BF16 or 4 FP32
        // outputs = 16 bytes); the slab is this wave's own, and its LDS
        // accesses complete in order
        auto run = [&](auto ch) {
            constexpr int CH = decltype(ch)::value;
            constexpr int PER_TOKEN = 32 * TB / CH;
#pragma unroll
            for (int it = 0; it < 32 * SB * PER_TOKEN / 64; ++it) {
                const int q = it * 64 + lane;
                const int tl = q / PER_TOKEN, rl = (q % PER_TOKEN) * CH;
                const int t = t0 + tw + 32 * s0 + tl;
                const int rg = rg0 + wn * 2 * TB + (rl >> 4);
                if (t >= T || rg >= RG) continue;
                const int row = rg * 16 + (rl & 15);
                const float sc = tsc[tw + 32 * s0 + tl] * 0.0625f;
                float v[CH];
#pragma unroll
                for (int e = 0; e < CH; e += 4) {
                    const float4 x = *reinterpret_cast<const float4 *>(slab + tl * EPS + rl + e);
                    v[e] = x.x * sc;
                    v[e + 1] = x.y * sc;
                    v[e + 2] = x.z * sc;
                    v[e + 3] = x.w * sc;
                }
                if (a.residual) {
#pragma unroll
                    for (int e = 0; e < CH; e += 4) {
                        const float4 x = *reinterpret_cast<const float4 *>(a.residual + (size_t)t * M + row + e);
                        v[e] = v[e] + x.x;
                        v[e + 1] = v[e + 1] + x.y;
                        v[e + 2] = v[e + 2] + x.z;
                        v[e + 3] = v[e + 3] + x.w;
                    }
                }
                if constexpr (CH == 8) {
                    uint4 o;
                    o.x = (uint32_t)float_to_bf16(v[0]) | ((uint32_t)float_to_bf16(v[1]) << 16);
                    o.y = (uint32_t)float_to_bf16(v[2]) | ((uint32_t)float_to_bf16(v[3]) << 16);
                    o.z = (uint32_t)float_to_bf16(v[4]) | ((uint32_t)float_to_bf16(v[5]) << 16);
                    o.w = (uint32_t)float_to_bf16(v[6]) | ((uint32_t)float_to_bf16(v[7]) << 16);
                    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(W.y) + (size_t)t * M + row) = o;
                } else {
                    *reinterpret_cast<float4 *>(static_cast<float *>(W.y) + (size_t)t * M + row) =
                        make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        };
        if (a.y_bf16) run(std::integral_constant<int, 8>{});
        else run(std::integral_constant<int, 4>{});
    }
}

template <int TA, int TB, int WMW, int WNW, int UNIT, int NST, int OCC = 2>
static int launch_g3(GemmArgs &a, hipStream_t st) {
    using S = G3Shape<TA, TB, WMW, WNW, UNIT>;
    int nt = 0;
    for (int i = 0; i < a.count; ++i) {
        a.w[i].nt_begin = nt;
        nt += (a.w[i].M / 16 + S::BNG - 1) / S::BNG;
    }
    a.n_tiles = nt;
    a.t_tiles = (a.T + S::BM - 1) / S::BM;
    const dim3 grid(a.n_tiles * a.t_tiles), block(S::NTH);
    auto k = gemm3_kernel<TA, TB, WMW, WNW, UNIT, NST, OCC>;
    const size_t lds = (size_t)S::template lds_bytes<NST>();
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return -6;
        attr = true;
    }
    hipLaunchKernelGGL(k, grid, block, lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_gemm3(GemmArgs &a, hipStream_t st) {
    // per-token activation scale, plain FP16 weight scales, one split per token
    if (a.block != 0 || a.scale_enc != 0 || (a.group != 64 && a.group != 128)) return 1;
    if ((long long)a.T * a.K >= (1ll << 31)) return 1;          // 32-bit activation offsets
    for (int i = 0; i < a.count; ++i) {
        if ((long long)a.w[i].M * a.K / 2 >= (1ll << 31)) return 1;
        for (int s = 0; s < a.seg_count; ++s)
            if (a.w[i].seg_split[s] != 1) return 1;
    }
    // Tile choice. Per SIMD the kernel is bound by the FP32 chain of its
    // blocks, so each candidate is scored by the rounds of work-groups it
    // needs over the CUs times the 32x32 blocks per K step its busiest SIMD
    // carries per round (waves on that SIMD x blocks per wave); the small
    // tile pays ~10% for its larger L2 traffic per MAC (measured):
    //   256 x 256, 8 waves (2 per SIMD, 8 blocks each), one work-group per CU;
    //   256 x 160 (G128) / 64 x 160 (G64), 10 waves (3 on the busiest SIMD),
    //     one work-group per CU: fits the grid when the 256-row tile leaves
    //     CUs idle;
    //   128 x 64, 4 waves of 2 blocks, three work-groups per CU.
    // the gemm3_tile option (0..9) picks one configuration (tests, tuning)
    int sel = options().gemm3_tile;
    if (sel < 0) {
        const bool g128 = a.group == 128;
        struct Cand { int sel, bm, bng, wgs, simd_blocks; double penalty; };
        const Cand cands[3] = {
            {0, 256, g128 ? 16 : 8, 1, g128 ? 16 : 8, 1.0},
            {g128 ? 9 : 8, g128 ? 256 : 64, 10, 1, g128 ? 12 : 3, 1.0},
            {g128 ? 3 : 4, 128, 4, 3, 6, 1.1},
        };
        const long long cus = device_cus();
        double best = 0.0;
        for (const Cand &c : cands) {
            long long nt = 0;
            for (int i = 0; i < a.count; ++i) nt += (a.w[i].M / 16 + c.bng - 1) / c.bng;
            const long long tiles = nt * ((a.T + c.bm - 1) / c.bm);
            const long long rounds = (tiles + cus * c.wgs - 1) / (cus * c.wgs);
            const double cost = (double)rounds * c.simd_blocks * c.penalty;
            if (sel < 0 || cost < best) {
                best = cost;
                sel = c.sel;
            }
        }
    }
    if (a.group == 128) {
        switch (sel) {
        case 8: return launch_g3<4, 1, 2, 5, 128, 3, 3>(a, st);   // 256 x 160, 10 waves
        case 9: return launch_g3<4, 1, 2, 5, 128, 2, 3>(a, st);   // 256 x 160, 10 waves, 2 stages
        case 5: return launch_g3<2, 2, 2, 2, 128, 3, 2>(a, st);   // 128 x 128, 4 waves
        case 6: return launch_g3<2, 2, 1, 4, 128, 3, 2>(a, st);   // 64 x 256, 4 waves
        case 7: return launch_g3<1, 2, 2, 2, 128, 3, 3>(a, st);   // 64 x 128, 4 waves, three per CU
        case 1: return launch_g3<4, 2, 1, 4, 128, 2>(a, st);      // 128 x 256, 4 waves, two per CU
        case 2: return launch_g3<4, 2, 2, 4, 128, 2>(a, st);      // 256 x 256, 8 waves, 2 stages
        case 3: return launch_g3<2, 1, 2, 2, 128, 2, 3>(a, st);   // 128 x 64, 4 waves, three per CU
        default: return launch_g3<4, 2, 2, 4, 128, 3>(a, st);     // 256 x 256, 8 waves, 3 stages
        }
    }
    // group 64: two chain updates per block and step
    switch (sel) {
    case 8: return launch_g3<1, 1, 2, 5, 64, 3, 3>(a, st);        // 64 x 160, 10 waves
    case 9: return launch_g3<2, 1, 2, 5, 64, 3, 3>(a, st);        // 128 x 160, 10 waves
    case 5: return launch_g3<2, 2, 2, 2, 64, 2, 2>(a, st);        // 128 x 128, 4 waves
    case 6: return launch_g3<2, 1, 1, 4, 64, 3, 2>(a, st);        // 64 x 128, 4 waves
    case 7: return launch_g3<1, 2, 2, 2, 64, 3, 3>(a, st);        // 64 x 128, 4 waves, three per CU
    case 1: return launch_g3<4, 1, 1, 4, 64, 2>(a, st);           // 128 x 128, 4 waves
    case 2: return launch_g3<2, 2, 2, 4, 64, 2>(a, st);           // 128 x 256, 8 waves
    case 4: return launch_g3<2, 1, 2, 2, 64, 2, 3>(a, st);        // 128 x 64, 4 waves, three per CU
    default: return launch_g3<4, 1, 2, 4, 64, 3>(a, st);          // 256 x 128, 8 waves
    }
}

}  // namespace kxw4
