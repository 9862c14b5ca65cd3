// kxw4_w4a4.hip — the W4A4 GEMM (x_gemm_w4a4, kernels_dpas.cpp:1500-1571):
// s4 activations against K64 weights with FP16|zp scales, one FP32 chain per
// output over the K64 groups u in K order (no split),
//   acc = fma((float)(d_u - zp_u * sum_u), ws_u * as_u, acc),
// on the 32x32x32 int8 MFMA.
//
// Operands. An s4 activation row of one 128-K step (64 bytes) has the nibble
// order of a packed weight tile row: dword i of 16-byte lane group g holds
// k = 32i + 8g + b. The activation unpacks as 16*a (nibble in the high half of
// a byte); the weight unpacks to the bytes w - zp_u, with the group's zero
// point folded in (range [-15, 15]). Each MFMA pair over a K64 group then
// returns 16 (d_u - zp_u sum_u) exactly, and the activation code sums are
// never read. The chain runs on the 16x values — fma(16x, m, 16acc) equals
// 16 fma(x, m, acc) exactly while the chain stays out of FP32's subnormal
// range — and the output is scaled by 1/16.
//
// Cost model: per output and K64 group the chain is one conversion, one
// multiply (ws * as, rounded as the reference rounds it) and one FMA, three
// VALU operations against half a 32-cycle MFMA; the kernel is VALU-bound, and
// each block's chain updates are interleaved with the next block's MFMAs.
// Tile structure, load ring, raster and output staging follow
// kxw4_gemm3.hip: a wave owns 32*TA tokens x 32*TB rows, a work-group
// WMW x WNW waves; per 128-K step the activation tile (XOR-swizzled), the
// packed weight tiles, the FP16|zp scales and the step's two activation
// scales per token reach LDS through direct global->LDS loads into a ring of
// NST stages.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace kxw4 {

constexpr int kW4GroupTT = 4;      // token tiles per raster group

#define KXW4_W4_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// Four int8 bytes w - zp from four nibbles held as w + 8 (the packed dword
// XOR 0x88888888, masked to one nibble per byte); c = (120 - zp) * 0x01010101.
// The byte sums w + 128 - zp stay in [113, 143], so no carry crosses a byte,
// and the XOR turns the excess-128 bytes into two's complement.
__device__ __forceinline__ uint32_t zp_bytes(uint32_t u, uint32_t c) { return (u + c) ^ 0x80808080u; }

__device__ __forceinline__ v4i unpack_k64_zp(uint32_t d0, uint32_t d1, uint32_t c) {
    const uint32_t x0 = d0 ^ 0x88888888u, x1 = d1 ^ 0x88888888u;
    v4i b;
    b.x = (int)zp_bytes(x0 & 0x0F0F0F0Fu, c);
    b.y = (int)zp_bytes((x0 >> 4) & 0x0F0F0F0Fu, c);
    b.z = (int)zp_bytes(x1 & 0x0F0F0F0Fu, c);
    b.w = (int)zp_bytes((x1 >> 4) & 0x0F0F0F0Fu, c);
    return b;
}

template <int TA, int TB, int WMW, int WNW>
struct W4Shape {
    static constexpr int NW = WMW * WNW;
    static constexpr int NTH = 64 * NW;
    static constexpr int UPS = 2;                        // K64 groups per 128-K step
    static constexpr int BM = WMW * 32 * TA;             // tokens per tile
    static constexpr int BNG = WNW * 2 * TB;             // row-groups per tile
    static constexpr int A_BYTES = BM * 64;
    static constexpr int B_BYTES = BNG * kTileBytes;
    static constexpr int S_BYTES = BNG * UPS * 32;       // [row-group][group][16] FP16|zp
    static constexpr int AS_BYTES = UPS * BM * 4;        // [group][token] FP32
    static constexpr int AS_OFF = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int STAGE = (AS_OFF + AS_BYTES + 1023) / 1024 * 1024;
    // loads per wave and stage, equal for every wave; chunk indices wrap when
    // the waves do not divide them (a few chunks are then loaded twice)
    static constexpr int A_CHUNKS = A_BYTES / 1024;
    static constexpr int A_LOADS = (A_CHUNKS + NW - 1) / NW;
    static constexpr int B_LOADS = (BNG + NW - 1) / NW;
    static constexpr int S_TOTAL = BNG * UPS * 2;        // 16-byte scale granules per stage
    static constexpr int s_lanes() {                     // a divisor of S_TOTAL: no range straddles the wrap
        int d = (S_TOTAL + NW - 1) / NW;
        while (S_TOTAL % d) ++d;
        return d;
    }
    static constexpr int S_LANES = s_lanes();
    // 256-byte (one float per lane) wave loads; when the waves outnumber the
    // 64-float rows of the [group][token] block, rows wrap and are loaded by
    // several waves (identical values)
    static constexpr int AS_LOADS = (UPS * BM + 64 * NW - 1) / (64 * NW);
    static constexpr int LOADS = A_LOADS + B_LOADS + 1 + AS_LOADS;
    static constexpr int EPS = 32 * TB + 8;              // output slab token stride (floats)
    static constexpr int slab_bytes(int sb) { return 32 * sb * EPS * 4; }
    template <int NST>
    static constexpr int slab_blocks() {
        return NW * slab_bytes(TA) <= NST * STAGE ? TA
             : (TA % 2 == 0 && NW * slab_bytes(TA / 2) <= NST * STAGE) ? TA / 2 : 1;
    }
    template <int NST>
    static constexpr int lds_bytes() {
        return NST * STAGE > NW * slab_bytes(slab_blocks<NST>()) ? NST * STAGE : NW * slab_bytes(slab_blocks<NST>());
    }
    static_assert(A_BYTES % 1024 == 0, "activation tile in whole 1 KB chunks");
    static_assert(S_LANES <= 64, "one scale load per wave and stage");
    static_assert((UPS * BM) % 64 == 0, "activation scale rows are whole wave loads");
};

template <int TA, int TB, int WMW, int WNW, int NST, int OCC>
__global__ __launch_bounds__(64 * WMW * WNW)
__attribute__((amdgpu_waves_per_eu(OCC, OCC))) void w4a4_kernel(const W4a4Args a) {
    using S = W4Shape<TA, TB, WMW, WNW>;
    constexpr int NW = S::NW, BM = S::BM, BNG = S::BNG, UPS = S::UPS;
    constexpr int A_BYTES = S::A_BYTES, B_BYTES = S::B_BYTES, STAGE = S::STAGE;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // ---- block -> (token tile, n-tile): the work-groups of one XCD
    // (blockIdx % 8) take consecutive tiles, kW4GroupTT token tiles at a time ----
    const int nblk = gridDim.x, id = blockIdx.x;
    const int q8 = nblk / 8, r8 = nblk % 8, xcd = id % 8, j8 = id / 8;
    const int L = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int nnt = a.n_tiles, ntt = a.t_tiles;
    const int group = L / (kW4GroupTT * nnt);
    const int first = group * kW4GroupTT;
    const int gsz = min(ntt - first, kW4GroupTT);
    const int within = L % (kW4GroupTT * nnt);
    const int tt = first + within % gsz;
    const int ntg = within / gsz;
    const int M = a.M, RG = M / 16;
    const int rg0 = ntg * BNG;
    const int t0 = tt * BM;
    const int K = a.K, T = a.T, NT = K / kTileK, G = K / 64;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;

    // ---- load issue: per-lane 32-bit source offsets that do not depend on
    // the K step (the launcher keeps T*64, M*K/2 and (K/64)*T below 2^31) ----
    uint32_t aoffs[S::A_LOADS];
#pragma unroll
    for (int i = 0; i < S::A_LOADS; ++i) {
        const int p = ((wave + NW * i) % S::A_CHUNKS) * 64 + lane;   // 16-byte granule this lane fills
        const int t = p >> 2;                                 // token of the tile
        const int c = (p & 3) ^ ((t >> 2) & 3);               // source chunk stored at slot p & 3
        aoffs[i] = (uint32_t)min(t0 + t, T - 1) * 64 + c * 16;   // rows past T: never stored
    }
    uint32_t boffs[S::B_LOADS];
#pragma unroll
    for (int i = 0; i < S::B_LOADS; ++i) {
        const int rg = min(rg0 + (wave + NW * i) % BNG, RG - 1);   // row-groups past M: never stored
        boffs[i] = (uint32_t)rg * NT * kTileBytes + lane * 16;
    }
    uint32_t soff;
    {
        const int gi = (wave * S::S_LANES + min(lane, S::S_LANES - 1)) % S::S_TOTAL;
        const int j = gi / (2 * UPS), u = (gi >> 1) % UPS, half = gi & 1;
        const int rg = min(rg0 + j, RG - 1);
        soff = ((uint32_t)rg * G + u) * 16 + half * 8;
    }
    uint32_t asoffs[S::AS_LOADS];
#pragma unroll
    for (int i = 0; i < S::AS_LOADS; ++i) {
        const int p = ((wave + NW * i) * 64) % (UPS * BM) + lane;   // float of the [group][token] block
        asoffs[i] = (uint32_t)(p / BM) * T + min(t0 + p % BM, T - 1);
    }
    auto issue = [&](int kb, int st) {
        uint8_t *base = smem + st * STAGE;
        const uint8_t *ak = a.q4 + (size_t)kb * T * 64;
        const uint8_t *wk = a.codes + (size_t)kb * kTileBytes;
        const float *sk = a.as4 + (size_t)kb * UPS * T;
#pragma unroll
        for (int i = 0; i < S::A_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(ak + aoffs[i]),
                                             KXW4_W4_LDS(base + ((wave + NW * i) % S::A_CHUNKS) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < S::B_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(wk + boffs[i]),
                                             KXW4_W4_LDS(base + A_BYTES + ((wave + NW * i) % BNG) * 1024), 16, 0, 0);
        // lanes past the wave's granules are masked off; the load still
        // counts once in vmcnt
        if (lane < S::S_LANES)
            __builtin_amdgcn_global_load_lds((const void *)(a.scales + (size_t)kb * UPS * 16 + soff),
                                             KXW4_W4_LDS(base + A_BYTES + B_BYTES + (wave * S::S_LANES) % S::S_TOTAL * 16),
                                             16, 0, 0);
#pragma unroll
        for (int i = 0; i < S::AS_LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(sk + asoffs[i]),
                                             KXW4_W4_LDS(base + S::AS_OFF + ((wave + NW * i) * 64) % (UPS * BM) * 4),
                                             4, 0, 0);
    };

    // ---- per-lane read offsets (lane = row/column l%32, K group l/32) ----
    const int m32 = lane & 31, kg = lane >> 5;
    const int tw = wm * 32 * TA;                               // first token of this wave in the tile
    const int hx = (m32 >> 2) & 3;                             // swizzle of this lane's rows
    const int arow = (tw + m32) * 64;
    const int aoff0 = arow + ((kg ^ hx) << 4);                 // lane group kg: MFMAs 0 and 1
    const int aoff1 = arow + (((kg + 2) ^ hx) << 4);           // lane group kg + 2: MFMAs 2 and 3
    const int jrel0 = wn * 2 * TB + (m32 >> 4);
    const int boff = A_BYTES + jrel0 * kTileBytes + (kg * 16 + (m32 & 15)) * 16;
    const int soff_lds = A_BYTES + B_BYTES + (jrel0 * UPS * 16 + (m32 & 15)) * 2;
    const int asoff_lds = S::AS_OFF + (tw + 4 * kg) * 4;

    float f[TA][TB][16];
#pragma unroll
    for (int i = 0; i < TA; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) f[i][j][r] = 0.0f;

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
        // weight operands of the step with the group zero points folded in;
        // MFMA c = 2h + u covers lane group kg + 2h and K64 group u
        v4i B[TB][4];
        float w[TB][UPS];
#pragma unroll
        for (int jb = 0; jb < TB; ++jb) {
            uint32_t zc[UPS];
#pragma unroll
            for (int u = 0; u < UPS; ++u) {
                const uint32_t p = *reinterpret_cast<const uint16_t *>(sb + soff_lds + (jb * 2 * UPS + u) * 32);
                w[jb][u] = half_bits_to_float((uint16_t)(p & 0xFFF0u));
                zc[u] = (uint32_t)(120 - sext4(p)) * 0x01010101u;
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const v4u wd = *reinterpret_cast<const v4u *>(sb + boff + jb * 2 * kTileBytes + h * 512);
                B[jb][2 * h] = unpack_k64_zp(wd.x, wd.y, zc[0]);
                B[jb][2 * h + 1] = unpack_k64_zp(wd.z, wd.w, zc[1]);
            }
        }
        // activation operands of token block ib (16*a), and the activation
        // scales of its tokens: register r of a block is token
        // 8(r/4) + 4kg + r%4, so four 16-byte reads per group
        auto load_a = [&](int ib, v4u &lo, v4u &hi) {
            lo = *reinterpret_cast<const v4u *>(sb + aoff0 + ib * 2048);
            hi = *reinterpret_cast<const v4u *>(sb + aoff1 + ib * 2048);
        };
        auto unpack_a = [&](const v4u &lo, const v4u &hi, v4i (&A)[4]) {
            A[0] = unpack_k64(lo.x, lo.y);
            A[1] = unpack_k64(lo.z, lo.w);
            A[2] = unpack_k64(hi.x, hi.y);
            A[3] = unpack_k64(hi.z, hi.w);
        };
        float asv[UPS][16];
        auto load_as = [&](int ib) {
#pragma unroll
            for (int u = 0; u < UPS; ++u)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = *reinterpret_cast<const float4 *>(sb + asoff_lds + (u * BM + 32 * ib + 8 * q) * 4);
                    asv[u][4 * q] = v.x;
                    asv[u][4 * q + 1] = v.y;
                    asv[u][4 * q + 2] = v.z;
                    asv[u][4 * q + 3] = v.w;
                }
        };
        constexpr int NB = TA * TB;
        v4i Acur[4], Anext[4];
        v4u an_lo, an_hi;
        {
            v4u lo, hi;
            load_a(0, lo, hi);
            unpack_a(lo, hi, Acur);
        }
        load_as(0);
        v16i acc[2][UPS];
        const v16i zero = {};
        auto update = [&](int b) {
            const int ib = b / TB, jb = b % TB;
#pragma unroll
            for (int u = 0; u < UPS; ++u) {
                const v16i &p = acc[b & 1][u];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    f[ib][jb][r] = __builtin_fmaf((float)p[r], w[jb][u] * asv[u][r], f[ib][jb][r]);
            }
        };
        // Software pipeline over the step's blocks (row block jb fastest):
        // stage b issues block b's MFMAs interleaved with block b-1's chain
        // updates; the next token block's operands are read at the start of
        // the stage before it and unpacked at its end, and the activation
        // scales of a token block are read once its predecessor's last
        // update has been issued.
#pragma unroll
        for (int b = 0; b <= NB; ++b) {
            const int ib = b / TB, jb = b % TB;
            const bool next_a = b < NB && jb == TB - 1 && ib + 1 < TA;
            if (b < NB) {
                if (jb == 0 && ib > 0) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) Acur[c] = Anext[c];
                }
                if (next_a) load_a(ib + 1, an_lo, an_hi);
                v16i &p0 = acc[b & 1][0];
                v16i &p1 = acc[b & 1][1];
                p0 = mfma32(Acur[0], B[jb][0], zero);
                p1 = mfma32(Acur[1], B[jb][1], zero);
                p0 = mfma32(Acur[2], B[jb][2], p0);
                p1 = mfma32(Acur[3], B[jb][3], p1);
            }
            if (b > 0) update(b - 1);
            if (b > 0 && b < NB) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 24, 0);
                }
            }
            if (next_a) unpack_a(an_lo, an_hi, Anext);
            if (b > 0 && b < NB && jb == 0) load_as(ib);
            __builtin_amdgcn_sched_barrier(0);
        }
        st = st == NST - 1 ? 0 : st + 1;
    }

    // ---- output: staged per wave in LDS, written as 16-byte row runs ----
    constexpr int EPS = S::EPS, SB = S::template slab_blocks<NST>();
    static_assert(TA % SB == 0, "slabs cover the wave tile");
    static_assert(S::template lds_bytes<NST>() <= 160 * 1024, "LDS");
    lds_sync();
    float *slab = reinterpret_cast<float *>(smem) + wave * (32 * SB * EPS);
#pragma unroll
    for (int s0 = 0; s0 < TA; s0 += SB) {
#pragma unroll
        for (int ib = s0; ib < s0 + SB; ++ib)
#pragma unroll
            for (int jb = 0; jb < TB; ++jb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    slab[(32 * (ib - s0) + 8 * (r >> 2) + 4 * kg + (r & 3)) * EPS + 32 * jb + m32] = f[ib][jb][r];
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
                float v[CH];
#pragma unroll
                for (int e = 0; e < CH; e += 4) {
                    const float4 x = *reinterpret_cast<const float4 *>(slab + tl * EPS + rl + e);
                    v[e] = x.x * 0.0625f;
                    v[e + 1] = x.y * 0.0625f;
                    v[e + 2] = x.z * 0.0625f;
                    v[e + 3] = x.w * 0.0625f;
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
                    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.y) + (size_t)t * M + row) = o;
                } else {
                    *reinterpret_cast<float4 *>(static_cast<float *>(a.y) + (size_t)t * M + row) =
                        make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        };
        if (a.y_bf16) run(std::integral_constant<int, 8>{});
        else run(std::integral_constant<int, 4>{});
    }
}

template <int TA, int TB, int WMW, int WNW, int NST, int OCC>
static int launch_w4(W4a4Args &a, hipStream_t st) {
    using S = W4Shape<TA, TB, WMW, WNW>;
    a.n_tiles = (a.M / 16 + S::BNG - 1) / S::BNG;
    a.t_tiles = (a.T + S::BM - 1) / S::BM;
    const dim3 grid(a.n_tiles * a.t_tiles), block(S::NTH);
    auto k = w4a4_kernel<TA, TB, WMW, WNW, NST, OCC>;
    const size_t lds = (size_t)S::template lds_bytes<NST>();
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

int launch_w4a4(W4a4Args &a, hipStream_t st) {
    // Default 128 x 64 (three work-groups per CU); when that grid gives fewer
    // than two work-groups per CU, 64 x 64 (twice the work-groups, more waves
    // per SIMD to overlap one wave's chain with another's MFMAs: cfg2 M=512
    // 196 -> 184 us). The 64 x 160 tile (10 waves, one work-group per CU)
    // balances the cfg2 M=512 grid but measures slower (207 us): with one
    // token block per wave the zero-point weight unpack is no longer shared.
    // the w4a4_tile option (0..4) picks one configuration (tests, tuning)
    int sel = options().w4a4_tile;
    if (sel < 0) {
        const long long tiles = (long long)((a.T + 127) / 128) * ((a.M / 16 + 3) / 4);
        sel = tiles < 2LL * device_cus() ? 4 : 0;
    }
    switch (sel) {
    case 3: return launch_w4<1, 1, 2, 5, 3, 3>(a, st);      // 64 tokens x 160 rows, 10 waves
    case 1: return launch_w4<2, 1, 2, 4, 3, 2>(a, st);      // 128 tokens x 128 rows, 8 waves
    case 2: return launch_w4<1, 2, 2, 2, 3, 2>(a, st);      // 64 tokens x 128 rows, 4 waves
    case 4: return launch_w4<1, 1, 2, 2, 3, 3>(a, st);      // 64 tokens x 64 rows, 4 waves
    default: return launch_w4<2, 1, 2, 2, 3, 2>(a, st);     // 128 tokens x 64 rows, 4 waves
    }
}

}  // namespace kxw4
