// kxw4_rowwave.hip — decode-shaped projections for up to 16 tokens with one
// split plan for all tokens of a weight: the GEMV (kernels_dpas.cpp:586-675),
// the fan-out GEMV (945-1102) and the batched GEMM at small T (1334-1490).
//
// Each wave owns one (row-group, split). It streams the split's 1 KB weight
// tiles through a ring of PF loads in flight and runs the split's reference
// chain in registers: the int8 MFMA leaves row n of tokens 4*(l/16)+r in
// register r of lane l for every unit, so a lane's four accumulators are four
// of the reference's chains, fed unit by unit in order. The waves of one
// row-group take consecutive splits (a work-group holds one or more
// row-groups of min(S, 8) waves each, at most 16 waves); with S > 1 the split
// partials meet in LDS and one wave adds them in split order starting from
// 0.0f.
//
// The activations (T x K int8) and the work-group's FP16 scales are staged
// into LDS once per work-group with direct global->LDS loads, so the
// weight-tile load is the only vector-memory instruction of the streaming
// loop. Activation rows are padded by 16 bytes, so the 8 or 16 token rows a
// 16-lane quarter reads fall on distinct banks, and every LDS address in the
// loop is a per-ring base plus an immediate offset. Whole rings run without
// predicates; only a split's last, partial ring selects the old accumulator
// for its padded positions.
//
// W8 (the W8A8 tier, x_gemv_w8a8_core / x_gemm_w8a8, kernels_dpas.cpp:
// 771-844, 1578-1629): 2 KB int8 tiles, two 16-byte loads per lane and tile,
// used as the K32 MFMA operand without an unpack; the MFMA result is the unit
// partial itself (no factor 16) and the chain is the reference mode's with
// zero point 0. The per-K32 scales are not staged (they would take 5 KB of
// LDS per row-group): one 2-byte load per lane and tile rides in the ring,
// and four lane shuffles hand each lane its row's four unit scales.
//
// K16 (the K16 tier, x_gemv_w4a8_core_k16, kernels_dpas.cpp:683-760): GEMV
// only, FP16|zp scales per K16 half. A K32 unit's lane groups 0-1 hold half 0
// and 2-3 half 1, so two MFMAs with the other half's lanes zeroed give the two
// half partials; each lane's zero point is folded into its weight bytes
// (w - zp, so no activation sums are needed and the partials carry no factor
// 16); one serial accumulator per split, which covers whole K32 tiles.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace kxw4 {

// wave budget of a plain work-group (wpw / wrg row-groups): 10 measured best
// at the cfg1 shape (5 row-groups of 2 splits: 20.7 us against 23.2 us at 8
// waves and 21.3 us for the balanced plan)
constexpr int kRwWaves = 10;
constexpr int kRwSplitWaves = 8;            // most waves that share one row-group's splits
constexpr int kRwMaxWaves = 16;
// K16 work-groups stay at 8 waves, so the kernel may keep 256 registers per
// lane (its two masked half MFMAs and scale folds per unit spill at 128)
constexpr int kRwK16Waves = 8;
constexpr size_t kRwLdsMax = 160 * 1024;
// weight tiles in flight per wave (a deeper ring measured slower: its loads
// at the start delay the activation staging)
constexpr int kRwRing = 4;

enum { kWfW4 = 0, kWfW8 = 1, kWfK16 = 2 };     // weight format of a row-wave instance

template <int TT, int UNIT, int MODE, bool ALT2, int PF, int WF>
__global__ __launch_bounds__(64 * (WF == kWfK16 ? kRwK16Waves : kRwMaxWaves)) void rowwave_kernel(const DecodeArgs a) {
    constexpr int UPS = kTileK / UNIT;
    constexpr bool W8 = WF == kWfW8, K16 = WF == kWfK16;
    static_assert(WF == kWfW4 || (UNIT == 32 && MODE == 1), "W8 / K16: K32 units, reference mode");
    static_assert(!K16 || ALT2, "K16 is a GEMV");
    constexpr int TB = W8 ? 2 : 1;                 // 16-byte loads per lane and tile
    constexpr float kInv16 = WF != kWfW4 ? 1.0f : 0.0625f;  // undoes the nibble unpack's factor 16
    static_assert(PF % 2 == 0, "the GEMV accumulator parity assumes an even ring");
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if ((int)blockIdx.x >= a.w[i].wg_begin) wi = i;
    const DecodeWeight &W = a.w[wi];
    // the work-group's waves: rows of wrg waves, one per row-group; R is the
    // most row-groups a work-group of this weight owns (the LDS sizes
    // follow it)
    const int nthreads = blockDim.x;
    const int S = W.seg_split[0], wrg = W.wrg;
    const int R = (W.M / 16 + W.wg_count - 1) / W.wg_count;
    const int K = a.K, T = a.T, M = W.M;
    const int NT = K / kTileK, Nu = K / UNIT, G = K / a.group;
    const int gsh = a.group >= UNIT ? __builtin_ctz(a.group / UNIT) : 0;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, n = lane & 15, g4 = lane >> 4;
    const int rgl = wave / wrg, wj = wave - rgl * wrg;
    // row-groups [rg0, rg0 + nrg) of the weight: the weight's wg_count
    // work-groups split its row-groups as evenly as possible
    const int bl = (int)blockIdx.x - W.wg_begin, RGw = M / 16;
    const int rg0 = bl * RGw / W.wg_count;
    const int nrg = (bl + 1) * RGw / W.wg_count - rg0;
    const bool active = rgl < nrg;
    const int rg = rg0 + (active ? rgl : 0);

    const int pitch = K + 16;                                 // padded activation row
    int8_t *Act = reinterpret_cast<int8_t *>(smem);
    uint16_t *Sc = reinterpret_cast<uint16_t *>(smem + (size_t)T * pitch);
    // the zero-point code-sum table exists only for FP16|zp W4 weights (W8
    // has no zero points and K16 folds them into the weight bytes), so the
    // other formats ask for less LDS
    const bool zp = WF == kWfW4 && a.scale_enc == 1;
    // W8 scales are not staged: they stream through the ring (below)
    float *Asc = reinterpret_cast<float *>(Sc + (W8 ? 0 : R * G * 16));
    int *Zs = reinterpret_cast<int *>(Asc + (MODE != 0 ? Nu * 16 : 0));
    float *Part = reinterpret_cast<float *>(Zs + (MODE != 0 && zp ? Nu * 16 : 0));
    // 16 zero words: the scale (and activation scale) read of a padded
    // position, so its chain step fma(p, 0, acc) leaves acc unchanged
    // (p is a finite integer and a chain that starts at +0 never holds -0)
    float *Zero = Part + (S > 1 ? R * (S - 1) * 256 : 0);

    // ---- stage activations and scales with direct global->LDS loads ----
    // LDS chunk x (16 bytes) is chunk x % (kc+1) of activation row x / (kc+1)
    // (the last chunk of a row is padding), then the work-group's scales.
    const int kc = K / 16;
    const int act_chunks = T * (kc + 1);
    const int total = act_chunks + (W8 ? 0 : nrg * G * 2);
    for (int c0 = wave * 64; c0 < total; c0 += nthreads) {
        const int x = c0 + lane;
        if (x < total) {
            const void *src;
            if (x < act_chunks) {
                const int t = x / (kc + 1), p = x - t * (kc + 1);
                src = a.q + (size_t)t * K + 16 * min(p, kc - 1);
            } else {
                src = W.scales + (size_t)rg0 * G * 16 + (size_t)(x - act_chunks) * 8;
            }
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(smem + (size_t)c0 * 16),
                                             16, 0, 0);
        }
    }

    // per-token mode: this lane's four token scales for the output, loaded
    // now (before the ring, so the staging wait below covers them) rather
    // than after the split sum, where they would add a memory round trip
    // (cfg1: 22.1 -> 21.2 us)
    float tsc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (a.block == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) tsc[r] = a.ascale[min(4 * g4 + r, T - 1)];
    }
    // likewise the residual of this lane's four outputs
    float rsd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.residual) {
#pragma unroll
        for (int r = 0; r < 4; ++r) rsd[r] = a.residual[(size_t)min(4 * g4 + r, T - 1) * M + rg * 16 + n];
    }

    // ---- the wave's first split and its ring ----
    const int sb = wj * S / wrg, se = (wj + 1) * S / wrg;
    // split ranges [Nu*s/S, Nu*(s+1)/S); S is a power of two (checked by
    // the launcher) and Nu*S fits in 32 bits
    const int ls = __builtin_ctz(S);
    int u0 = (Nu * sb) >> ls, u1 = (Nu * (sb + 1)) >> ls;
    int kt0 = u0 / UPS, ntw = (u1 + UPS - 1) / UPS - kt0;
    const v4u *wrow = reinterpret_cast<const v4u *>(W.codes + (size_t)rg * NT * kTileBytes * TB) + lane;
    v4u ring[PF][TB];
    // W8: the tile's FP16 scales ride in the ring, one per lane: lane n+16j
    // holds unit j's scale of row n (the tile's 128 bytes of the [rg][G][16]
    // table); the chain spreads them to the row's lanes with shuffles
    uint32_t sring[W8 ? PF : 1];
    const uint16_t *wsc = W.scales + ((size_t)rg * G + g4) * 16 + n;
    // tile i of the current split; an empty split (more splits than units)
    // or an idle wave reads a valid tile it never uses
    auto load = [&](int i, int p) {
        const int kt = min(kt0 + max(i, 0), NT - 1);
        const size_t t = (size_t)kt * (kTileBytes * TB / 16);
#pragma unroll
        for (int h = 0; h < TB; ++h) ring[p][h] = wrow[t + 64 * h];
        if constexpr (W8) sring[p] = wsc[(size_t)kt * (kTileK / 32) * 16];
    };
    constexpr int LPT = TB + (W8 ? 1 : 0);         // loads per tile
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PF; ++p) load(min(p, ntw - 1), p);
    __builtin_amdgcn_sched_barrier(0);
    // the staging loads were issued before the PF ring loads and complete first
    KXW4_WAIT_VMCNT(PF * LPT);
    const bool ref_block = a.block == 32;
    if (MODE != 0 && UNIT == 32 && ref_block) {
        // per-unit (= per-K32) activation scale and zero-point code sum,
        // [Nu][16 token slots]; each thread reads four consecutive units of
        // one token row with one 16-byte load (rows are K/32 entries, a
        // multiple of 4) and scatters them into the token-minor table
        const int n4 = Nu / 4;
        for (int x = tid; x < 16 * n4; x += nthreads) {
            const int slot = x / n4, u = 4 * (x - slot * n4);
            const size_t src = (size_t)min(slot, T - 1) * Nu + u;
            const float4 sc = *reinterpret_cast<const float4 *>(a.ascale + src);
            Asc[u * 16 + slot] = sc.x;
            Asc[(u + 1) * 16 + slot] = sc.y;
            Asc[(u + 2) * 16 + slot] = sc.z;
            Asc[(u + 3) * 16 + slot] = sc.w;
            if (zp) {
                const int4 sm = *reinterpret_cast<const int4 *>(a.asum + src);
                Zs[u * 16 + slot] = sm.x;
                Zs[(u + 1) * 16 + slot] = sm.y;
                Zs[(u + 2) * 16 + slot] = sm.z;
                Zs[(u + 3) * 16 + slot] = sm.w;
            }
        }
    } else if (MODE != 0) {
        // per-unit activation scale and zero-point code sum, [Nu][16 tokens]
        for (int x = tid; x < Nu * 16; x += nthreads) {
            const int u = x >> 4, t = min(x & 15, T - 1);
            Asc[x] = ref_block ? a.ascale[(size_t)t * (K / 32) + u] : 1.0f;
            if (zp) {
                int sm = 0;
                for (int q = (u * UNIT) / 32; q < ((u + 1) * UNIT) / 32; ++q)
                    sm += a.asum[(size_t)t * (K / 32) + q];
                Zs[x] = sm;
            }
        }
    }
    if (tid < 16) Zero[tid] = 0.0f;
    lds_sync_after_dma();

    // ---- streaming: one chain per split, in registers ----
    const bool gemm_var = a.variant == kVarGemm;
    // this lane's activation row (MFMA row n; with up to 8 tokens rows 8-15
    // repeat rows 0-7 and are never stored) and its K-slot group
    const int ta = TT == 8 ? min(n & 7, T - 1) : min(n, T - 1);
    const int8_t *abase = Act + (size_t)ta * pitch + 16 * g4;
    const uint16_t *sbase = Sc + rgl * G * 16 + n;
    float res[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    if (active) {
        for (int s = sb; s < se; ++s) {
            if (s != sb) {
                u0 = (Nu * s) >> ls;
                u1 = (Nu * (s + 1)) >> ls;
                kt0 = u0 / UPS;
                ntw = (u1 + UPS - 1) / UPS - kt0;
#pragma unroll
                for (int p = 0; p < PF; ++p) load(min(p, ntw - 1), p);
            }
            float f0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, f1[4] = {0.0f, 0.0f, 0.0f, 0.0f};

            // One ring of PF tiles starting at tile ib of the split. PRED
            // marks the rings that may hold padded positions or units outside
            // the split.
            auto ring_pass = [&](int ib, auto pred) {
                constexpr bool PRED = decltype(pred)::value;
                const int8_t *ar = abase + (size_t)(kt0 + ib) * kTileK;
                const uint16_t *sr = sbase + (MODE == 0 ? (size_t)(kt0 + ib) * UPS * 16 : 0);
#pragma unroll
                for (int p = 0; p < PF; ++p) {
                    const int i = ib + p;
                    const int kb = kt0 + i;
                    const v4i A0 = *reinterpret_cast<const v4i *>(ar + p * kTileK);
                    const v4i A1 = *reinterpret_cast<const v4i *>(ar + p * kTileK + 64);
                    const v4u wd = ring[p][0];
                    // W8: unit j's scale of this lane's row, from lane n + 16j
                    uint32_t s8[W8 ? 4 : 1];
                    if constexpr (W8) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) s8[j] = (uint32_t)__shfl((int)sring[p], n + 16 * j);
                    }
#pragma unroll
                    for (int j = 0; j < UPS; ++j) {
                        const int u = kb * UPS + j;
                        const bool in = !PRED || (i < ntw && (UNIT == 128 || (u >= u0 && u < u1)));
                        const v4i zero = {0, 0, 0, 0};
                        v4i acc;
                        if constexpr (UNIT == 128) {
                            acc = mfma_k64(A0, unpack_k64(wd.x, wd.y), zero);
                            acc = mfma_k64(A1, unpack_k64(wd.z, wd.w), acc);
                        } else if constexpr (UNIT == 64) {
                            acc = j == 0 ? mfma_k64(A0, unpack_k64(wd.x, wd.y), zero)
                                         : mfma_k64(A1, unpack_k64(wd.z, wd.w), zero);
                        } else {
                            const v4i c = j < 2 ? A0 : A1;
                            const long av = (j & 1) ? (long)(((uint64_t)(uint32_t)c.w << 32) | (uint32_t)c.z)
                                                    : (long)(((uint64_t)(uint32_t)c.y << 32) | (uint32_t)c.x);
                            long bv;
                            if constexpr (K16) {
                                // the unit's two K16 scale words; lane groups
                                // 0-1 carry half 0, 2-3 half 1
                                const uint32_t s0 = *(in ? &sbase[(2 * u) * 16] : reinterpret_cast<const uint16_t *>(Zero) + n);
                                const uint32_t s1 = *(in ? &sbase[(2 * u + 1) * 16] : reinterpret_cast<const uint16_t *>(Zero) + n);
                                const uint32_t x = (j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w) ^ 0x88888888u;
                                const uint32_t cz = (uint32_t)(120 - sext4(g4 < 2 ? s0 : s1)) * 0x01010101u;
                                const uint64_t lo = ((x & 0x0F0F0F0Fu) + cz) ^ 0x80808080u;
                                const uint64_t hi = (((x >> 4) & 0x0F0F0F0Fu) + cz) ^ 0x80808080u;
                                bv = (long)(lo | (hi << 32));
                                const v4i ph[2] = {mfma_k32(av, g4 < 2 ? bv : 0l, zero), mfma_k32(av, g4 < 2 ? 0l : bv, zero)};
                                const float4 asv = *reinterpret_cast<const float4 *>(in ? Asc + u * 16 + 4 * g4 : Zero + 4 * g4);
                                const float avr[4] = {asv.x, asv.y, asv.z, asv.w};
#pragma unroll
                                for (int h = 0; h < 2; ++h) {
                                    const float w = half_bits_to_float((uint16_t)((h ? s1 : s0) & 0xFFF0u));
#pragma unroll
                                    for (int r = 0; r < 4; ++r) f0[r] = __builtin_fmaf((float)ph[h][r] * w, avr[r], f0[r]);
                                }
                                continue;
                            } else if constexpr (W8) {
                                const v4u h = ring[p][j >> 1];
                                bv = (j & 1) ? (long)(((uint64_t)h.w << 32) | h.z)
                                             : (long)(((uint64_t)h.y << 32) | h.x);
                            } else {
                                bv = unpack_k32(j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w);
                            }
                            acc = mfma_k32(av, bv, zero);
                        }
                        // MODE 0 has unit == group, so unit u reads scale u
                        const uint16_t *sp = MODE == 0 ? &sr[(p * UPS + j) * 16] : &sbase[(u >> gsh) * 16];
                        uint32_t sv;
                        if constexpr (W8) sv = in ? s8[W8 ? j : 0] : 0u;
                        else sv = *(in ? sp : reinterpret_cast<const uint16_t *>(Zero) + n);
                        // GEMV: units at odd offsets from the split start feed the
                        // second accumulator. With an even ring and an even number
                        // of units per tile the parity is fixed by p (whole-tile
                        // units) or j; when the split starts on an odd unit the two
                        // accumulators trade roles, and their final sum commutes.
                        float *F = (ALT2 && (UNIT == 128 ? (p & 1) : (j & 1))) ? f1 : f0;
                        if constexpr (MODE == 0) {
                            const float w = half_bits_to_float((uint16_t)sv);
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float nf = __builtin_fmaf((float)acc[r], w, F[r]);
                                F[r] = nf;
                            }
                        } else {
                            const float w = half_bits_to_float(zp ? (uint16_t)(sv & 0xFFF0u) : (uint16_t)sv);
                            const int z = sext4(sv);
                            v4i zv = {0, 0, 0, 0};
                            if (WF == kWfW4)
                                zv = *reinterpret_cast<const v4i *>(zp ? Zs + u * 16 + 4 * g4
                                                                       : reinterpret_cast<const int *>(Zero) + 4 * g4);
                            const float4 av = *reinterpret_cast<const float4 *>(in ? Asc + u * 16 + 4 * g4 : Zero + 4 * g4);
                            const float avr[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                int pv = acc[r];
                                if (zp) pv -= (z * zv[r]) << 4;
                                const float pf = (float)pv;
                                float nf;
                                if (!ref_block) nf = __builtin_fmaf(pf, w, F[r]);
                                else if (gemm_var) nf = __builtin_fmaf(pf, w * avr[r], F[r]);
                                else nf = __builtin_fmaf(pf * w, avr[r], F[r]);
                                F[r] = nf;
                            }
                        }
                    }
                    load(min(i + PF, ntw - 1), p);
                    // keep each slot's unpack behind the previous slot's load, so
                    // the wait before it covers only that slot
                    __builtin_amdgcn_sched_barrier(0);
                }
            };

            // whole rings run unpredicated when the split starts and ends on
            // tile boundaries; the rest (at most one ring then) is predicated
            const bool aligned = u0 % UPS == 0 && u1 % UPS == 0;
            int ib = 0;
            if (aligned)
                for (; ib + PF <= ntw; ib += PF) ring_pass(ib, std::false_type{});
            for (; ib < ntw; ib += PF) ring_pass(ib, std::true_type{});
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = (ALT2 && !K16) ? f0[r] + f1[r] : f0[r];
                // split 0 stays in the registers of the wave that adds the splits
                if (S > 1 && s > 0) Part[((rgl * (S - 1) + s - 1) * 4 + r) * 64 + lane] = v;
                else res[r] = v;
            }
        }
    }

    // ---- ordered split sum and output ----
    if (S > 1) {
        lds_sync();
        if (!active || wj != 0) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float sum = 0.0f + res[r];
            for (int s = 1; s < S; ++s) sum = sum + Part[((rgl * (S - 1) + s - 1) * 4 + r) * 64 + lane];
            res[r] = sum;
        }
    } else if (!active) {
        return;
    }
    const int row = rg * 16 + n;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int t = 4 * g4 + r;
        if (t >= T) continue;
        const float v = a.block == 0 ? res[r] * (tsc[r] * kInv16) : res[r] * kInv16;
        float out;
        if (a.residual) out = v + rsd[r];
        else if (ALT2 && S > 1) out = v + 0.0f;
        else out = v;
        if (a.y_bf16) static_cast<uint16_t *>(W.y)[(size_t)t * M + row] = float_to_bf16(out);
        else static_cast<float *>(W.y)[(size_t)t * M + row] = out;
    }
}

template <int TT, int UNIT, int MODE, bool ALT2, int PF, int WF = kWfW4>
static int rw_launch(const DecodeArgs &a, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    auto k = rowwave_kernel<TT, UNIT, MODE, ALT2, PF, WF>;
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kRwLdsMax) != hipSuccess)
            return -6;
        attr = true;
    }
    hipLaunchKernelGGL(k, grid, block, lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

template <int TT, int UNIT>
static int rw_mode(const DecodeArgs &a, int mode, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    const bool alt2 = a.variant == kVarGemv;
    if (mode == 0)
        return alt2 ? rw_launch<TT, UNIT, 0, true, kRwRing>(a, grid, block, lds, st)
                    : rw_launch<TT, UNIT, 0, false, kRwRing>(a, grid, block, lds, st);
    return alt2 ? rw_launch<TT, UNIT, 1, true, kRwRing>(a, grid, block, lds, st)
                : rw_launch<TT, UNIT, 1, false, kRwRing>(a, grid, block, lds, st);
}

template <int TT>
static int rw_unit(const DecodeArgs &a, int unit, int mode, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    if (unit == 128) return rw_mode<TT, 128>(a, mode, grid, block, lds, st);
    if (unit == 64) return rw_mode<TT, 64>(a, mode, grid, block, lds, st);
    return rw_mode<TT, 32>(a, mode, grid, block, lds, st);
}

int launch_rowwave(DecodeArgs &a, hipStream_t st) {
    if (a.T < 1 || a.T > 16) return 1;
    const int unit = a.block == 32 ? 32 : a.group;
    const int nu = a.K / unit, g = a.K / a.group;
    const int mode = (a.block == 0 && a.scale_enc == 0) ? 0 : 1;
    // Plain shape: a budget of kRwWaves waves per work-group, wpw / wrg
    // row-groups each. When the LDS holds only one such work-group per CU
    // (large tables: 16 token rows, long K), the CU's only memory parallelism
    // is that work-group, so it takes 16 waves instead; so do weights that
    // need four or more rounds of work-groups per CU (lm_head-sized), where
    // fewer, larger work-groups stage the activations fewer times (W8A8
    // lm_head T=8: 311 -> 271 us). Otherwise, when the plain shape leaves a
    // partial last round of work-groups over the CUs (the CUs holding one
    // more work-group finish last), the weights' row-groups are instead
    // dealt to exactly k work-groups per CU, each owning ceil(row-groups /
    // work-groups) row-groups at most, and the LDS request keeps a (k+1)-th
    // work-group off every CU; that plan is kept only when it lowers the
    // most row-groups a CU streams.
    int rg_total = 0, wrg_max = 1;
    for (int i = 0; i < a.count; ++i) {
        DecodeWeight &w = a.w[i];
        const int S = w.seg_split[0];
        for (int s = 1; s < a.seg_count; ++s)
            if (w.seg_split[s] != S) return 1;
        if (S < 1 || S > 16 || (S & (S - 1))) return 1;
        w.wrg = std::min(S, kRwSplitWaves);
        wrg_max = std::max(wrg_max, w.wrg);
        rg_total += w.M / 16;
    }
    const int cus = device_cus();
    // option rowwave_rpw = r: r row-groups per work-group (r * min(S, 8) waves)
    const int rpw = options().rowwave_rpw;
    const int max_waves = a.group == 16 ? kRwK16Waves : kRwMaxWaves;
    if (rpw < 0 || rpw * wrg_max > max_waves) return 1;
    int wpw = rpw ? rpw * wrg_max : std::min(kRwWaves, max_waves);
    int wg = 0, waves = 0, rmax = 1, part = 0;
    // k > 0: k work-groups per CU over all weights; k = 0: the plain shape
    auto plan = [&](int k) {
        wg = 0;
        waves = 0;
        rmax = 1;
        part = 0;
        for (int i = 0; i < a.count; ++i) {
            DecodeWeight &w = a.w[i];
            const int RG = w.M / 16, S = w.seg_split[0];
            const int per = std::max(1, wpw / w.wrg);
            int n = k ? (int)(((long long)k * cus * RG + rg_total / 2) / rg_total) : (RG + per - 1) / per;
            n = std::max(1, std::min(n, RG));
            const int R = (RG + n - 1) / n;
            w.wg_begin = wg;
            w.wg_count = n;
            wg += n;
            rmax = std::max(rmax, R);
            waves = std::max(waves, (k ? R : per) * w.wrg);
            if (S > 1) part = std::max(part, R * (S - 1));
        }
    };
    // the work-group's LDS: padded activation rows, its row-groups' scales,
    // the per-unit activation scales and, for FP16|zp W4 weights (the
    // kernel's zp), the zero-point code sums, the split partials
    const bool zp_table = !a.w8 && a.group != 16 && a.scale_enc == 1;
    auto lds_bytes = [&]() {
        return (size_t)a.T * (a.K + 16) + (a.w8 ? 0 : (size_t)rmax * g * 32) +
               (mode != 0 ? (size_t)(zp_table ? 2 : 1) * nu * 16 * 4 : 0) + (size_t)part * 256 * 4 + 64;
    };
    plan(0);
    int k = 0;
    if (!rpw && (2 * lds_bytes() > kRwLdsMax || wg >= 4 * cus)) {
        wpw = max_waves;
        plan(0);
        if (lds_bytes() > kRwLdsMax) {          // the larger tables do not fit
            wpw = std::min(kRwWaves, max_waves);
            plan(0);
        }
    } else if (!rpw && !options().rowwave_plain_grid && wg >= cus && wg % cus != 0) {
        const int load_plain = (wg + cus - 1) / cus * rmax;
        k = wg / cus;
        plan(k);
        if (waves > max_waves || k * rmax >= load_plain) {
            k = 0;
            plan(0);
        }
    }
    size_t lds = lds_bytes();
    if (lds > kRwLdsMax) return 1;
    if (k) lds = std::max(lds, (size_t)160 * 1024 / (k + 1) + 1024);
    const dim3 block(64 * waves);
    const dim3 grid(wg);
    if (a.w8) {
        if (unit != 32 || mode != 1) return 1;
        const bool alt2 = a.variant == kVarGemv;
        if (a.T <= 8)
            return alt2 ? rw_launch<8, 32, 1, true, kRwRing, kWfW8>(a, grid, block, lds, st)
                        : rw_launch<8, 32, 1, false, kRwRing, kWfW8>(a, grid, block, lds, st);
        return alt2 ? rw_launch<16, 32, 1, true, kRwRing, kWfW8>(a, grid, block, lds, st)
                    : rw_launch<16, 32, 1, false, kRwRing, kWfW8>(a, grid, block, lds, st);
    }
    if (a.group == 16) {
        if (unit != 32 || mode != 1 || a.variant != kVarGemv) return 1;
        return a.T <= 8 ? rw_launch<8, 32, 1, true, kRwRing, kWfK16>(a, grid, block, lds, st)
                        : rw_launch<16, 32, 1, true, kRwRing, kWfK16>(a, grid, block, lds, st);
    }
    if (a.T <= 8) return rw_unit<8>(a, unit, mode, grid, block, lds, st);
    return rw_unit<16>(a, unit, mode, grid, block, lds, st);
}

}  // namespace kxw4
