// kxw4_rowwave.hip — decode-shaped projections for up to 16 tokens with one
// split plan for every token and weight of a launch: the GEMV
// (kernels_dpas.cpp:586-675), the fan-out GEMV (945-1102) and the batched
// GEMM at small T (1334-1490).
//
// Balance. A decode projection is a weight stream, and each CU's share of the
// HBM bandwidth follows the bytes it keeps in flight, so every CU gets the
// same rows: the rows of all weights of the launch, taken in order, are cut
// into 8-row halves of row-groups (one 128-byte line of each lane group of a
// packed tile, so no line is fetched by two work-groups) and work-group b of
// the launch owns halves [H*b/NWG, H*(b+1)/NWG). With NWG = k * CUs and the
// LDS request padded so that no CU holds more than k, each CU streams the
// same bytes to within one half.
//
// Waves. A work-group's rows are cut into `spw` slices of one or two halves;
// each slice has min(S, 8) waves, one per split (two in turn when S = 16).
// A wave reads its slice as a 16-row window: lane n takes the window's row r
// with r = n (mod 16), which may lie in either of the two row-groups a window
// at an 8-row offset spans, so each lane addresses its own row-group's tile.
// The int8 MFMA does not care which row-group a column comes from: it leaves
// row n of tokens 4*(l/16)+r in register r of lane l for every unit, and a
// lane's four accumulators run four of the reference's chains, fed unit by
// unit in order. Lanes of a window with fewer than 16 rows read the line of
// another lane of their lane group (no extra memory traffic) and store
// nothing. With S > 1 the split partials meet in LDS and one wave adds them in
// split order starting from 0.0f.
//
// The activations (T x K int8) and the work-group's FP16 scales are staged
// into LDS once per work-group with direct global->LDS loads, so the
// weight-tile loads (and, for the per-token group-64 and W8 instances, the
// scales that ride beside them) are the only vector-memory instructions of
// the streaming loop. Activation rows are padded by 16 bytes, so the 8 or 16
// token rows a 16-lane quarter reads fall on distinct banks. Whole rings run
// without predicates; only a split's last, partial ring selects the old
// accumulator for its padded positions. Weight tiles are read once per
// launch, so their loads are non-temporal (they do not displace the
// activations from L2).
//
// W8 (the W8A8 tier, x_gemv_w8a8_core / x_gemm_w8a8, kernels_dpas.cpp:
// 771-844, 1578-1629): 2 KB int8 tiles, two 16-byte loads per lane and tile,
// used as the K32 MFMA operand without an unpack; the MFMA result is the unit
// partial itself (no factor 16) and the chain is the reference mode's with
// zero point 0. The per-K32 scales are not staged: one 2-byte load per lane
// and tile rides in the ring, and four lane shuffles hand each lane its row's
// four unit scales.
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

constexpr size_t kRwLdsMax = 160 * 1024;
constexpr int kRwSplitWaves = 8;            // most waves that share one slice's splits
constexpr int kRwMaxHalves = 2;             // halves of a slice: one 16-row window
// zero words at the end of the work-group's LDS: 16 (a padded position's
// scale reads), 144 for the one- and two-token K16 instances (a 4-tile
// ring's activation reads of the lanes that hold the other half: 4*128 + 64
// bytes)
constexpr int kRwK16ZeroWords = 144;

enum { kWfW4 = 0, kWfW8 = 1, kWfK16 = 2 };     // weight format of a row-wave instance

// Waves a work-group may hold. It sets the register budget per lane: the
// 8-deep ring and the K16 tier's two masked half MFMAs per unit need 256
// registers (two waves per SIMD), the 4-deep ring fits 128 (four).
__host__ __device__ constexpr int rw_max_waves(int wf, int pf) { return wf == kWfK16 || pf > 4 ? 8 : 16; }

template <int TT, int UNIT, int MODE, bool ALT2, int PF, int WF>
__global__ __launch_bounds__(64 * rw_max_waves(WF, PF)) void rowwave_kernel(const DecodeArgs a) {
    constexpr int UPS = kTileK / UNIT;
    constexpr bool W8 = WF == kWfW8, K16 = WF == kWfK16;
    // per-token W4 at group 64 (plain FP16 scales, unit = group): the tile's
    // two scales ride in the ring too, one 2-byte load per lane and unit, so
    // staging holds only the activations and the stream starts without
    // waiting for the scale table's HBM reads (cfg2 M=1, 8.7 KB per
    // row-group: 0.1-0.9 us faster on the boxes measured). At group 128 the
    // table is a fifth of that and the extra load per tile cost more than the
    // wait (cfg1: 0.7 us slower); group 32 would need four loads per tile
    // and spills.
    constexpr bool SRW4 = WF == kWfW4 && MODE == 0 && UNIT == 64;
    // TT = 1 or 2 (at most TT tokens): the MFMA leaves token 4*(l/16) + r in
    // register r of lane l, so only registers r < TT hold real tokens and the
    // chain runs on those alone (T = 1: a quarter of the chain's work)
    constexpr int NR = TT < 4 ? TT : 4;
    static_assert(TT >= 8 || (WF == kWfW4 && (MODE == 0 || MODE == 2 || MODE == 4)) || WF == kWfK16,
                  "short-token chains: per-token W4, the folded-zero-point GEMV and K16");
    static_assert(WF == kWfW4 || (UNIT == 32 && MODE == 1), "W8 / K16: K32 units, reference mode");
    static_assert(!K16 || ALT2, "K16 is a GEMV");
    // MODE 2 / 3: the reference mode of x_gemv_w4a8 / x_gemm_w4a8 themselves
    // (K32 activation blocks, FP16|zp weights) with every mode flag known at
    // compile time (MODE 3: the GEMM's x * (ws * as) association, MODE 2 the
    // GEMV's and fan-out's (x * ws) * as) and each unit's zero point folded
    // into the weight bytes (the K16 unpack: bytes w - z), so the MFMA returns
    // d - z * asum and the code-sum table and its per-output correction are
    // gone. MODE 1 keeps the other reference-mode combinations (per-token
    // activations with FP16|zp weights, K32 blocks with plain FP16 weights)
    // behind runtime flags. MODE 4 / 5 are MODE 2 / 3 at weight group 64 as
    // a compile-time fact, so the two units of a group share their scale
    // word's zero-point broadcast and scale conversion.
    constexpr bool ZF = MODE >= 2;
    constexpr bool ZGEMM = MODE == 3 || MODE == 5;
    static_assert(!ZGEMM || !ALT2, "the GEMM association has one accumulator");
    static_assert(!ZF || (WF == kWfW4 && UNIT == 32), "folded zero points: W4, K32 units");
    constexpr int TB = W8 ? 2 : 1;                 // 16-byte loads per lane and tile
    // undoes the nibble unpack's factor 16 (the folded and W8/K16 bytes have none)
    constexpr float kInv16 = WF != kWfW4 || ZF ? 1.0f : 0.0625f;
    static_assert(PF % 2 == 0, "the GEMV accumulator parity assumes an even ring");
    static_assert(!(K16 && NR < 4) || PF * kTileK + 64 <= 4 * kRwK16ZeroWords,
                  "a ring's zero reads stay inside the zero words");
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int nthreads = blockDim.x, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, n = lane & 15, g4 = lane >> 4;
    const int S = a.rw_S, wrg = a.rw_wrg, spw = a.rw_spw;
    const int K = a.K, T = a.T;
    const int NT = K / kTileK, Nu = K / UNIT, G = K / a.group;
    const int gsh = MODE >= 4 ? 1 : a.group >= UNIT ? __builtin_ctz(a.group / UNIT) : 0;

    // ---- this work-group's halves [h0, h1), this wave's slice ----
    const int b = blockIdx.x, NWG = gridDim.x, H = a.rw_halves;
    const int h0 = (int)((long long)H * b / NWG), h1 = (int)((long long)H * (b + 1) / NWG);
    const int sl = wave / wrg, wj = wave - sl * wrg;
    const int sh0 = h0 + (h1 - h0) * sl / spw, sh1 = h0 + (h1 - h0) * (sl + 1) / spw;
    const bool active = sl < spw && sh1 > sh0;
    const int gr_lo = (8 * h0) >> 4;                          // first row-group (all weights in order)
    const int n_gr = h1 > h0 ? ((8 * h1 - 1) >> 4) - gr_lo + 1 : 0;

    // This lane's row: r0 + off (off = (n - r0) mod 16) when the slice holds
    // that many rows; otherwise the lane reads the row of lane n ^ 8 (the
    // same lines of its lane group) and stores nothing.
    const int r0 = 8 * (active ? sh0 : h0), L = active ? 8 * (sh1 - sh0) : 8;
    const int off = (n - r0) & 15;
    const bool act = off < L;
    const int row = r0 + (act ? off : (off ^ 8));
    const int pitch = K + 16;                                 // padded activation row
    int8_t *Act = reinterpret_cast<int8_t *>(smem);
    uint16_t *Sc = reinterpret_cast<uint16_t *>(smem + (size_t)T * pitch);
    // The weight that holds a row-group, its first row-group and its
    // pointers, chosen with uniform indices: scalar loads of the kernel
    // arguments, made opaque so the choice stays a select. Indexed per lane,
    // the kernel arguments are vector memory loads, and their wait also
    // waits for the staging loads issued before them, so the weight ring
    // would start only once the staging had landed.
    // (global address space: through the asm statements the compiler could
    // no longer infer it and would make the ring's loads flat ones)
    using gcodes_t = __attribute__((address_space(1))) const uint8_t *;
    using gscales_t = __attribute__((address_space(1))) const uint16_t *;
    struct WPick { gcodes_t codes; gscales_t scales; int rg_begin, idx; };
    auto pick_weight = [&](int grp) {
        WPick w{(gcodes_t)a.w[0].codes, (gscales_t)a.w[0].scales, a.w[0].rg_begin, 0};
#pragma unroll
        for (int i = 1; i < kMaxWeights; ++i) {
            const int j = i < a.count ? i : 0;
            gcodes_t ci = (gcodes_t)a.w[j].codes;
            gscales_t si = (gscales_t)a.w[j].scales;
            int ri = a.w[j].rg_begin;
            asm volatile("" : "+s"(ci), "+s"(si), "+s"(ri));
            const bool in = i < a.count && grp >= ri;
            w.codes = in ? ci : w.codes;
            w.scales = in ? si : w.scales;
            w.rg_begin = in ? ri : w.rg_begin;
            w.idx = in ? i : w.idx;
        }
        return w;
    };
    // the row's weight, its row within the weight, and its pointers
    const int gr = row >> 4;
    const WPick wp = pick_weight(gr);
    const int wsel = wp.idx;
    const int lrg = gr - wp.rg_begin;
    const int lrow = lrg * 16 + (row & 15);
    __attribute__((address_space(1))) const v4u *wrow =
        reinterpret_cast<__attribute__((address_space(1))) const v4u *>(wp.codes + (size_t)lrg * NT * kTileBytes * TB) +
        (row & 15) + 16 * g4;
    const uint16_t *sbase = Sc + (gr - gr_lo) * G * 16 + (row & 15);
    const gscales_t wsc = wp.scales + ((size_t)lrg * G + g4) * 16 + (row & 15);

    // the zero-point code-sum table exists only for FP16|zp W4 weights (W8
    // has no zero points and K16 folds them into the weight bytes), so the
    // other formats ask for less LDS
    const bool zp = WF == kWfW4 && a.scale_enc == 1 && !ZF;
    // W8 and per-token W4 scales are not staged: they stream through the
    // ring (below)
    float *Asc = reinterpret_cast<float *>(Sc + (W8 || SRW4 ? 0 : a.rw_grmax * G * 16));
    int *Zs = reinterpret_cast<int *>(Asc + (MODE != 0 ? Nu * 16 : 0));
    float *Part = reinterpret_cast<float *>(Zs + (MODE != 0 && zp ? Nu * 16 : 0));
    // 16 zero words: the scale (and activation scale) read of a padded
    // position, so its chain step fma(p, 0, acc) leaves acc unchanged
    // (p is a finite integer and a chain that starts at +0 never holds -0)
    float *Zero = Part + (S > 1 ? spw * (S - 1) * 256 : 0);

    // ---- stage activations and scales with direct global->LDS loads ----
    // LDS chunk x (16 bytes) is chunk x % (kc+1) of activation row x / (kc+1)
    // (the last chunk of a row is padding), then the work-group's row-groups'
    // scales, each [G][16].
    const int kc = K / 16;
    const int act_chunks = T * (kc + 1);
    const int total = act_chunks + (W8 || SRW4 ? 0 : n_gr * G * 2);
    for (int c0 = wave * 64; c0 < total; c0 += nthreads) {
        const int x = c0 + lane;
        if (x < total) {
            const void *src;
            if (x < act_chunks) {
                const int t = x / (kc + 1), p = x - t * (kc + 1);
                src = a.q + (size_t)t * K + 16 * min(p, kc - 1);
            } else {
                const int sx = x - act_chunks, gri = sx / (2 * G), part = sx - gri * 2 * G;
                const int gr = gr_lo + gri;
                const WPick sw = pick_weight(gr);
                src = (const void *)(sw.scales + (size_t)(gr - sw.rg_begin) * G * 16 + (size_t)part * 8);
            }
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(smem + (size_t)c0 * 16),
                                             16, 0, 0);
        }
    }

    // per-token mode: this lane's four token scales for the output, loaded
    // now (before the ring, so the staging wait below covers them) rather
    // than after the split sum, where they would add a memory round trip;
    // likewise the residual of this lane's outputs (one weight per launch).
    // The K16 instances load them after the stream instead: held across it,
    // they are the registers its two half MFMAs per unit lack (they spilled).
    float tsc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    float rsd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto load_epilogue_inputs = [&]() {
        if (a.block == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) tsc[r] = a.ascale[min(4 * g4 + r, T - 1)];
        }
        if (a.residual) {
#pragma unroll
            for (int r = 0; r < 4; ++r) rsd[r] = a.residual[(size_t)min(4 * g4 + r, T - 1) * a.w[0].M + lrow];
        }
    };
    if constexpr (!K16) load_epilogue_inputs();

    // ---- the wave's first split and its ring ----
    const int sb = wj * S / wrg, se = (wj + 1) * S / wrg;
    // split ranges [Nu*s/S, Nu*(s+1)/S); S is a power of two (checked by
    // the launcher) and Nu*S fits in 32 bits
    const int ls = __builtin_ctz(S);
    int u0 = (Nu * sb) >> ls, u1 = (Nu * (sb + 1)) >> ls;
    int kt0 = u0 / UPS, ntw = (u1 + UPS - 1) / UPS - kt0;
    v4u ring[PF][TB];
    // W8: the tile's FP16 scales ride in the ring, one per lane: lane n+16j
    // holds unit j's scale of row n (the tile's 128 bytes of the [rg][G][16]
    // table); the chain spreads them to the row's lanes with shuffles
    uint32_t sring[W8 ? PF : 1];
    // per-token W4: unit j of the tile's scale of this lane's row
    uint16_t wring[SRW4 ? PF : 1][SRW4 ? UPS : 1];
    const gscales_t wsr = wp.scales + (size_t)lrg * G * 16 + (row & 15);
    // tile i of the current split; an empty split (more splits than units)
    // or an idle wave reads a valid tile it never uses
    auto load = [&](int i, int p) {
        const int kt = min(kt0 + max(i, 0), NT - 1);
        const size_t t = (size_t)kt * (kTileBytes * TB / 16);
#pragma unroll
        for (int h = 0; h < TB; ++h) ring[p][h] = __builtin_nontemporal_load(&wrow[t + 64 * h]);
        if constexpr (W8) sring[p] = wsc[(size_t)kt * (kTileK / 32) * 16];
        if constexpr (SRW4) {
#pragma unroll
            for (int j = 0; j < UPS; ++j) wring[p][j] = wsr[((size_t)kt * UPS + j) * 16];
        }
    };
    constexpr int LPT = TB + (W8 ? 1 : 0) + (SRW4 ? UPS : 0);   // loads per tile
    // With the scales riding in the ring (three loads per tile) the stream
    // starts after the staging has landed: issued beside it, cfg2 M=1 (17 KB
    // of activations per work-group) measured 12.4-12.6 against 11.9-12.1 us.
    if constexpr (SRW4) KXW4_WAIT_VMCNT(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PF; ++p) load(min(p, ntw - 1), p);
    __builtin_amdgcn_sched_barrier(0);
    // the staging loads were issued before the PF ring loads and complete first
    KXW4_WAIT_VMCNT(PF * LPT);
    // (the epilogue inputs count as arriving here: otherwise the compiler
    // hoists their first use, the token scale's 1/16, next to their loads,
    // and the wait it puts there also waits for the staging)
    if constexpr (!K16) {
#pragma unroll
        for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(tsc[r]), "+v"(rsd[r]));
    }
    const bool ref_block = ZF || a.block == 32;
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
    // (K16 with one or two tokens: 144 words, which the lanes whose
    // activation bytes belong to the other half read for a ring's tiles)
    // (a work-group may have fewer threads than words)
    for (int i = tid; i < (K16 && NR < 4 ? kRwK16ZeroWords : 16); i += nthreads) Zero[i] = 0.0f;
    lds_sync_after_dma();

    // ---- streaming: one chain per split, in registers ----
    const bool gemm_var = ZF ? ZGEMM : a.variant == kVarGemm;
    // this lane's activation row (MFMA row n; with up to 8 tokens rows 8-15
    // repeat rows 0-7 and are never stored) and its K-slot group
    const int ta = TT <= 8 ? min(n & 7, T - 1) : min(n, T - 1);
    const int8_t *abase = Act + (size_t)ta * pitch + 16 * g4;
    // K16 with one or two tokens: whether this lane's activation bytes (K
    // slots 8*g4 .. 8*g4+7 of each unit, row n) belong to its row's half
    const bool k16_keep = (n < 8) == (g4 < 2);
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
            // LOADS: whether the pass refills each slot with the tile PF
            // ahead. The split's last pass loads nothing: a load past the
            // split's last tile would hold its registers, and every later use
            // of them (the split sum, the epilogue) would wait for it.
            auto ring_pass = [&](int ib, auto pred, auto loads) {
                constexpr bool PRED = decltype(pred)::value;
                constexpr bool LOADS = decltype(loads)::value;
                // K16 with one or two tokens: lanes holding the other half's
                // K slots read zeros (the ring's tiles are immediate offsets
                // 0 .. PF*128+64 from the zero area)
                const int8_t *ar = K16 && NR < 4 && !k16_keep ? reinterpret_cast<const int8_t *>(Zero)
                                                             : abase + (size_t)(kt0 + ib) * kTileK;
#pragma unroll
                for (int p = 0; p < PF; ++p) {
                    const int i = ib + p;
                    const int kb = kt0 + i;
                    // (K16 with one or two tokens: MFMA row t + 8h carries half
                    // h of token t -- rows 0-7 keep K slots 0-15, lane groups
                    // 0-1, rows 8-15 slots 16-31, lane groups 2-3 -- so one
                    // MFMA per unit gives both half partials)
                    const v4i A0 = *reinterpret_cast<const v4i *>(ar + p * kTileK);
                    const v4i A1 = *reinterpret_cast<const v4i *>(ar + p * kTileK + 64);
                    const v4u wd = ring[p][0];
                    // W8: unit j's scale of this lane's row, from lane n + 16j
                    uint32_t s8[W8 ? 4 : 1];
                    if constexpr (W8) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) s8[j] = (uint32_t)__shfl((int)sring[p], n + 16 * j);
                    }
                    // folded zero points with one or two tokens: the tile's
                    // scale words and activation scales, read together
                    // before its units (read per unit, each unit waited
                    // for its own two LDS round trips)
                    // (K16 with one or two tokens likewise: its units' two
                    // scale words each)
                    constexpr bool kTileScales = (ZF || K16) && NR < 4;
                    constexpr int SWU = K16 ? 2 : 1;              // scale words per unit
                    uint32_t zsw[kTileScales ? UPS : 1][SWU];
                    float zas[kTileScales ? UPS : 1][NR];
                    if constexpr (kTileScales) {
#pragma unroll
                        for (int j = 0; j < UPS; ++j) {
                            const int u = kb * UPS + j;
                            const bool in = !PRED || (i < ntw && (u >= u0 && u < u1));
#pragma unroll
                            for (int q = 0; q < SWU; ++q)
                                zsw[j][q] = *(in ? &sbase[(K16 ? 2 * u + q : (u >> gsh)) * 16]
                                                 : reinterpret_cast<const uint16_t *>(Zero) + n);
                            const float *ap = in ? Asc + u * 16 + 4 * g4 : Zero + 4 * g4;
#pragma unroll
                            for (int r = 0; r < NR; ++r) zas[j][r] = ap[r];
                        }
                    }
#pragma unroll
                    for (int j = 0; j < UPS; ++j) {
                        const int u = kb * UPS + j;
                        const bool in = !PRED || (i < ntw && (UNIT == 128 || (u >= u0 && u < u1)));
                        const v4i zero = {0, 0, 0, 0};
                        long av = 0;
                        if constexpr (UNIT == 32) {
                            const v4i c = j < 2 ? A0 : A1;
                            av = (j & 1) ? (long)(((uint64_t)(uint32_t)c.w << 32) | (uint32_t)c.z)
                                         : (long)(((uint64_t)(uint32_t)c.y << 32) | (uint32_t)c.x);
                        }
                        float avr[4] = {1.0f, 1.0f, 1.0f, 1.0f};
                        v4i zv = {0, 0, 0, 0};
                        if constexpr (kTileScales) {
#pragma unroll
                            for (int r = 0; r < NR; ++r) avr[r] = zas[j][r];
                        } else if constexpr (MODE != 0) {
                            const float4 a4 = *reinterpret_cast<const float4 *>(in ? Asc + u * 16 + 4 * g4 : Zero + 4 * g4);
                            avr[0] = a4.x;
                            avr[1] = a4.y;
                            avr[2] = a4.z;
                            avr[3] = a4.w;
                            if (WF == kWfW4 && zp)
                                zv = *reinterpret_cast<const v4i *>(in ? Zs + u * 16 + 4 * g4
                                                                       : reinterpret_cast<const int *>(Zero) + 4 * g4);
                        }
                        {
                            const uint16_t *sw = sbase;
                            v4i acc;
                            if constexpr (UNIT == 128) {
                                acc = mfma_k64(A0, unpack_k64(wd.x, wd.y), zero);
                                acc = mfma_k64(A1, unpack_k64(wd.z, wd.w), acc);
                            } else if constexpr (UNIT == 64) {
                                acc = j == 0 ? mfma_k64(A0, unpack_k64(wd.x, wd.y), zero)
                                             : mfma_k64(A1, unpack_k64(wd.z, wd.w), zero);
                            } else {
                                long bv;
                                if constexpr (K16 && kTileScales) {
                                    // the unit's two K16 scale words (lane groups
                                    // 0-1 carry half 0, 2-3 half 1), its zero point
                                    // folded in as in the folded-zero-point
                                    // instances: bytes 0x80 | (w ^ 8) minus z + 8,
                                    // then XOR 0x80 (the bytes w - z)
                                    const uint32_t s0 = zsw[j][0], s1 = zsw[j][1];
                                    const uint32_t d = j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w;
                                    const uint32_t zz = __builtin_amdgcn_perm(0u, ((g4 < 2 ? s0 : s1) & 0xFu) ^ 8u, 0u);
                                    const uint32_t lo = ((((d ^ 0x08080808u) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                                    const uint32_t hi = (((((d >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                                    bv = (long)((uint64_t)lo | ((uint64_t)hi << 32));
                                    // half 0 of token r in register r of lanes 0-15,
                                    // half 1 in lanes 32-47, brought down 32 lanes (the
                                    // swap's other operand, whose low lanes it
                                    // overwrites, is a register no token uses: r + 2)
                                    const v4i acc1 = mfma_k32(av, bv, zero);
                                    int ph1[NR];
#pragma unroll
                                    for (int r = 0; r < NR; ++r)
                                        ph1[r] = (int)__builtin_amdgcn_permlane32_swap((unsigned)acc1[r], (unsigned)acc1[r + 2],
                                                                                      false, false)[1];
#pragma unroll
                                    for (int h = 0; h < 2; ++h) {
                                        const float ws = half_bits_to_float((uint16_t)((h ? s1 : s0) & 0xFFF0u));
#pragma unroll
                                        for (int r = 0; r < NR; ++r)
                                            f0[r] = __builtin_fmaf((float)(h ? ph1[r] : acc1[r]) * ws, zas[j][r], f0[r]);
                                    }
                                    // (with one or two tokens the registers allow a
                                    // tile's units to overlap; the chain updates stay
                                    // in unit order)
#pragma unroll
                                    for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(f0[r]));
                                    continue;
                                } else if constexpr (K16) {
                                    // the unit's two K16 scale words; lane groups
                                    // 0-1 carry half 0, 2-3 half 1
                                    const uint32_t s0 = *(in ? &sw[(2 * u) * 16] : reinterpret_cast<const uint16_t *>(Zero) + n);
                                    const uint32_t s1 = *(in ? &sw[(2 * u + 1) * 16] : reinterpret_cast<const uint16_t *>(Zero) + n);
                                    const uint32_t x = (j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w) ^ 0x88888888u;
                                    const uint32_t cz = (uint32_t)(120 - sext4(g4 < 2 ? s0 : s1)) * 0x01010101u;
                                    const uint64_t lo = ((x & 0x0F0F0F0Fu) + cz) ^ 0x80808080u;
                                    const uint64_t hi = (((x >> 4) & 0x0F0F0F0Fu) + cz) ^ 0x80808080u;
                                    bv = (long)(lo | (hi << 32));
                                    const v4i ph[2] = {mfma_k32(av, g4 < 2 ? bv : 0l, zero), mfma_k32(av, g4 < 2 ? 0l : bv, zero)};
#pragma unroll
                                    for (int h = 0; h < 2; ++h) {
                                        const float ws = half_bits_to_float((uint16_t)((h ? s1 : s0) & 0xFFF0u));
#pragma unroll
                                        for (int r = 0; r < NR; ++r) f0[r] = __builtin_fmaf((float)ph[h][r] * ws, avr[r], f0[r]);
                                    }
                                    // (one unit at a time: hoisting the next units'
                                    // scale and activation reads above this one's
                                    // MFMAs made the instance spill)
                                    __builtin_amdgcn_sched_barrier(0);
                                    continue;
                                } else if constexpr (W8) {
                                    const v4u hh = ring[p][j >> 1];
                                    bv = (j & 1) ? (long)(((uint64_t)hh.w << 32) | hh.z)
                                                 : (long)(((uint64_t)hh.y << 32) | hh.x);
                                } else if constexpr (ZF) {
                                    // the unit's zero point folded in: each
                                    // nibble w becomes the byte 0x80 | (w ^ 8)
                                    // = 136 + w (one three-input bit operation),
                                    // minus z + 8 (the scale word's low nibble
                                    // XOR 8, broadcast to every byte) leaves
                                    // 128 + w - z in [113, 143] (no borrow
                                    // crosses a byte), and the XOR gives the
                                    // int8 bytes w - z
                                    uint32_t s0;
                                    if constexpr (kTileScales) s0 = zsw[j][0];
                                    else s0 = *(in ? &sw[(u >> gsh) * 16] : reinterpret_cast<const uint16_t *>(Zero) + n);
                                    const uint32_t d = j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w;
                                    const uint32_t zz = __builtin_amdgcn_perm(0u, (s0 & 0xFu) ^ 8u, 0u);
                                    const uint32_t lo = ((((d ^ 0x08080808u) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                                    const uint32_t hi = (((((d >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                                    bv = (long)((uint64_t)lo | ((uint64_t)hi << 32));
                                } else {
                                    bv = unpack_k32(j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w);
                                }
                                acc = mfma_k32(av, bv, zero);
                            }
                            // MODE 0 has unit == group, so unit u reads scale u
                            const uint16_t *sp = &sw[(MODE == 0 ? u : (u >> gsh)) * 16];
                            uint32_t sv;
                            if constexpr (W8) sv = in ? s8[j] : 0u;
                            else if constexpr (SRW4) sv = in ? (uint32_t)wring[p][j] : 0u;
                            else if constexpr (kTileScales) sv = zsw[j][0];
                            else sv = *(in ? sp : reinterpret_cast<const uint16_t *>(Zero) + n);
                            // GEMV: units at odd offsets from the split start feed the
                            // second accumulator. With an even ring and an even number
                            // of units per tile the parity is fixed by p (whole-tile
                            // units) or j; when the split starts on an odd unit the two
                            // accumulators trade roles, and their final sum commutes.
                            float *F = (ALT2 && (UNIT == 128 ? (p & 1) : (j & 1))) ? f1 : f0;
                            if constexpr (MODE == 0) {
                                const float ws = half_bits_to_float((uint16_t)sv);
#pragma unroll
                                for (int r = 0; r < NR; ++r) F[r] = __builtin_fmaf((float)acc[r], ws, F[r]);
                            } else {
                                const float ws = half_bits_to_float(zp || ZF ? (uint16_t)(sv & 0xFFF0u) : (uint16_t)sv);
                                const int z = sext4(sv);
#pragma unroll
                                for (int r = 0; r < NR; ++r) {
                                    int pv = acc[r];
                                    if (zp) pv -= (z * zv[r]) << 4;
                                    const float pf = (float)pv;
                                    float nf;
                                    if (!ref_block) nf = __builtin_fmaf(pf, ws, F[r]);
                                    else if (gemm_var) nf = __builtin_fmaf(pf, ws * avr[r], F[r]);
                                    else nf = __builtin_fmaf(pf * ws, avr[r], F[r]);
                                    F[r] = nf;
                                }
                            }
                        }
                        // (folded zero points: one unit at a time, its
                        // chain updates kept in it; with no branch left in
                        // the unit the compiler otherwise sinks every
                        // unit's updates below the ring and spills the
                        // partials. With one or two tokens the registers
                        // allow the units of a tile to overlap: their LDS
                        // reads issue together and each chain update runs
                        // after the next unit's MFMA.)
                        if constexpr (ZF) {
#pragma unroll
                            for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(f0[r]), "+v"(f1[r]));
                            if constexpr (NR >= 4) __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                    if constexpr (LOADS) load(min(i + PF, ntw - 1), p);
                    // keep each slot's unpack behind the previous slot's load, so
                    // the wait before it covers only that slot
                    __builtin_amdgcn_sched_barrier(0);
                }
            };

            // whole rings run unpredicated when the split starts and ends on
            // tile boundaries; the rest (at most one ring then) is predicated
            const bool aligned = u0 % UPS == 0 && u1 % UPS == 0;
            using T_ = std::true_type;
            using F_ = std::false_type;
            // Only the per-token group-64 instances take the load-free last
            // pass (cfg2 M=1: 13.3-13.9 against 13.7-14.3 us). The others keep
            // one refilling pass: a second copy of their ring spills (K16,
            // group 32), takes more than the 80 registers that let two 10-wave
            // work-groups share a CU (group 128), or measured slower (W8:
            // lm_head 249 against 242 us).
            constexpr bool kLastNoLoads = WF == kWfW4 && UNIT == 64 && MODE == 0;
            int ib = 0;
            // (the last ring, full or not, runs predicated: one copy of the
            // ring code without loads, not two)
            if (aligned)
                for (; ib + PF < ntw || (!kLastNoLoads && ib + PF <= ntw); ib += PF) ring_pass(ib, F_{}, T_{});
            for (; ib < ntw; ib += PF) {
                if (!kLastNoLoads || ib + PF < ntw) ring_pass(ib, T_{}, T_{});
                else if constexpr (kLastNoLoads) ring_pass(ib, T_{}, F_{});
            }
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float v = (ALT2 && !K16) ? f0[r] + f1[r] : f0[r];
                // split 0 stays in the registers of the wave that adds the splits
                if (S > 1 && s > 0) Part[((sl * (S - 1) + s - 1) * 4 + r) * 64 + lane] = v;
                else res[r] = v;
            }
        }
    }

    // ---- ordered split sum and output ----
    if (S > 1) {
        lds_sync();
        if (!active || wj != 0) return;
        // S - 1 partials per live register, all read before the ordered
        // adds (a loop over s would wait for each read in turn)
        // (registers r in groups of RB, at most 16 reads in flight)
        auto split_sum = [&](auto sc) {
            constexpr int SC = decltype(sc)::value;
            constexpr int RB = (SC - 1) * NR <= 16 ? NR : 1;
#pragma unroll
            for (int r0 = 0; r0 < NR; r0 += RB) {
                float p[RB][SC - 1];
#pragma unroll
                for (int r = 0; r < RB; ++r)
#pragma unroll
                    for (int j = 1; j < SC; ++j)
                        p[r][j - 1] = Part[((sl * (SC - 1) + j - 1) * 4 + r0 + r) * 64 + lane];
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    float sum = 0.0f + res[r0 + r];
#pragma unroll
                    for (int j = 1; j < SC; ++j) sum = sum + p[r][j - 1];
                    res[r0 + r] = sum;
                }
            }
        };
        // (S is a power of two, at most 16: checked by the launcher). Only
        // the one- and two-token instances, whose few live registers make
        // S - 1 the whole wait: in the others the batch costs registers
        // that the two work-groups per CU of the group-128 launches need.
        if constexpr (NR < 4) {
            switch (S) {
            case 2: split_sum(std::integral_constant<int, 2>{}); break;
            case 4: split_sum(std::integral_constant<int, 4>{}); break;
            case 8: split_sum(std::integral_constant<int, 8>{}); break;
            default: split_sum(std::integral_constant<int, 16>{}); break;
            }
        } else if (S == 2) {
            split_sum(std::integral_constant<int, 2>{});
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float sum = 0.0f + res[r];
                for (int s = 1; s < S; ++s) sum = sum + Part[((sl * (S - 1) + s - 1) * 4 + r) * 64 + lane];
                res[r] = sum;
            }
        }
    } else if (!active) {
        return;
    }
    if (!act) return;
    // this lane's output buffer and height, chosen with uniform indices
    // (scalar loads of the kernel arguments, made opaque so the choice stays
    // a select): a per-lane index into the kernel arguments is a vector
    // memory load, whose wait would also wait for the ring's last loads
    if constexpr (K16) load_epilogue_inputs();
    __attribute__((address_space(1))) uint8_t *wy = (__attribute__((address_space(1))) uint8_t *)a.w[0].y;
    int wm = a.w[0].M;
#pragma unroll
    for (int i = 1; i < kMaxWeights; ++i) {
        __attribute__((address_space(1))) uint8_t *yi = (__attribute__((address_space(1))) uint8_t *)a.w[i < a.count ? i : 0].y;
        int mi = a.w[i < a.count ? i : 0].M;
        asm volatile("" : "+s"(yi), "+s"(mi));
        wy = wsel == i ? yi : wy;
        wm = wsel == i ? mi : wm;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int t = 4 * g4 + r;
        if (t >= T) continue;
        const float v = a.block == 0 ? res[r] * (tsc[r] * kInv16) : res[r] * kInv16;
        float out;
        if (a.residual) out = v + rsd[r];
        else if (ALT2 && S > 1) out = v + 0.0f;
        else out = v;
        if (a.y_bf16) ((__attribute__((address_space(1))) uint16_t *)wy)[(size_t)t * wm + lrow] = float_to_bf16(out);
        else ((__attribute__((address_space(1))) float *)wy)[(size_t)t * wm + lrow] = out;
    }
}

template <int TT, int UNIT, int MODE, bool ALT2, int PF, int WF>
static int rw_launch(const DecodeArgs &a, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    auto k = rowwave_kernel<TT, UNIT, MODE, ALT2, PF, WF>;
    static bool attr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -6;
    if (!attr[dev]) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kRwLdsMax) != hipSuccess)
            return -6;
        attr[dev] = true;
    }
    hipLaunchKernelGGL(k, grid, block, lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

template <int TT, int UNIT, int MODE, bool ALT2, int WF>
static int rw_ring(const DecodeArgs &a, int pf, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    if constexpr (WF != kWfK16 && TT >= 8) {
        if (pf == 8) return rw_launch<TT, UNIT, MODE, ALT2, 8, WF>(a, grid, block, lds, st);
    }
    return rw_launch<TT, UNIT, MODE, ALT2, 4, WF>(a, grid, block, lds, st);
}

template <int TT, int UNIT>
static int rw_mode(const DecodeArgs &a, int mode, int pf, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    const bool alt2 = a.variant == kVarGemv;
    if (mode == 0)
        return alt2 ? rw_ring<TT, UNIT, 0, true, kWfW4>(a, pf, grid, block, lds, st)
                    : rw_ring<TT, UNIT, 0, false, kWfW4>(a, pf, grid, block, lds, st);
    if constexpr (TT < 8) {
        // one or two tokens: the folded-zero-point GEMV only
        if constexpr (UNIT == 32) {
            if (mode == 2 && alt2) return rw_ring<TT, 32, 2, true, kWfW4>(a, pf, grid, block, lds, st);
            if (mode == 4 && alt2) return rw_ring<TT, 32, 4, true, kWfW4>(a, pf, grid, block, lds, st);
        }
        return 1;
    } else {
        if constexpr (UNIT == 32) {
            if (mode == 3) return rw_ring<TT, 32, 3, false, kWfW4>(a, pf, grid, block, lds, st);
            if (mode == 5) return rw_ring<TT, 32, 5, false, kWfW4>(a, pf, grid, block, lds, st);
            if (mode == 2)
                return alt2 ? rw_ring<TT, 32, 2, true, kWfW4>(a, pf, grid, block, lds, st)
                            : rw_ring<TT, 32, 2, false, kWfW4>(a, pf, grid, block, lds, st);
            if (mode == 4)
                return alt2 ? rw_ring<TT, 32, 4, true, kWfW4>(a, pf, grid, block, lds, st)
                            : rw_ring<TT, 32, 4, false, kWfW4>(a, pf, grid, block, lds, st);
        }
        return alt2 ? rw_ring<TT, UNIT, 1, true, kWfW4>(a, pf, grid, block, lds, st)
                    : rw_ring<TT, UNIT, 1, false, kWfW4>(a, pf, grid, block, lds, st);
    }
}

template <int TT>
static int rw_unit(const DecodeArgs &a, int unit, int mode, int pf, dim3 grid, dim3 block, size_t lds,
                   hipStream_t st) {
    if (unit == 128) return rw_mode<TT, 128>(a, mode, pf, grid, block, lds, st);
    if (unit == 64) return rw_mode<TT, 64>(a, mode, pf, grid, block, lds, st);
    return rw_mode<TT, 32>(a, mode, pf, grid, block, lds, st);
}

int launch_rowwave(DecodeArgs &a, hipStream_t st) {
    if (a.T < 1 || a.T > 16) return 1;
    const int unit = a.block == 32 ? 32 : a.group;
    const int nu = a.K / unit, g = a.K / a.group;
    int mode = (a.block == 0 && a.scale_enc == 0) ? 0 : 1;
    // one split plan for every token and weight
    const int S = a.w[0].seg_split[0];
    if (S < 1 || S > 16 || (S & (S - 1))) return 1;
    int rows = 0;
    for (int i = 0; i < a.count; ++i) {
        for (int s = 0; s < a.seg_count; ++s)
            if (a.w[i].seg_split[s] != S) return 1;
        a.w[i].rg_begin = rows / 16;
        rows += a.w[i].M;
    }
    const int wf = a.w8 ? kWfW8 : a.group == 16 ? kWfK16 : kWfW4;
    // K32 activation blocks against FP16|zp W4 weights (x_gemv_w4a8,
    // x_gemm_w4a8): the folded-zero-point instances
    // (modes 4 / 5: the same at group 64)
    if (wf == kWfW4 && a.block == 32 && a.scale_enc == 1)
        mode = (a.variant == kVarGemm ? 3 : 2) + (a.group == 64 ? 2 : 0);
    if (wf != kWfW4 && (unit != 32 || mode != 1)) return 1;
    if (wf == kWfK16 && a.variant != kVarGemv) return 1;
    const int wrg = std::min(S, kRwSplitWaves);
    const int H = rows / 8;
    const int cus = device_cus();
    const Options &opt = options();
    // ring depth 4 (8 on request: measured no faster at the decode shapes)
    const int pf = opt.rowwave_ring == 8 && wf != kWfK16 ? 8 : 4;
    const int max_waves = rw_max_waves(wf, pf);
    const int spw_cap = std::max(1, max_waves / wrg);
    const int spw_want = opt.rowwave_spw ? std::min(opt.rowwave_spw, spw_cap) : spw_cap;
    // k work-groups per CU: the fewest that keep every slice within one
    // 16-row window at spw_want slices per work-group (or the option's k)
    const int k = opt.rowwave_k ? opt.rowwave_k
                                : std::max(1, (H + cus * spw_want * kRwMaxHalves - 1) / (cus * spw_want * kRwMaxHalves));
    const int nwg = std::max(1, std::min(cus * k, H));
    const int hmax = (H + nwg - 1) / nwg;                   // most halves a work-group owns
    // the fewest slices that keep every slice within one window (fewer
    // waves for the same bytes), unless the option sets them
    int spw = opt.rowwave_spw ? spw_want : std::min(spw_cap, (hmax + kRwMaxHalves - 1) / kRwMaxHalves);
    spw = std::max(1, std::min(spw, hmax));
    if ((hmax + spw - 1) / spw > kRwMaxHalves) return 1;
    const int grmax = (hmax + 1) / 2 + 1;                   // row-groups a work-group's halves touch
    a.rw_S = S;
    a.rw_wrg = wrg;
    a.rw_spw = spw;
    a.rw_halves = H;
    a.rw_grmax = grmax;
    // the work-group's LDS: padded activation rows, its row-groups' scales,
    // the per-unit activation scales and, for FP16|zp W4 weights, the
    // zero-point code sums, the split partials, the zero words
    const bool zp_table = wf == kWfW4 && a.scale_enc == 1 && mode < 2;
    auto lds_for = [&](int T) {
        return (size_t)T * (a.K + 16) + (wf == kWfW8 || (wf == kWfW4 && mode == 0 && unit == 64) ? 0 : (size_t)grmax * g * 32) +
               (mode != 0 ? (size_t)(zp_table ? 2 : 1) * nu * 16 * 4 : 0) +
               (S > 1 ? (size_t)spw * (S - 1) * 256 * 4 : 0) + (wf == kWfK16 && T <= 2 ? 4 * kRwK16ZeroWords : 64);
    };
    size_t lds = lds_for(a.T);
    if (lds > kRwLdsMax) {
        // W4 weights hand the shape back: the K-parallel kernel reads the
        // weight once for every token.
        if (wf == kWfW4) return 1;
        // The tokens' activations do not fit (long K at W8 or K16, which
        // have no other kernel): run the tokens in chunks that do. A token's
        // outputs depend on its own activation row only, so the bits are the
        // same; every chunk streams the weights again.
        int tc = a.T - 1;
        while (tc > 0 && lds_for(tc) > kRwLdsMax) --tc;
        if (tc == 0 || a.seg_count != 1 || a.dbg) return 1;
        const size_t per_tok = a.block ? (size_t)(a.K / a.block) : 1;   // activation scales (and sums) per token
        for (int t0 = 0; t0 < a.T; t0 += tc) {
            DecodeArgs c = a;
            c.T = std::min(tc, a.T - t0);
            c.seg_end[0] = c.T;
            c.q = a.q + (size_t)t0 * a.K;
            c.ascale = a.ascale + (size_t)t0 * per_tok;
            c.asum = a.asum ? a.asum + (size_t)t0 * per_tok : nullptr;
            c.residual = a.residual ? a.residual + (size_t)t0 * a.w[0].M : nullptr;
            for (int i = 0; i < a.count; ++i)
                c.w[i].y = static_cast<uint8_t *>(a.w[i].y) + (size_t)t0 * a.w[i].M * (a.y_bf16 ? 2 : 4);
            const int r = launch_rowwave(c, st);
            if (r) return r < 0 ? r : -6;   // (a later chunk cannot be refused: it is no larger)
        }
        return 0;
    }
    // no CU takes a (k+1)-th work-group of this launch at a time
    lds = std::max(lds, kRwLdsMax / (k + 1) + 1024);
    const dim3 block(64 * spw * wrg);
    const dim3 grid(nwg);
    if (wf == kWfW8) {
        const bool alt2 = a.variant == kVarGemv;
        if (a.T <= 8)
            return alt2 ? rw_ring<8, 32, 1, true, kWfW8>(a, pf, grid, block, lds, st)
                        : rw_ring<8, 32, 1, false, kWfW8>(a, pf, grid, block, lds, st);
        return alt2 ? rw_ring<16, 32, 1, true, kWfW8>(a, pf, grid, block, lds, st)
                    : rw_ring<16, 32, 1, false, kWfW8>(a, pf, grid, block, lds, st);
    }
    if (wf == kWfK16) {
        // one or two tokens: the chains of the real tokens' registers only
        if (a.T == 1) return rw_ring<1, 32, 1, true, kWfK16>(a, 4, grid, block, lds, st);
        if (a.T == 2) return rw_ring<2, 32, 1, true, kWfK16>(a, 4, grid, block, lds, st);
        return a.T <= 8 ? rw_ring<8, 32, 1, true, kWfK16>(a, 4, grid, block, lds, st)
                        : rw_ring<16, 32, 1, true, kWfK16>(a, 4, grid, block, lds, st);
    }
    // one or two tokens in per-token mode or the folded-zero-point GEMV: the
    // short chains (4-deep ring)
    const bool short_ok = pf == 4 && (mode == 0 || ((mode == 2 || mode == 4) && a.variant == kVarGemv));
    if (short_ok && a.T == 1) return rw_unit<1>(a, unit, mode, pf, grid, block, lds, st);
    if (short_ok && a.T == 2) return rw_unit<2>(a, unit, mode, pf, grid, block, lds, st);
    if (a.T <= 8) return rw_unit<8>(a, unit, mode, pf, grid, block, lds, st);
    return rw_unit<16>(a, unit, mode, pf, grid, block, lds, st);
}

}  // namespace kxw4
