// kxw4_persist.hip — persistent decode kernel for up to 8 tokens in the
// per-token (config) mode: the GEMV (kernels_dpas.cpp:586-675), the fan-out
// GEMV (945-1102) and the batched GEMM at decode sizes (1334-1490).
//
// Work is counted in chains: one chain is one (row-group, split) of one
// weight, the unit of the reference's in-order FP32 accumulation. The chains
// of all weights, in (weight, row-group, split) order, are cut into one
// contiguous range per work-group, one work-group of 16 waves per CU, so
// every CU streams the same share of the weights (to within one chain). Inside
// a work-group with C chains:
//   * the first 16*floor(C/16) chains are dealt round-robin to the waves; a
//     wave streams each of its chains' 1 KB tiles and runs the chain in
//     registers (the int8 MFMA leaves row n of tokens 4*(l/16)+r in register
//     r of lane l, so a lane's accumulators are four of the reference's
//     chains, fed unit by unit in order);
//   * the remaining C % 16 chains are cut along K over all 16 waves, which
//     write their units' exact partials (16 P, an integer below 2^22) to LDS;
//     after the stream one wave per such chain runs its chain from LDS.
// Every wave streams its tiles through one ring of PF loads in flight that
// runs across its chain boundaries. The splits of a row-group are added in
// split order from 0.0f: in LDS when the row-group lies in one work-group,
// and through a device-scope exchange (the last of the work-groups sharing
// it adds and writes) when the range boundary cuts it.
//
// The activations (T x K int8), the FP16 scales of the work-group's
// row-groups and the token scales are staged into LDS once per work-group
// with direct global->LDS loads; activation rows are padded by 16 bytes so
// the token rows a 16-lane quarter reads fall on distinct banks.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace kxw4 {

constexpr int kPsWaves = 16;
constexpr int kPsThreads = 64 * kPsWaves;
constexpr int kPsMaxT = 8;
constexpr int kPsMaxS = 16;
constexpr int kPsMaxWg = 256;
constexpr int kPsPF = 4;
constexpr int kPsRunMax = 8;        // runs (remainder pieces + whole chains) per wave
constexpr size_t kPsLdsMax = 160 * 1024;

// Split results of row-groups cut between work-groups: slot b belongs to the
// cut row-group whose first chain lies in work-group b. The counters start at
// zero when the library loads and the last arriver puts them back to zero.
// Launches that overlap on one GPU share these and must not run concurrently.
__device__ __attribute__((aligned(256))) float g_ps_xpart[kPsMaxWg * kPsMaxS * kPsMaxT * 16];
// one counter per 256 bytes: atomics on a shared cache line serialize
constexpr int kPsCtrStride = 64;
__device__ __attribute__((aligned(256))) unsigned g_ps_xcount[kPsMaxWg * kPsCtrStride];

// One chain: weight, row-group within it, split, its units [u0, u1) and
// weight tiles [kt0, kt0 + nt).
struct PsChain {
    int wi, rl, s, S, u0, u1, kt0, nt;
};

template <int UPS>
__device__ __forceinline__ PsChain ps_chain(const DecodeArgs &a, int c, int Nu) {
    PsChain g;
    g.wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (c >= a.w[i].cbeg) g.wi = i;
    const DecodeWeight &W = a.w[g.wi];
    g.S = W.seg_split[0];
    const int ls = __builtin_ctz(g.S);
    const int local = c - W.cbeg;
    g.rl = local >> ls;
    g.s = local & (g.S - 1);
    g.u0 = (Nu * g.s) >> ls;
    g.u1 = (Nu * (g.s + 1)) >> ls;
    g.kt0 = g.u0 / UPS;
    g.nt = (g.u1 + UPS - 1) / UPS - g.kt0;
    return g;
}

// work-group holding chain c when C = q*G + r chains are cut into G ranges
// [floor(b*C/G), floor((b+1)*C/G)): start from c/(q+1) and step up
__device__ __forceinline__ int ps_wg_of_chain(int c, int q, int r, int G) {
    auto start = [&](int b) { return q * b + (r * b) / G; };
    int b = c / (q + 1);
    while (b + 1 < G && start(b + 1) <= c) ++b;
    return b;
}

// LDS layout in bytes: activations, scales [row-group][G][16] FP16 of the
// work-group's row-groups, remainder partials [slot][unit][TP][16] float
// (units padded by 8 for the serial chains' last batch), chain results
// [chain][TP][16] float, token scales, zero words, the waves' run tables
// (a header and kPsRunMax entries each), the chain table, hand-off counters,
// a dummy target.
struct PsLds {
    size_t act, sc, part, res, tsc, zero, runs, chains, ctl, dummy, total;
};

__host__ __device__ inline PsLds ps_lds(int T, int TP, int K, int G, int nrg, int rslots, int lmax, int cmax) {
    PsLds L;
    L.act = 0;
    L.sc = L.act + ((size_t)T * (K + 16) + 15) / 16 * 16;
    L.part = L.sc + (size_t)nrg * G * 32;
    L.res = L.part + (size_t)rslots * (lmax + 8) * TP * 16 * 4;
    L.tsc = L.res + (size_t)cmax * TP * 16 * 4;
    L.zero = L.tsc + kPsMaxT * 4;
    L.runs = L.zero + 16 * 4;
    L.chains = L.runs + (size_t)kPsWaves * (kPsRunMax + 1) * 32;
    L.ctl = L.chains + (size_t)cmax * 32;
    L.dummy = L.ctl + 16 * 4;
    L.total = L.dummy + 64 * 4;
    return L;
}

// LDS counters of the hand-offs inside a work-group: relaxed LDS atomics
// behind LDS-only fences.
__device__ __forceinline__ void ps_signal(int *ctr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The wait is bounded (about 2^22 polls, far beyond any legitimate wait), so
// a hand-off that never comes ends the kernel with wrong outputs instead of
// holding the GPU.
__device__ __forceinline__ void ps_wait(int *ctr, int target) {
    for (int spin = 0; spin < (1 << 22); ++spin) {
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) >=
            target)
            break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int UNIT, bool ALT2, int TP>
__global__ __launch_bounds__(kPsThreads) void persist_kernel(const DecodeArgs a) {
    constexpr int UPS = kTileK / UNIT;
    constexpr int PF = kPsPF;
    constexpr int W = kPsWaves;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int K = a.K, T = a.T;
    const int NT = K / kTileK, Nu = K / UNIT, G = Nu;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, n = lane & 15, g4 = lane >> 4;

    // ---- the work-group's chains and row-groups ----
    // range of work-group b: [floor(b*C/G), floor((b+1)*C/G)) with
    // C = q*G + r, so floor(b*C/G) = q*b + floor(r*b/G) in 32-bit math
    const int GW = gridDim.x;
    const int c0 = a.ps_q * (int)blockIdx.x + (a.ps_r * (int)blockIdx.x) / GW;
    const int c1 = a.ps_q * ((int)blockIdx.x + 1) + (a.ps_r * ((int)blockIdx.x + 1)) / GW;
    const int nc = c1 - c0;
    const int F = nc / W, nrem = nc - F * W;
    auto rg_of = [&](const PsChain &g) { return a.w[g.wi].rg_begin + g.rl; };
    const PsChain gfirst = ps_chain<UPS>(a, c0, Nu), glast = ps_chain<UPS>(a, c1 - 1, Nu);
    const int rgA = rg_of(gfirst), rgB = rg_of(glast);
    const int nrg = rgB - rgA + 1;
    const int lmax = (Nu + a.ps_smin - 1) / a.ps_smin;

    const PsLds L = ps_lds(T, TP, K, G, a.ps_nrg, a.ps_rslots, lmax, a.ps_cmax);
    int8_t *Act = reinterpret_cast<int8_t *>(smem + L.act);
    uint16_t *Sc = reinterpret_cast<uint16_t *>(smem + L.sc);
    float *Part = reinterpret_cast<float *>(smem + L.part);
    float *Res = reinterpret_cast<float *>(smem + L.res);
    float *Tsc = reinterpret_cast<float *>(smem + L.tsc);
    float *Zero = reinterpret_cast<float *>(smem + L.zero);
    float *dummy = reinterpret_cast<float *>(smem + L.dummy) + lane;
    const int pslot = (lmax + 8) * TP * 16;      // floats per remainder slot

    // ---- stage activations and the range's scales ----
    {
        const int kc = K / 16;
        const int act_chunks = T * (kc + 1);
        const int total = act_chunks + nrg * G * 2;
        for (int c = wave * 64; c < total; c += kPsThreads) {
            const int x = c + lane;
            if (x < total) {
                const void *src;
                if (x < act_chunks) {
                    const int t = x / (kc + 1), p = x - t * (kc + 1);
                    src = a.q + (size_t)t * K + 16 * min(p, kc - 1);
                } else {
                    const int y = x - act_chunks;
                    const int rg = rgA + y / (2 * G), off = y % (2 * G);
                    int wi = 0;
                    for (int i = 1; i < a.count; ++i)
                        if (rg >= a.w[i].rg_begin) wi = i;
                    src = a.w[wi].scales + (size_t)(rg - a.w[wi].rg_begin) * G * 16 + off * 8;
                }
                __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(smem + (size_t)c * 16),
                                                 16, 0, 0);
            }
        }
        // the token scales
        if (wave == 0 && lane < T)
            __builtin_amdgcn_global_load_lds((const void *)(a.ascale + lane),
                                             (__attribute__((address_space(3))) void *)(smem + L.tsc), 4, 0, 0);
        if (wave == 1 && lane < 16) Zero[lane] = 0.0f;
        if (wave == 1 && lane >= 16 && lane < 19) reinterpret_cast<int *>(smem + L.ctl)[lane - 16] = 0;
    }

    // ---- run tables ----
    // A wave's runs: its piece of the remainder chains (their tiles
    // concatenated and cut into 16 equal pieces), then its whole chains
    // (wave, wave + 16, ...). Wave 0 builds them while the staging loads fly:
    // first the chain table, one chain per lane, then each of lanes 0..15 the
    // table of one wave. Chain entry: u0, u1, first tile, tiles, tile address
    // (lane 0), row-group relative to the range's first. Run entry: tile
    // address (lane 0), first tile, tiles, chain units [u0, u1), row-group,
    // chain | slot << 16 | whole << 24. Header: runs, steps, remainder steps.
    int *ctab = reinterpret_cast<int *>(smem + L.chains);
    int *tab = reinterpret_cast<int *>(smem + L.runs) + wave * (kPsRunMax + 1) * 8;
    int *rem_done = reinterpret_cast<int *>(smem + L.ctl);
    if (wave == 0) {
        for (int i = lane; i < nc; i += 64) {
            const PsChain g = ps_chain<UPS>(a, c0 + i, Nu);
            const uint64_t ad = reinterpret_cast<uint64_t>(a.w[g.wi].codes + ((size_t)g.rl * NT + g.kt0) * kTileBytes);
            int *e = ctab + i * 8;
            e[0] = g.u0;
            e[1] = g.u1;
            e[2] = g.kt0;
            e[3] = g.nt;
            e[4] = (int)(uint32_t)ad;
            e[5] = (int)(uint32_t)(ad >> 32);
            e[6] = rg_of(g) - rgA;
        }
        if (lane < W) {
            // this lane builds the table of wave `lane`; its own chain table
            // writes above precede these reads (one wave, LDS in order)
            const int w = lane;
            int *tw = reinterpret_cast<int *>(smem + L.runs) + w * (kPsRunMax + 1) * 8;
            int nr = 0, st = 0;
            auto put = [&](int ci, int slot, bool whole, int t0, int nt) {
                if (nr < kPsRunMax) {
                    const int *ce = ctab + ci * 8;
                    const uint64_t ad = ((uint64_t)(uint32_t)ce[5] << 32 | (uint32_t)ce[4]) + (uint64_t)t0 * kTileBytes;
                    int *e = tw + (1 + nr) * 8;
                    e[0] = (int)(uint32_t)ad;
                    e[1] = (int)(uint32_t)(ad >> 32);
                    e[2] = ce[2] + t0;
                    e[3] = nt;
                    e[4] = ce[0];
                    e[5] = ce[1];
                    e[6] = ce[6];
                    e[7] = ci | (slot << 16) | ((whole ? 1 : 0) << 24);
                }
                ++nr;
                st += nt;
            };
            int rt = 0;
            for (int k = 0; k < nrem; ++k) rt += ctab[(F * W + k) * 8 + 3];
            const int ra = rt * w / W, rb = rt * (w + 1) / W;
            int pos = 0;
            for (int k = 0; k < nrem && pos < rb; ++k) {
                const int t = ctab[(F * W + k) * 8 + 3];
                const int lo = max(ra, pos), hi = min(rb, pos + t);
                if (lo < hi) put(F * W + k, k, false, lo - pos, hi - lo);
                pos += t;
            }
            const int sr = st;
            for (int f = 0; f < F; ++f) put(f * W + w, 0, true, 0, ctab[(f * W + w) * 8 + 3]);
            tw[0] = nr;
            tw[1] = st;
            tw[2] = sr;
        }
    }
    // The row-groups at the two ends of the range may be cut by the range
    // boundary: their local chains are [0, nfirst) and [nc - nlast, nc).
    // Their owners count them done in LDS; waves 0 and 1 publish them as
    // soon as they are, while the other waves still stream.
    int *cnt_first = rem_done + 1, *cnt_last = rem_done + 2;
    auto rg_info = [&](int rg, int &wi, int &rl, int &S, int &cr0) {
        wi = 0;
        for (int i = 1; i < a.count; ++i)
            if (rg >= a.w[i].rg_begin) wi = i;
        rl = rg - a.w[wi].rg_begin;
        S = a.w[wi].seg_split[0];
        cr0 = a.w[wi].cbeg + rl * S;
    };
    int nfirst = 0, nlast = 0;
    {
        int wi, rl, S, cr0;
        rg_info(rgA, wi, rl, S, cr0);
        if (cr0 < c0 || cr0 + S > c1) nfirst = min(cr0 + S, c1) - c0;
        if (nrg > 1) {
            rg_info(rgB, wi, rl, S, cr0);
            if (cr0 + S > c1) nlast = c1 - cr0;
        }
    }
    auto chain_done = [&](int ci) {
        if (ci < nfirst) ps_signal(cnt_first);
        if (ci >= nc - nlast) ps_signal(cnt_last);
    };

    // ---- ring ----
    // the tables are in LDS and every wave's staging loads are issued
    // before any ring load
    lds_sync_after_dma();
    const int nruns = __builtin_amdgcn_readfirstlane(tab[0]);
    const int steps = __builtin_amdgcn_readfirstlane(tab[1]);
    const int steps_rem = __builtin_amdgcn_readfirstlane(tab[2]);
    // loader cursor: run, tile within it, its tiles, address of this lane's
    // 16 bytes of the next tile
    v4u ring[PF];
    int lk = 0, lt = 0, lnt = 0;
    const uint8_t *lp;
    auto entry_addr = [&](int k) {
        const int *e = tab + (1 + k) * 8;
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane(e[0]);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane(e[1]);
        return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo) + lane * 16;
    };
    if (nruns > 0) {
        lp = entry_addr(0);
        lnt = __builtin_amdgcn_readfirstlane(tab[8 + 3]);
    } else {
        // no work: re-read a valid tile that is never used
        lp = a.w[0].codes + lane * 16;
        lk = 1;
    }
    auto load = [&](v4u &dst) {
        // a global (not flat) load: the address was rebuilt from integers,
        // and a flat load would also count against the LDS wait counter
        dst = *(const __attribute__((address_space(1))) v4u *)(lp);
        if (lk >= nruns) return;        // past the last tile: keep re-reading it
        if (++lt < lnt) {
            lp += kTileBytes;
        } else if (++lk < nruns) {
            lt = 0;
            lp = entry_addr(lk);
            lnt = __builtin_amdgcn_readfirstlane(tab[(1 + lk) * 8 + 3]);
        }
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PF; ++p) load(ring[p]);
    __builtin_amdgcn_sched_barrier(0);
    // the staging loads were issued before the ring's PF loads
    __builtin_amdgcn_s_waitcnt(0x0F70 | PF);
    lds_sync_after_dma();

    // ---- stream ----
    // this lane's MFMA row: token n & 7 (rows 8-15 repeat 0-7, never stored)
    const int ta = min(n & 7, T - 1);
    const int8_t *abase = Act + (size_t)ta * (K + 16) + 16 * g4;
    // processor cursor: run fields of the current run
    int pk = 0, pt = 0, pnt = 0, kt = 0, u0 = 0, u1 = 0, rgl = 0, pci = 0, pslotn = 0;
    bool whole = true;
    auto take = [&](int k) {
        const int *e = tab + (1 + k) * 8;
        kt = __builtin_amdgcn_readfirstlane(e[2]);
        pnt = __builtin_amdgcn_readfirstlane(e[3]);
        u0 = __builtin_amdgcn_readfirstlane(e[4]);
        u1 = __builtin_amdgcn_readfirstlane(e[5]);
        rgl = __builtin_amdgcn_readfirstlane(e[6]);
        const int x = __builtin_amdgcn_readfirstlane(e[7]);
        pci = x & 0xFFFF;
        pslotn = (x >> 16) & 0xFF;
        whole = (x >> 24) & 1;
        pt = 0;
    };
    if (nruns > 0) take(0);
    if (steps_rem == 0) ps_signal(rem_done);
    float f0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, f1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int ib = 0; ib < steps; ib += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            if (ib + p < steps) {
                const int8_t *ar = abase + (size_t)kt * kTileK;
                const v4i A0 = *reinterpret_cast<const v4i *>(ar);
                const v4i A1 = *reinterpret_cast<const v4i *>(ar + 64);
                const v4u wd = ring[p];
#pragma unroll
                for (int j = 0; j < UPS; ++j) {
                    const int u = kt * UPS + j;
                    const bool in = u >= u0 && u < u1;
                    const v4i zero = {0, 0, 0, 0};
                    v4i acc;
                    if constexpr (UNIT == 128) {
                        acc = mfma_k64(A0, unpack_k64(wd.x, wd.y), zero);
                        acc = mfma_k64(A1, unpack_k64(wd.z, wd.w), acc);
                    } else {
                        static_assert(UNIT == 64, "per-token mode has unit = group in {64, 128}");
                        acc = j == 0 ? mfma_k64(A0, unpack_k64(wd.x, wd.y), zero)
                                     : mfma_k64(A1, unpack_k64(wd.z, wd.w), zero);
                    }
                    if (whole) {
                        // a unit outside the chain reads a zero scale, so its
                        // step fma(p, 0, f) leaves f unchanged (p is a finite
                        // integer and a chain that starts at +0 never holds -0)
                        const uint16_t *sp = in ? Sc + ((size_t)rgl * G + u) * 16 + n
                                                : reinterpret_cast<const uint16_t *>(Zero) + n;
                        const float w = half_bits_to_float(*sp);
                        float *Fr = (ALT2 && ((u - u0) & 1)) ? f1 : f0;
#pragma unroll
                        for (int r = 0; r < 4; ++r) Fr[r] = __builtin_fmaf((float)acc[r], w, Fr[r]);
                    } else {
                        float *pp = Part + (size_t)pslotn * pslot + (size_t)(u - u0) * TP * 16 + n;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int t = 4 * g4 + r;
                            // 16*P is exact in FP32 (|16*P| < 2^24)
                            float *dst = (in && t < TP) ? pp + t * 16 : dummy;
                            *dst = (float)acc[r];
                        }
                    }
                }
                ++kt;
                if (++pt == pnt) {
                    if (whole) {
                        float *rp = Res + (size_t)pci * TP * 16 + n;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int t = 4 * g4 + r;
                            float *dst = t < TP ? rp + t * 16 : dummy;
                            *dst = ALT2 ? f0[r] + f1[r] : f0[r];
                            f0[r] = 0.0f;
                            f1[r] = 0.0f;
                        }
                        chain_done(pci);
                    }
                    if (++pk < nruns) take(pk);
                }
                // this wave's remainder partials are all in LDS
                if (ib + p + 1 == steps_rem) ps_signal(rem_done);
            }
            load(ring[p]);
            // keep each slot's unpack behind the previous slot's load, so the
            // wait before it covers only that slot
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Drain the ring's last (re-)loads: the waves' paths join below.
    __builtin_amdgcn_s_waitcnt(0);

    // ---- remainder chains, one wave each, from their LDS partials, once
    // every wave has written its pieces ----
    if (wave < nrem) {
        ps_wait(rem_done, W);
        const int ci = F * W + wave;
        const PsChain g = ps_chain<UPS>(a, c0 + ci, Nu);
        const int len = g.u1 - g.u0;
        const int rgr = rg_of(g) - rgA;
        for (int it = lane; it < T * 16; it += 64) {
            const int t = it >> 4, nn = it & 15;
            const float *pp = Part + (size_t)wave * pslot + t * 16 + nn;
            const uint16_t *sp = Sc + ((size_t)rgr * G + g.u0) * 16 + nn;
            float acc0 = 0.0f, acc1 = 0.0f;
            for (int k = 0; k < len; k += 8) {
                float pv[8];
                uint32_t sv[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    pv[q] = pp[(size_t)(k + q) * TP * 16];
                    sv[q] = sp[min(k + q, len - 1) * 16];
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    float &acc = (ALT2 && (q & 1)) ? acc1 : acc0;
                    const float nf = __builtin_fmaf(pv[q], half_bits_to_float((uint16_t)sv[q]), acc);
                    acc = k + q < len ? nf : acc;
                }
            }
            Res[(size_t)ci * TP * 16 + t * 16 + nn] = ALT2 ? acc0 + acc1 : acc0;
        }
        chain_done(ci);
    }

    // ---- outputs ----
    auto wout = [&](int wi, int rl, int t, int nn, float val) {
        const DecodeWeight &Wt = a.w[wi];
        const int M = Wt.M, row = rl * 16 + nn;
        const float v = val * (Tsc[t] * 0.0625f);
        const float out = (ALT2 && Wt.seg_split[0] > 1) ? v + 0.0f : v;
        if (a.y_bf16) static_cast<uint16_t *>(Wt.y)[(size_t)t * M + row] = float_to_bf16(out);
        else static_cast<float *>(Wt.y)[(size_t)t * M + row] = out;
    };
    // A cut row-group: publish this work-group's splits; the last of the
    // work-groups sharing it adds all splits in order and writes the outputs.
    // Device-scope atomic stores and loads bypass the non-coherent caches,
    // and the stores complete before the count.
    auto exchange = [&](int rg) {
        int wi, rl, S, cr0;
        rg_info(rg, wi, rl, S, cr0);
        const int sa = max(c0, cr0) - cr0, sb = min(c1, cr0 + S) - cr0;
        const int slot = ps_wg_of_chain(cr0, a.ps_q, a.ps_r, GW);
        const int nwg = ps_wg_of_chain(cr0 + S - 1, a.ps_q, a.ps_r, GW) - slot + 1;
        float *xs = g_ps_xpart + (size_t)slot * (kPsMaxS * kPsMaxT * 16);
        for (int i = lane; i < (sb - sa) * T * 16; i += 64) {
            const int sl = i / (T * 16), e = i - sl * (T * 16);
            __hip_atomic_store(&xs[(sa + sl) * T * 16 + e],
                               Res[(size_t)(cr0 + sa + sl - c0) * TP * 16 + (e >> 4) * 16 + (e & 15)],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);                 // vmcnt(0): the stores are done
        unsigned old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(&g_ps_xcount[slot * kPsCtrStride], 1u, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if ((int)old == nwg - 1) {
            for (int it = lane; it < T * 16; it += 64) {
                float v = 0.0f;
                for (int s = 0; s < S; ++s)
                    v = v + __hip_atomic_load(&xs[s * T * 16 + it], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wout(wi, rl, it >> 4, it & 15, v);
            }
            if (lane == 0)
                __hip_atomic_store(&g_ps_xcount[slot * kPsCtrStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    if (wave == 0 && nfirst > 0) {
        ps_wait(cnt_first, nfirst);
        exchange(rgA);
    }
    if (wave == 1 && nlast > 0) {
        ps_wait(cnt_last, nlast);
        exchange(rgB);
    }
    lds_sync();

    // ---- the row-groups inside the range: split sums in LDS ----
    for (int x = tid; x < nrg * T * 16; x += kPsThreads) {
        const int rgi = x / (T * 16), it = x - rgi * (T * 16);
        int wi, rl, S, cr0;
        rg_info(rgA + rgi, wi, rl, S, cr0);
        if (cr0 < c0 || cr0 + S > c1) continue;          // cut: exchanged above
        const int t = it >> 4, nn = it & 15;
        float v = 0.0f;
        for (int s = 0; s < S; ++s) v = v + Res[(size_t)(cr0 + s - c0) * TP * 16 + t * 16 + nn];
        wout(wi, rl, t, nn, v);
    }
}

template <int UNIT, bool ALT2, int TP>
static int ps_launch(const DecodeArgs &a, int grid, size_t lds, hipStream_t st) {
    auto k = persist_kernel<UNIT, ALT2, TP>;
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kPsLdsMax) != hipSuccess)
            return -6;
        attr = true;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(kPsThreads), lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

template <int UNIT>
static int ps_tp(const DecodeArgs &a, int tp, int grid, size_t lds, hipStream_t st) {
    const bool alt2 = a.variant == kVarGemv;
    switch (tp) {
    case 1: return alt2 ? ps_launch<UNIT, true, 1>(a, grid, lds, st) : ps_launch<UNIT, false, 1>(a, grid, lds, st);
    case 2: return alt2 ? ps_launch<UNIT, true, 2>(a, grid, lds, st) : ps_launch<UNIT, false, 2>(a, grid, lds, st);
    case 4: return alt2 ? ps_launch<UNIT, true, 4>(a, grid, lds, st) : ps_launch<UNIT, false, 4>(a, grid, lds, st);
    default: return alt2 ? ps_launch<UNIT, true, 8>(a, grid, lds, st) : ps_launch<UNIT, false, 8>(a, grid, lds, st);
    }
}

int launch_persist(DecodeArgs &a, hipStream_t st) {
    // per-token activations and plain FP16 scales: the unit is the group
    if (a.T < 1 || a.T > kPsMaxT || a.block != 0 || a.scale_enc != 0 || a.residual) return 1;
    if (a.group != 64 && a.group != 128) return 1;
    const int unit = a.group, nu = a.K / unit, g = nu;
    long long chains = 0;
    int rgs = 0, smax = 1, smin = kPsMaxS;
    for (int i = 0; i < a.count; ++i) {
        DecodeWeight &w = a.w[i];
        const int S = w.seg_split[0];
        for (int s = 1; s < a.seg_count; ++s)
            if (w.seg_split[s] != S) return 1;
        // every split must own at least one unit
        if (S < 1 || S > kPsMaxS || (S & (S - 1)) || nu < S) return 1;
        w.rg_begin = rgs;
        w.cbeg = (int)chains;
        rgs += w.M / 16;
        chains += (long long)(w.M / 16) * S;
        smax = std::max(smax, S);
        smin = std::min(smin, S);
    }
    if (chains <= 0 || chains > (1LL << 30)) return 1;
    const int tp = a.T <= 1 ? 1 : a.T <= 2 ? 2 : a.T <= 4 ? 4 : 8;
    const int grid = (int)std::min<long long>(std::min(device_cus(), kPsMaxWg), chains);
    // chains per work-group: floor or ceil of chains / grid; the remainder
    // slots, the row-group span and the result buffer follow from it
    const int cmax = (int)((chains + grid - 1) / grid), cmin = (int)(chains / grid);
    const int rslots = std::max(cmax % kPsWaves, cmin % kPsWaves);
    const int nrg_max = (cmax + smin - 1) / smin + 1;
    const int lmax = (nu + smin - 1) / smin;
    const PsLds L = ps_lds(a.T, tp, a.K, g, nrg_max, rslots, lmax, cmax);
    if (L.total > kPsLdsMax) return 1;
    // runs per wave: the whole chains plus the remainder chains its piece
    // (at most ceil(remainder tiles / 16)) can touch; the shortest chain has
    // floor(units / smax / UPS) whole tiles
    {
        const int ups = kTileK / unit;
        const int tmin = std::max(1, nu / smax / ups);
        const int tmax = (nu + smin - 1) / smin / ups + 2;
        const int piece = (rslots * tmax + kPsWaves - 1) / kPsWaves;
        const int runs = cmax / kPsWaves + (piece + tmin - 1) / tmin + 1;
        if (runs > kPsRunMax) return 1;
    }
    // the kernel recomputes the LDS layout from these
    a.ps_smin = smin;
    a.ps_nrg = nrg_max;
    a.ps_rslots = rslots;
    a.ps_cmax = cmax;
    a.ps_q = (int)(chains / grid);
    a.ps_r = (int)(chains % grid);
    a.total_chains = (int)chains;
    if (unit == 128) return ps_tp<128>(a, tp, grid, L.total, st);
    return ps_tp<64>(a, tp, grid, L.total, st);
}

}  // namespace kxw4
