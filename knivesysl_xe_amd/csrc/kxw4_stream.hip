// kxw4_stream.hip — persistent decode kernel for up to 8 tokens in the
// per-token (config) mode: the GEMV (kernels_dpas.cpp:586-675), the fan-out
// GEMV (945-1102) and the batched GEMM at decode sizes (1334-1490).
//
// Work is counted in chains: one chain is one (row-group, split) of one
// weight, the unit of the reference's in-order FP32 accumulation. The chains
// of all weights, in (weight, row-group, split) order, are cut into one
// contiguous range per work-group and the grid is one work-group per CU, so
// every CU streams the same number of weight tiles. A work-group walks its
// range one row-group segment at a time, with two kinds of waves:
//   * 8 streamer waves share a segment's 1 KB weight tiles round-robin (wave
//     w takes tiles w, w+8, ...), so a work-group reads consecutive
//     kilobytes, and write each unit's exact partial (16*P, an integer
//     below 2^24 held in FP32) to LDS.
//     The tiles and the segment's FP16 scales flow through a ring of PF
//     loads per wave that runs across segments; the streamers issue no other
//     global memory operation, so their waits stay partial;
//   * 4 chain waves share each segment: they run the reference chain of
//     every (split, token, row) from LDS, add the splits in split order from
//     0.0f and write the outputs.
// Streamers and chain waves hand segments over through LDS counters (ready,
// released) over three partial buffers, so a chain wave may trail by two
// segments without stalling the stream.
// A row-group whose splits are cut between work-groups (at most one at each
// end of a range) is finished by whichever work-group arrives last: each
// publishes its split partials with device-scope atomic stores to a static
// buffer and bumps a counter; the last adds all splits in order. No
// work-group waits for another. The cut segments are streamed first, so the
// exchange overlaps the rest of the stream.
//
// The activations (T x K int8) are staged into LDS once per work-group with
// direct global->LDS loads; rows are padded by 16 bytes.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace kxw4 {

constexpr int kStWaves = 8;                          // streamer waves
constexpr int kStThreads = 64 * kStWaves;
constexpr int kStChainWaves = 4;                     // chain waves (share each segment)
constexpr int kStXWave = kStWaves + kStChainWaves;   // the exchange wave
constexpr int kStAllThreads = 64 * (kStXWave + 1);
constexpr int kStBuf = 3;                            // partial / scale buffers
constexpr int kStMaxT = 8;
constexpr int kStMaxWg = 256;                        // work-groups (and exchange slots) at most
constexpr int kStMaxS = 16;
constexpr int kStPF = 4;                             // ring depth per streamer wave
constexpr size_t kStLdsMax = 160 * 1024;

// Split partials of row-groups cut between work-groups: slot b belongs to the
// cut row-group whose first chain lies in work-group b. The counters start at
// zero when the library loads and the last arriver puts them back to zero.
// Launches that overlap on one GPU share these and must not run concurrently.
__device__ __attribute__((aligned(256))) float g_st_xpart[kStMaxWg * kStMaxS * kStMaxT * 16];
__device__ unsigned g_st_xcount[kStMaxWg];

struct StSeg {
    int wi;        // weight
    int rl;        // row-group within the weight
    int S;         // the weight's split count
    int sa, sb;    // splits [sa, sb) of the row-group in this segment
    int ka, kb;    // weight tiles [ka, kb)
    int steps;     // ceil((kb - ka) / streamer waves)
    int cr0;       // first chain of the row-group
};

// LDS layout in bytes: activations, partial buffers [unit][TP][16] float,
// scale buffers [group][16] FP16 (both padded by 8 units), two split-partial
// buffers [split][TP][16] float, the split partials of the two cut segments, the
// outputs [segment][TP][16] float, per-token activation scales, hand-off
// counters, dummies.
struct StLds {
    size_t act, part, sc, spart, xcut, tsc, ctl, dummy, total;
};

__host__ __device__ inline StLds stream_lds(int T, int TP, int K, int nu, int g, int smax) {
    StLds L;
    L.act = 0;
    L.part = L.act + (size_t)T * (K + 16);
    L.sc = L.part + (size_t)kStBuf * (nu + 8) * TP * 16 * 4;
    L.spart = L.sc + (size_t)kStBuf * (g + 8) * 16 * 2;
    L.xcut = L.spart + (size_t)2 * smax * TP * 16 * 4;
    L.tsc = L.xcut + (size_t)2 * smax * TP * 16 * 4;
    L.ctl = L.tsc + kStMaxT * 4;
    L.dummy = L.ctl + 16 * 4;
    L.total = L.dummy + 64 * 4;
    return L;
}

__device__ __forceinline__ int st_weight_of_chain(const DecodeArgs &a, int c) {
    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (c >= a.w[i].cbeg) wi = i;
    return wi;
}

// work-group holding chain c when C chains are cut into G ranges
// [floor(b*C/G), floor((b+1)*C/G))
__device__ __forceinline__ int st_wg_of_chain(long long c, long long C, long long G) {
    return (int)(((c + 1) * G - 1) / C);
}

template <int UPS>
__device__ __forceinline__ StSeg st_segment(const DecodeArgs &a, int c0, int c1, int nseg, int o,
                                            int rg0, int Nu) {
    // processing order: the two cut ends first, then the middle
    const int k = (nseg < 2 || o == 0) ? 0 : (o == 1 ? nseg - 1 : o - 1);
    const int R = rg0 + k;
    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if (R >= a.w[i].rg_begin) wi = i;
    const DecodeWeight &W = a.w[wi];
    StSeg g;
    g.wi = wi;
    g.S = W.seg_split[0];
    g.rl = R - W.rg_begin;
    g.cr0 = W.cbeg + g.rl * g.S;
    g.sa = max(c0, g.cr0) - g.cr0;
    g.sb = min(c1, g.cr0 + g.S) - g.cr0;
    const int ls = __builtin_ctz(g.S);
    const int ua = (Nu * g.sa) >> ls, ub = (Nu * g.sb) >> ls;
    g.ka = ua / UPS;
    g.kb = (ub + UPS - 1) / UPS;
    g.steps = (g.kb - g.ka + kStWaves - 1) / kStWaves;
    return g;
}

template <int NSC>
struct StSlot {
    v4u wd;
    v4u sc[NSC];
};

// LDS counters of the hand-offs inside a work-group: relaxed LDS atomics
// behind LDS-only fences, so no wait touches a vector-memory counter.
__device__ __forceinline__ void st_signal(int *ctr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The wait is bounded (about 2^22 polls, far beyond any legitimate wait), so
// a hand-off that never comes ends the kernel with wrong outputs instead of
// holding the GPU.
__device__ __forceinline__ void st_wait(int *ctr, int target) {
    for (int spin = 0; spin < (1 << 22); ++spin) {
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) >= target)
            break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// UNIT = weight group (per-token mode); TP = token rows of a partial buffer
// (T rounded up to 1, 2, 4 or 8), so the chain loop's LDS offsets are
// compile-time constants.
template <int UNIT, bool ALT2, int NSC, int TP>
__global__ __launch_bounds__(kStAllThreads) void stream_kernel(const DecodeArgs a) {
    constexpr int UPS = kTileK / UNIT;
    constexpr int PF = kStPF;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int K = a.K, T = a.T;
    const int NT = K / kTileK, Nu = K / UNIT, G = K / UNIT;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, n = lane & 15, g4 = lane >> 4;

    // ---- this work-group's chain range and its row-group segments ----
    const long long C = a.total_chains, GW = gridDim.x;
    const int c0 = (int)((long long)blockIdx.x * C / GW);
    const int c1 = (int)((long long)(blockIdx.x + 1) * C / GW);
    auto rg_of_chain = [&](int c) {
        const DecodeWeight &W = a.w[st_weight_of_chain(a, c)];
        return W.rg_begin + ((c - W.cbeg) >> __builtin_ctz(W.seg_split[0]));
    };
    const int rg0 = rg_of_chain(c0);
    const int nseg = rg_of_chain(c1 - 1) - rg0 + 1;

    const StLds L = stream_lds(T, TP, K, Nu, G, a.smax);
    int *Pb = reinterpret_cast<int *>(smem + L.part);
    uint16_t *Sb = reinterpret_cast<uint16_t *>(smem + L.sc);
    float *Xb = reinterpret_cast<float *>(smem + L.spart);
    float *Tsc = reinterpret_cast<float *>(smem + L.tsc);
    int *ready = reinterpret_cast<int *>(smem + L.ctl);     // [kStBuf] streamer waves done per buffer use
    int *rel = ready + kStBuf;                               // [kStBuf] chain waves done per buffer use
    int *cut = rel + kStBuf;                                 // [2] cut segment 0 / 1 chained
    int *chained = cut + 2;                                  // [2] chain waves done per split buffer use
    float *Xc = reinterpret_cast<float *>(smem + L.xcut);
    // partial and scale buffers carry 8 units of padding for the chains'
    // last batch
    const int pbuf = (Nu + 8) * TP * 16, sbuf = (G + 8) * 16, xbuf = a.smax * TP * 16;

    // output of segment g (any ordinal) for token t, row nn of its row-group
    auto wout = [&](const StSeg &g, int t, int nn, float val) {
        const DecodeWeight &W = a.w[g.wi];
        const int M = W.M, row = g.rl * 16 + nn;
        const float v = val * (Tsc[t] * 0.0625f);
        const float out = (ALT2 && g.S > 1) ? v + 0.0f : v;
        if (a.y_bf16) static_cast<uint16_t *>(W.y)[(size_t)t * M + row] = float_to_bf16(out);
        else static_cast<float *>(W.y)[(size_t)t * M + row] = out;
    };
    // the two cut ends of the range (segment ordinals 0 and 1)
    auto is_cut = [&](const StSeg &g) { return !(g.sa == 0 && g.sb == g.S); };

    if (wave == kStXWave) {
        // ================= exchange wave =================
        // A row-group cut between work-groups: publish this work-group's
        // splits; the last of the work-groups sharing it adds all splits in
        // order and writes the outputs. Device-scope atomic loads and stores
        // bypass the non-coherent caches; the stores complete before the
        // count.
        lds_sync_after_dma();
        for (int o = 0; o < min(nseg, 2); ++o) {
            const StSeg g = st_segment<UPS>(a, c0, c1, nseg, o, rg0, Nu);
            if (!is_cut(g)) continue;
            st_wait(&cut[o], kStChainWaves);
            const float *X = Xc + o * xbuf;
            const int slot = st_wg_of_chain(g.cr0, C, GW);
            const int nwg = st_wg_of_chain(g.cr0 + g.S - 1, C, GW) - slot + 1;
            float *xs = g_st_xpart + (size_t)slot * (kStMaxS * kStMaxT * 16);
            const int mine = (g.sb - g.sa) * T * 16;
            for (int i = lane; i < mine; i += 64) {
                const int sl = i / (T * 16), e = i - sl * (T * 16);
                __hip_atomic_store(&xs[(g.sa + sl) * T * 16 + e], X[sl * TP * 16 + e], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);                 // vmcnt(0): the stores are done
            unsigned old = 0;
            if (lane == 0)
                old = __hip_atomic_fetch_add(&g_st_xcount[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __builtin_amdgcn_readfirstlane(old);
            if ((int)old != nwg - 1) continue;
            for (int it = lane; it < T * 16; it += 64) {
                float val = 0.0f;
                for (int s = 0; s < g.S; ++s)
                    val = val + __hip_atomic_load(&xs[s * T * 16 + it], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wout(g, it >> 4, it & 15, val);
            }
            if (lane == 0) __hip_atomic_store(&g_st_xcount[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    if (wave >= kStWaves) {
        // ================= chain waves =================
        // Their only global memory operations are output stores (no loads
        // whose results they wait for); cut row-groups go to the exchange
        // wave.
        const int cw = wave - kStWaves;
        if (cw == 0) {
            if (lane < 2 * kStBuf + 4) ready[lane] = 0;
            if (lane < T) Tsc[lane] = a.ascale[lane];
        }
        lds_sync_after_dma();

        for (int go = 0; go < nseg; ++go) {
            const int buf = go % kStBuf;
            const StSeg g = st_segment<UPS>(a, c0, c1, nseg, go, rg0, Nu);
            const bool cutseg = go < 2 && is_cut(g);
            float *X = cutseg ? Xc + go * xbuf : Xb + (go & 1) * xbuf;
            st_wait(&ready[buf], kStWaves * (go / kStBuf + 1));

            // ---- chains: one item per (split, token row, row); the chain
            // waves take interleaved slices of 64 items. Items run over TP
            // token rows (rows past T are skipped), so decoding one is
            // shifts; units run in batches of 8 at constant LDS offsets.
            {
                constexpr int per_split = TP * 16;
                const int items = (g.sb - g.sa) * per_split;
                const int ls = __builtin_ctz(g.S);
                const int lmin = Nu >> ls;                // shortest split, in units
                const int lmax = (Nu + g.S - 1) >> ls;    // longest
                const float *P = reinterpret_cast<const float *>(Pb + buf * pbuf) - g.ka * UPS * TP * 16;
                const uint16_t *Sc = Sb + buf * sbuf;
                for (int it = cw * 64 + lane; it - lane < items; it += kStChainWaves * 64) {
                    const int ic = min(it, items - 1);
                    const int sl = ic / per_split, o = ic % per_split;
                    const int s = g.sa + sl;
                    const int u0 = (Nu * s) >> ls;
                    const int len = ((Nu * (s + 1)) >> ls) - u0;
                    const float *pp = P + u0 * TP * 16 + o;
                    const uint16_t *sp = Sc + u0 * 16 + (o & 15);
                    float acc0 = 0.0f, acc1 = 0.0f;
                    // one batch of 8 units; in the last, units past the
                    // item's split (read from the buffers' padding or the
                    // next split) are not added
                    auto batch = [&](int k, auto pred) {
                        constexpr bool PRED = decltype(pred)::value;
                        float pv[8];
                        uint32_t sv[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            pv[q] = pp[q * TP * 16];
                            sv[q] = sp[q * 16];
                        }
                        pp += 8 * TP * 16;
                        sp += 8 * 16;
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            float &acc = ((q & 1) && ALT2) ? acc1 : acc0;
                            const float f = __builtin_fmaf(pv[q], half_bits_to_float((uint16_t)sv[q]), acc);
                            acc = (!PRED || k + q < len) ? f : acc;
                        }
                    };
                    int k = 0;
                    for (; k + 8 <= lmin; k += 8) batch(k, std::false_type{});
                    if (k < lmax) batch(k, std::true_type{});
                    if (it < items) X[it] = ALT2 ? acc0 + acc1 : acc0;
                }
            }
            // this wave has read the segment's partials and scales, and its
            // splits are in X (every segment counts, cut or not)
            st_signal(&rel[buf]);
            st_signal(&chained[go & 1]);
            // Every chain wave's splits are in X, and every chain wave is past
            // its split sums of two segments back, whose X buffer the next
            // segment rewrites.
            st_wait(&chained[go & 1], kStChainWaves * (go / 2 + 1));
            if (cutseg) {
                st_signal(&cut[go]);
                continue;
            }
            // ordered split sum of this wave's slice of the outputs, written
            // out right away
            for (int it = cw * 64 + lane; it < T * 16; it += kStChainWaves * 64) {
                float val;
                if (g.S == 1) {
                    val = X[it];
                } else {
                    // loads in batches of 4, sums in split order from 0.0f
                    val = 0.0f;
                    for (int s0 = 0; s0 < g.S; s0 += 4) {
                        float v[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] = X[min(s0 + q, g.S - 1) * TP * 16 + it];
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            if (s0 + q < g.S) val = val + v[q];
                    }
                }
                wout(g, it >> 4, it & 15, val);
            }
        }
        return;
    }

    // ================= streamer waves =================
    // stage the activations with direct global->LDS loads
    {
        const int kc = K / 16;
        const int total = T * (kc + 1);
        for (int c = wave * 64; c < total; c += kStThreads) {
            const int x = c + lane;
            if (x < total) {
                const int t = x / (kc + 1), p = x - t * (kc + 1);
                __builtin_amdgcn_global_load_lds(a.q + (size_t)t * K + 16 * min(p, kc - 1),
                                                 (__attribute__((address_space(3))) void *)(smem + L.act + (size_t)c * 16),
                                                 16, 0, 0);
            }
        }
    }

    // Segment geometry for this wave: its first tile, its valid steps (tiles
    // ka + wave + 8m < kb) and the segment's steps. Computed once per
    // segment; the steps themselves only advance pointers, so the streaming
    // loop's scalar work stays small.
    struct Geo {
        int ka, steps, valid;
        const uint8_t *tile;      // this lane's 16 bytes of the wave's first tile
        const v4u *scales;        // the row-group's scale block
    };
    auto geo = [&](int o) {
        const StSeg g = st_segment<UPS>(a, c0, c1, nseg, o, rg0, Nu);
        const DecodeWeight &W = a.w[g.wi];
        Geo r;
        r.ka = g.ka;
        r.steps = g.steps;
        r.valid = max(0, (g.kb - g.ka - wave + kStWaves - 1) / kStWaves);
        const int kt = min(g.ka + wave, g.kb - 1);
        r.tile = W.codes + ((size_t)g.rl * NT + kt) * kTileBytes + lane * 16;
        r.scales = reinterpret_cast<const v4u *>(W.scales + (size_t)g.rl * G * 16);
        return r;
    };

    // The ring: every step issues exactly one tile load (past a wave's valid
    // tiles it re-reads its last one; past the range, the range's last tile),
    // so a ring slot always has PF-1 younger loads behind it.
    StSlot<NSC> ring[PF];
    int lo = 0, lm = 0;
    Geo lg = geo(0);
    const uint8_t *lp = lg.tile;
    auto load = [&](StSlot<NSC> &s) {
        s.wd = *reinterpret_cast<const v4u *>(lp);
        if (lm == 0 && lo < nseg) {
#pragma unroll
            for (int c = 0; c < NSC; ++c) s.sc[c] = lg.scales[min(tid + kStThreads * c, 2 * G - 1)];
        }
        if (++lm < lg.valid) lp += kStWaves * kTileBytes;
        // after the range's last segment lm only grows past valid, so lp
        // stays on that segment's last tile
        if (lm == lg.steps && lo < nseg && ++lo < nseg) {
            lm = 0;
            lg = geo(lo);
            lp = lg.tile;
        }
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PF; ++p) load(ring[p]);
    __builtin_amdgcn_sched_barrier(0);
    // the staging loads were issued before the preload's PF loads
    __builtin_amdgcn_s_waitcnt(0x0F70 | PF);
    lds_sync_after_dma();

    // this lane's MFMA row: token n & 7 (rows 8-15 repeat 0-7, never stored)
    const int ta = min(n & 7, T - 1);
    const int8_t *abase = reinterpret_cast<const int8_t *>(smem + L.act) + (size_t)ta * (K + 16) + 16 * g4;
    float *dummy = reinterpret_cast<float *>(smem + L.dummy) + lane;
    // steps over all segments; the ring runs whole passes, and the steps past
    // the last one only keep issuing (re-)loads, so every path through a pass
    // issues the same loads and the waits stay partial
    int total = 0;
    for (int o = 0; o < nseg; ++o) total += st_segment<UPS>(a, c0, c1, nseg, o, rg0, Nu).steps;
    int po = 0, pm = 0, buf = 0;
    Geo pg = geo(0);
    // this wave's activation operand and partial slots of its current tile
    const int8_t *ap = abase + (size_t)min(pg.ka + wave, NT - 1) * kTileK;
    float *pp = reinterpret_cast<float *>(Pb) + (wave * UPS * TP) * 16 + n;
    for (int ib = 0; ib < total; ib += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const bool live = ib + p < total;
            if (live) {
                // the buffer's previous segment must have been read
                if (pm == 0 && po >= kStBuf) st_wait(&rel[buf], kStChainWaves * (po / kStBuf));
                const bool valid = pm < pg.valid;
                const v4i A0 = *reinterpret_cast<const v4i *>(ap);
                const v4i A1 = *reinterpret_cast<const v4i *>(ap + 64);
                const v4u wd = ring[p].wd;
#pragma unroll
                for (int j = 0; j < UPS; ++j) {
                    const v4i zero = {0, 0, 0, 0};
                    v4i acc;
                    if constexpr (UNIT == 128) {
                        acc = mfma_k64(A0, unpack_k64(wd.x, wd.y), zero);
                        acc = mfma_k64(A1, unpack_k64(wd.z, wd.w), acc);
                    } else if constexpr (UNIT == 64) {
                        acc = j == 0 ? mfma_k64(A0, unpack_k64(wd.x, wd.y), zero)
                                     : mfma_k64(A1, unpack_k64(wd.z, wd.w), zero);
                    } else {
                        const uint32_t d = j == 0 ? wd.x : j == 1 ? wd.y : j == 2 ? wd.z : wd.w;
                        const v4i c = j < 2 ? A0 : A1;
                        const long av = (j & 1) ? (long)(((uint64_t)(uint32_t)c.w << 32) | (uint32_t)c.z)
                                                : (long)(((uint64_t)(uint32_t)c.y << 32) | (uint32_t)c.x);
                        acc = mfma_k32(av, unpack_k32(d), zero);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = 4 * g4 + r;
                        // 16*P is exact in FP32 (|16*P| < 2^24)
                        float *dst = (valid && t < T) ? pp + (j * TP + t) * 16 : dummy;
                        *dst = (float)acc[r];
                    }
                }
                if (pm == 0) {
                    uint16_t *Sc = Sb + buf * sbuf;
#pragma unroll
                    for (int c = 0; c < NSC; ++c) {
                        const int x = tid + kStThreads * c;
                        if (x < 2 * G) reinterpret_cast<v4u *>(Sc)[x] = ring[p].sc[c];
                    }
                }
                if (++pm < pg.valid) {
                    ap += kStWaves * kTileK;
                    pp += kStWaves * UPS * TP * 16;
                }
                if (pm == pg.steps) {
                    st_signal(&ready[buf]);
                    pm = 0;
                    if (++po < nseg) {
                        buf = po % kStBuf;
                        pg = geo(po);
                        ap = abase + (size_t)min(pg.ka + wave, NT - 1) * kTileK;
                        pp = reinterpret_cast<float *>(Pb + buf * pbuf) + (wave * UPS * TP) * 16 + n;
                    }
                }
            }
            load(ring[p]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Drain the ring's last (re-)loads: the compiler joins this exit with the
    // other waves' paths, which must not inherit pending loads.
    __builtin_amdgcn_s_waitcnt(0);
}

template <int UNIT, bool ALT2, int NSC, int TP>
static int st_launch(const DecodeArgs &a, int grid, size_t lds, hipStream_t st) {
    auto k = stream_kernel<UNIT, ALT2, NSC, TP>;
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kStLdsMax) != hipSuccess)
            return -6;
        attr = true;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(kStAllThreads), lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

template <int UNIT, int NSC>
static int st_tp(const DecodeArgs &a, int tp, int grid, size_t lds, hipStream_t st) {
    const bool alt2 = a.variant == kVarGemv;
    switch (tp) {
    case 1: return alt2 ? st_launch<UNIT, true, NSC, 1>(a, grid, lds, st) : st_launch<UNIT, false, NSC, 1>(a, grid, lds, st);
    case 2: return alt2 ? st_launch<UNIT, true, NSC, 2>(a, grid, lds, st) : st_launch<UNIT, false, NSC, 2>(a, grid, lds, st);
    case 4: return alt2 ? st_launch<UNIT, true, NSC, 4>(a, grid, lds, st) : st_launch<UNIT, false, NSC, 4>(a, grid, lds, st);
    default: return alt2 ? st_launch<UNIT, true, NSC, 8>(a, grid, lds, st) : st_launch<UNIT, false, NSC, 8>(a, grid, lds, st);
    }
}

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kStMaxWg;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = kStMaxWg;
        cus[dev] = n;
    }
    return cus[dev];
}

int launch_stream(DecodeArgs &a, hipStream_t st) {
    // per-token activations and plain FP16 scales: the unit is the group
    if (a.T < 1 || a.T > kStMaxT || a.block != 0 || a.scale_enc != 0 || a.residual) return 1;
    const int unit = a.group, nu = a.K / unit, g = nu;
    // the scale block of a row-group rides in the ring: NSC 16-byte chunks
    // per streamer lane, one per unit size
    const int nsc = unit == 128 ? 1 : unit == 64 ? 2 : 3;
    if (2 * g > nsc * kStThreads) return 1;
    long long chains = 0;
    int rgs = 0, smax = 1;
    for (int i = 0; i < a.count; ++i) {
        DecodeWeight &w = a.w[i];
        const int S = w.seg_split[0];
        for (int s = 1; s < a.seg_count; ++s)
            if (w.seg_split[s] != S) return 1;
        // every split must own at least one unit
        if (S < 1 || S > kStMaxS || (S & (S - 1)) || nu < S) return 1;
        w.rg_begin = rgs;
        w.cbeg = (int)chains;
        rgs += w.M / 16;
        chains += (long long)(w.M / 16) * S;
        smax = std::max(smax, S);
    }
    if (chains <= 0 || chains > (1LL << 30)) return 1;
    const int tp = a.T <= 1 ? 1 : a.T <= 2 ? 2 : a.T <= 4 ? 4 : 8;
    const int grid = (int)std::min<long long>(std::min(device_cus(), kStMaxWg), chains);
    const StLds L = stream_lds(a.T, tp, a.K, nu, g, smax);
    if (L.total > kStLdsMax) return 1;
    a.smax = smax;
    a.total_rg = rgs;
    a.total_chains = (int)chains;
    if (unit == 128) return st_tp<128, 1>(a, tp, grid, L.total, st);
    if (unit == 64) return st_tp<64, 2>(a, tp, grid, L.total, st);
    return st_tp<32, 3>(a, tp, grid, L.total, st);
}

}  // namespace kxw4
