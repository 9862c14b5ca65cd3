// kxw4_decode.hip — decode-shaped projections (T <= 64 tokens): the GEMV
// (kernels_dpas.cpp:586-675), the fan-out GEMV (945-1102) and the batched /
// packed GEMM at small T (1334-1490).
//
// The integer work and the float chain are decoupled:
//   * a work-group owns one 16-row row-group (and a slice of at most `ts`
//     tokens). Its 8 waves stream the row-group's 128-K weight tiles -- wave
//     w takes tiles w, w+8, w+16, ..., so the waves read consecutive
//     kilobytes -- through a ring of PFW tiles in flight per wave. The
//     streaming loop is one basic block: ring loads, nibble unpack, int8
//     MFMAs, LDS stores of each unit's exact 16*P (predicates are address
//     selects into a dummy word), so the memory waits stay partial;
//   * the row-group's FP16 scales are staged into LDS once per work-group;
//     for T <= 8 one 16-byte activation load per lane and tile carries both
//     64-K chunks (lanes 8-15 fetch the second) and a DPP row rotate
//     rebuilds the MFMA operands, so a tile costs two vector-memory
//     instructions instead of four (the address units were the bottleneck);
//   * after a barrier, every (output, split) pair runs the reference chain
//     of its split over the units [Nu*s/S, Nu*(s+1)/S): two alternating
//     accumulators (GEMV) or one (fan-out, GEMM), as independent lanes;
//   * after a second barrier one lane per output adds the split partials in
//     split order starting from 0.0f (S == 1 stores the chain directly) and
//     writes the result. S is per token, so packed segments with different
//     plans share one launch.
// Parallelism does not depend on the split plan: every row-group is one
// work-group whatever S is. The token slice bounds the LDS one row-group's
// partials need.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

#include <algorithm>

namespace kxw4 {

constexpr int kDcWaves = 8;
constexpr int kDcThreads = 64 * kDcWaves;
constexpr int kChainBatch = 8;     // units whose LDS reads a chain issues together
constexpr int kScaleChunks = 3;    // 16-byte scale chunks a thread stages (G*2 <= 3*512)

// AT: activation tiling. 0 = up to 8 tokens, one load per tile carrying both
// chunks; 1, 2, 4 = that many 16-token MFMA row blocks, one load per chunk.
template <int AT>
struct DcStage {
    v4u wd;
    v4i A[AT == 0 ? 1 : 2 * AT];
};

// LDS words: partials [nu][tl][16] int32, scales [g][16] uint16, split
// partials [smax][tl][16] float, in the general mode the activation scale and
// code sum [nu][tl], then 64 dummy words.
__host__ __device__ inline int decode_lds_words(int nu, int g, int tl, int smax, bool side) {
    return nu * tl * 16 + g * 8 + smax * tl * 16 + (side ? 2 * nu * tl : 0) + 64;
}

template <int AT, int UNIT, int MODE, bool DEBUG, int PFW>
__global__ __launch_bounds__(kDcThreads) void decode_kernel(const DecodeArgs a) {
    constexpr int UPS = kTileK / UNIT;
    constexpr int TB = AT == 0 ? 1 : AT;                  // 16-token MFMA row blocks
    extern __shared__ int lds[];

    int wi = 0;
    for (int i = 1; i < a.count; ++i)
        if ((int)blockIdx.x >= a.w[i].rg_begin) wi = i;
    const DecodeWeight &W = a.w[wi];
    const int rg = (int)blockIdx.x - W.rg_begin;
    const int t0 = (int)blockIdx.y * a.ts;                 // first token of this slice
    const int TL = min(a.ts, a.T - t0);                    // tokens in this slice
    const int K = a.K, M = W.M;
    const int NT = K / kTileK, Nu = K / UNIT, G = K / a.group;
    const int gsh = __builtin_ctz(a.group / UNIT);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, n = lane & 15, g4 = lane >> 4;
    const int ntw = NT > wave ? (NT - wave + kDcWaves - 1) / kDcWaves : 0;   // tiles of this wave
    const bool ref_block = a.block == 32;
    const bool zp = a.scale_enc == 1;
    const int SMAX = a.smax;

    int *P = lds;
    uint16_t *S = reinterpret_cast<uint16_t *>(lds + Nu * TL * 16);
    float *Part = reinterpret_cast<float *>(lds + Nu * TL * 16 + G * 8);
    float *Asc = Part + SMAX * TL * 16;
    int *Zs = reinterpret_cast<int *>(Asc + Nu * TL);
    // Stores of an invalid position (or of rows past the slice) go to this
    // lane's dummy word: address selects, not branches.
    int *dummy = lds + decode_lds_words(Nu, G, TL, SMAX, MODE != 0) - 64 + lane;

    // ---- scale staging: the row-group's [G][16] FP16 block, issued first ----
    const v4u *sglob = reinterpret_cast<const v4u *>(W.scales + (size_t)rg * G * 16);
    v4u sreg[kScaleChunks];
#pragma unroll
    for (int c = 0; c < kScaleChunks; ++c)
        sreg[c] = sglob[min((int)threadIdx.x + kDcThreads * c, 2 * G - 1)];

    // The output phase's per-token scale and residual of this thread's (at
    // most two) outputs, loaded now: read after the split sum they add a
    // dependent memory round trip at the end of the launch.
    float tsc_pre[2] = {1.0f, 1.0f}, rsd_pre[2] = {0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int o = (int)threadIdx.x + kDcThreads * k;
        if (o < TL * 16) {
            const int t = t0 + (o >> 4);
            if (a.block == 0) tsc_pre[k] = a.ascale[t];
            if (a.residual) rsd_pre[k] = a.residual[(size_t)t * M + rg * 16 + (o & 15)];
        }
    }

    const uint8_t *wbase = W.codes + (size_t)rg * NT * kTileBytes + lane * 16;
    // Activation rows. MFMA rows are independent: a row past the slice reads
    // a valid token and is never stored, so no lane predicate on the loads.
    const int8_t *abase[TB];
    if constexpr (AT == 0) {
        const int t = n & 7;
        abase[0] = a.q + (size_t)(t0 + (t < TL ? t : TL - 1)) * K + 16 * g4 + (n >> 3) * 64;
    } else {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const int t = tb * 16 + n;
            abase[tb] = a.q + (size_t)(t0 + (t < TL ? t : TL - 1)) * K + 16 * g4;
        }
    }

    auto load = [&](DcStage<AT> &s, int i) {
        const int kb = wave + kDcWaves * i;
        s.wd = *reinterpret_cast<const v4u *>(wbase + (size_t)kb * kTileBytes);
        if constexpr (AT == 0) {
            s.A[0] = *reinterpret_cast<const v4i *>(abase[0] + (size_t)kb * kTileK);
        } else {
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                s.A[2 * tb] = *reinterpret_cast<const v4i *>(abase[tb] + (size_t)kb * kTileK);
                s.A[2 * tb + 1] = *reinterpret_cast<const v4i *>(abase[tb] + (size_t)kb * kTileK + 64);
            }
        }
    };

    auto mfma_store = [&](const DcStage<AT> &s, int i, bool valid) {
        const int kb = wave + kDcWaves * i;
        v4i A[TB][2];
        if constexpr (AT == 0) {
            A[0][0] = s.A[0];
            A[0][1] = rotate8(s.A[0]);
        } else {
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                A[tb][0] = s.A[2 * tb];
                A[tb][1] = s.A[2 * tb + 1];
            }
        }
#pragma unroll
        for (int j = 0; j < UPS; ++j) {
            v4i acc[TB];
            const v4i zero = {0, 0, 0, 0};
            if constexpr (UNIT == 128) {
                const v4i b0 = unpack_k64(s.wd.x, s.wd.y), b1 = unpack_k64(s.wd.z, s.wd.w);
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    acc[tb] = mfma_k64(A[tb][0], b0, zero);
                    acc[tb] = mfma_k64(A[tb][1], b1, acc[tb]);
                }
            } else if constexpr (UNIT == 64) {
                const v4i bb = j == 0 ? unpack_k64(s.wd.x, s.wd.y) : unpack_k64(s.wd.z, s.wd.w);
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) acc[tb] = mfma_k64(A[tb][j], bb, zero);
            } else {
                const uint32_t d = j == 0 ? s.wd.x : j == 1 ? s.wd.y : j == 2 ? s.wd.z : s.wd.w;
                const long bb = unpack_k32(d);
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    const v4i cc = A[tb][j >> 1];
                    const long av = (j & 1) ? (long)(((uint64_t)(uint32_t)cc.w << 32) | (uint32_t)cc.z)
                                            : (long)(((uint64_t)(uint32_t)cc.y << 32) | (uint32_t)cc.x);
                    acc[tb] = mfma_k32(av, bb, zero);
                }
            }
            const int u = kb * UPS + j;
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = tb * 16 + 4 * g4 + r;
                    int *dst = (valid && t < TL) ? &P[(u * TL + t) * 16 + n] : dummy;
                    *dst = acc[tb][r];
                }
        }
    };

    // ---- phase 1: stream the row-group through the ring ----
    if (ntw > 0) {
        DcStage<AT> st[PFW];
#pragma unroll
        for (int s = 0; s < PFW; ++s) load(st[s], min(s, ntw - 1));
        // The trip count is padded to whole rings and positions past the
        // wave's tiles redo its last tile into the dummy word, so the loop
        // body is one basic block and the memory waits stay partial.
        for (int ib = 0; ib < ntw; ib += PFW) {
#pragma unroll
            for (int s = 0; s < PFW; ++s) {
                const int i = ib + s;
                mfma_store(st[s], min(i, ntw - 1), i < ntw);
                load(st[s], min(i + PFW, ntw - 1));
            }
        }
    }
#pragma unroll
    for (int c = 0; c < kScaleChunks; ++c) {
        const int x = (int)threadIdx.x + kDcThreads * c;
        if (x < 2 * G) reinterpret_cast<v4u *>(S)[x] = sreg[c];
    }
    // general mode: per-unit activation scale and code sums of the slice
    if (MODE != 0) {
        for (int x = threadIdx.x; x < Nu * TL; x += kDcThreads) {
            const int u = x / TL, tl = x - u * TL, tg = t0 + tl;
            if (ref_block) Asc[x] = a.ascale[(size_t)tg * (K / 32) + u];
            if (zp) {
                int sm = 0;
                for (int q = (u * UNIT) / 32; q < ((u + 1) * UNIT) / 32; ++q)
                    sm += a.asum[(size_t)tg * (K / 32) + q];
                Zs[x] = sm;
            }
        }
    }
    __syncthreads();

    // split count of slice token tl (its packed segment's plan). With one
    // segment it is a scalar, read once and made opaque: a per-lane segment
    // index into the kernel arguments is a vector memory load, and its wait
    // after the stream adds a memory round trip to the launch.
    int split1 = W.seg_split[0];
    asm volatile("" : "+s"(split1));
    auto split_of = [&](int tl) {
        if (a.seg_count == 1) return split1;
        const int tg = t0 + tl;
        int seg = 0;
        while (seg + 1 < a.seg_count && tg >= a.seg_end[seg]) ++seg;
        return W.seg_split[seg];
    };

    // ---- phase 2: one chain per (split, output): units [Nu*s/S, Nu*(s+1)/S) ----
    const bool alt2 = a.variant == kVarGemv;
    const int items = SMAX * TL * 16;
    for (int it = threadIdx.x; it < items; it += kDcThreads) {
        const int s = it / (TL * 16), o = it - s * (TL * 16);
        const int tl = o >> 4, nn = o & 15;
        const int Sp = split_of(tl);
        if (s >= Sp) continue;
        const int u0 = Nu * s / Sp, u1 = Nu * (s + 1) / Sp;
        float acc0 = 0.0f, acc1 = 0.0f;
        for (int ub = u0; ub < u1; ub += kChainBatch) {
            int pv[kChainBatch], zv[kChainBatch];
            uint32_t sv[kChainBatch];
            float av[kChainBatch];
#pragma unroll
            for (int q = 0; q < kChainBatch; ++q) {
                const int x = ub + q < u1 ? ub + q : u1 - 1;
                pv[q] = P[(x * TL + tl) * 16 + nn];
                sv[q] = S[(x >> gsh) * 16 + nn];
                av[q] = (MODE != 0 && ref_block) ? Asc[x * TL + tl] : 1.0f;
                zv[q] = (MODE != 0 && zp) ? Zs[x * TL + tl] : 0;
            }
            // unit ub+q sits at offset (ub-u0)+q from the split start, and
            // ub-u0 is a multiple of the (even) batch, so the GEMV's
            // alternating accumulator is fixed by q's parity
#pragma unroll
            for (int q = 0; q < kChainBatch; ++q) {
                if (ub + q >= u1) break;
                int p = pv[q];
                float w;
                if (MODE == 0) {
                    w = half_bits_to_float((uint16_t)sv[q]);
                } else {
                    w = half_bits_to_float(zp ? (uint16_t)(sv[q] & 0xFFF0u) : (uint16_t)sv[q]);
                    if (zp) p -= (sext4(sv[q]) * zv[q]) << 4;
                    if (DEBUG) a.dbg[((size_t)(t0 + tl) * M + rg * 16 + nn) * Nu + ub + q] = p >> 4;
                }
                const float pf = (float)p;
                auto step = [&](float acc) {
                    if (MODE == 0 || !ref_block) return __builtin_fmaf(pf, w, acc);
                    if (a.variant == kVarGemm) return __builtin_fmaf(pf, w * av[q], acc);
                    return __builtin_fmaf(pf * w, av[q], acc);
                };
                if ((q & 1) && alt2) acc1 = step(acc1);
                else acc0 = step(acc0);
            }
        }
        Part[(s * TL + tl) * 16 + nn] = alt2 ? acc0 + acc1 : acc0;
    }
    __syncthreads();
    if (DEBUG) return;

    // ---- phase 3: ordered split sum and output, one lane per output ----
    static_assert(kDcThreads * 2 >= 64 * 16, "at most two outputs per thread (T <= 64)");
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int o = (int)threadIdx.x + kDcThreads * k;
        if (o >= TL * 16) break;
        const int tl = o >> 4, nn = o & 15;
        const int Sp = split_of(tl);
        float val;
        if (Sp == 1) {
            val = Part[tl * 16 + nn];
        } else {
            val = 0.0f;
            for (int s = 0; s < Sp; ++s) val = val + Part[(s * TL + tl) * 16 + nn];
        }
        const int t = t0 + tl, row = rg * 16 + nn;
        const float v = a.block == 0 ? val * (tsc_pre[k] * 0.0625f) : val * 0.0625f;
        float out;
        if (a.residual) out = v + rsd_pre[k];
        else if (alt2 && Sp > 1) out = v + 0.0f;
        else out = v;
        if (a.y_bf16) static_cast<uint16_t *>(W.y)[(size_t)t * M + row] = float_to_bf16(out);
        else static_cast<float *>(W.y)[(size_t)t * M + row] = out;
    }
}

template <int AT, int UNIT, int MODE, bool DEBUG, int PFW>
static int launch_one(const DecodeArgs &a, dim3 grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((decode_kernel<AT, UNIT, MODE, DEBUG, PFW>), grid, dim3(kDcThreads), lds, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

template <int AT, int UNIT>
static int launch_dc(const DecodeArgs &a, int mode, bool debug, dim3 grid, size_t lds,
                     hipStream_t st) {
    constexpr int PFW = AT <= 1 ? 4 : AT == 2 ? 2 : 1;
    if (debug) return launch_one<AT, UNIT, 1, true, PFW>(a, grid, lds, st);
    if (mode == 0) return launch_one<AT, UNIT, 0, false, PFW>(a, grid, lds, st);
    return launch_one<AT, UNIT, 1, false, PFW>(a, grid, lds, st);
}

template <int AT>
static int launch_dc_unit(const DecodeArgs &a, int unit, int mode, bool debug, dim3 grid,
                          size_t lds, hipStream_t st) {
    if (unit == 128) return launch_dc<AT, 128>(a, mode, debug, grid, lds, st);
    if (unit == 64) return launch_dc<AT, 64>(a, mode, debug, grid, lds, st);
    return launch_dc<AT, 32>(a, mode, debug, grid, lds, st);
}

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

int launch_decode(DecodeArgs &a, bool debug, hipStream_t st) {
    // Up to 16 tokens go to the row-wave kernel, the rest stay here. The
    // decode_kernel option forces the K-parallel kernel (kparallel) or
    // prefers the row-wave kernel (rowwave); the tests use both to cover
    // every kernel at the decode shapes.
    // W8 and K16 weights run on the row-wave kernel only; 1 hands the shape
    // back to the caller (the GEMM path for W8)
    if (a.w8 || a.group == 16) return debug ? 1 : launch_rowwave(a, st);
    const int force = options().decode_kernel;
    bool no_rowwave = force == kDecodeKParallel;
    // Per-token weights with at most 8 tokens and no more row-groups than
    // CUs stay here: one work-group per row-group whose waves read
    // consecutive kilobytes beats the row-wave kernel's per-split streams
    // when every CU holds at most one row-group (T = 4: 5.5 against 6.4 us
    // at M = K = 4096) -- except for one or two tokens with at most 8 splits
    // of at most 8 tiles each, where the row-wave kernel's short chains and
    // single ring win (cfg0: 5.3 against 5.4 us; K = 2048: 4.6 against 5.0).
    if (force != kDecodeRowwave && a.block == 0 && a.scale_enc == 0 && a.T <= 8) {
        int rgs = 0;
        for (int i = 0; i < a.count; ++i) rgs += a.w[i].M / 16;
        const int S = a.w[0].seg_split[0];
        const bool short_rowwave = a.T <= 2 && S <= 8 && (a.K / kTileK) <= 8 * S;
        if (rgs <= device_cus() && !short_rowwave) no_rowwave = true;
    }
    if (!debug && !no_rowwave) {
        const int r = launch_rowwave(a, st);
        if (r != 1) return r;
    }
    constexpr size_t kBudget = 64 * 1024;
    const int unit = a.block == 32 ? 32 : a.group;
    const int nu = a.K / unit, g = a.K / a.group;
    if (2 * g > kScaleChunks * kDcThreads) return -2;
    const int mode = (a.block == 0 && a.scale_enc == 0) ? 0 : 1;
    const bool side = mode != 0 || debug;
    int smax = 1;
    for (int i = 0; i < a.count; ++i)
        for (int s = 0; s < a.seg_count; ++s) smax = std::max(smax, a.w[i].seg_split[s]);
    a.smax = smax;
    // token slice: the largest (at most 64) whose partials fit in LDS
    auto bytes = [&](int ts) { return (size_t)4 * decode_lds_words(nu, g, ts, smax, side); };
    int ts = a.T < 64 ? a.T : 64;
    while (ts > 1 && bytes(ts) > kBudget) ts = (ts + 1) / 2;
    if (bytes(ts) > kBudget) return -2;
    a.ts = ts;
    int rgs = 0;
    for (int i = 0; i < a.count; ++i) {
        a.w[i].rg_begin = rgs;
        rgs += a.w[i].M / 16;
    }
    a.total_rg = rgs;
    const dim3 grid(rgs, (a.T + ts - 1) / ts);
    const size_t lds = bytes(ts);
    if (ts <= 8) return launch_dc_unit<0>(a, unit, mode, debug, grid, lds, st);
    if (ts <= 16) return launch_dc_unit<1>(a, unit, mode, debug, grid, lds, st);
    if (ts <= 32) return launch_dc_unit<2>(a, unit, mode, debug, grid, lds, st);
    return launch_dc_unit<4>(a, unit, mode, debug, grid, lds, st);
}

}  // namespace kxw4
