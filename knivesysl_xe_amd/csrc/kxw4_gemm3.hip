// kxw4_gemm3.hip — prefill projections in the per-token mode (the BASELINE
// configurations) on the 32x32x32 int8 MFMA: x_gemm_w4a8 / gemm_rc16
// arithmetic (kernels_dpas.cpp:1255-1332, 1334-1490) with one split per
// token.
//
// Cost model (measured on the MI355X): the FP32 chain needs one int->float
// conversion and one FMA per output and weight group. A 32x32 block's four
// 32x32x32 MFMAs over a 128-K step take ~131 cycles of the matrix core and
// its 32 chain instructions per lane ~70 cycles of the VALU, and a SIMD
// overlaps the two only partly: interleaved in one wave they take the sum
// (~217 cycles), in two or four waves per SIMD ~190 and ~174. Per 32x32
// block the 16x16x64 MFMA is 13-18% slower still (it needs twice the operand
// bytes per MAC and leaves fewer issue slots). The kernel is therefore
// bound by issuing the chain beside the MFMAs, and it is laid out to keep
// both busy and to add little else:
//   * each wave owns a 32*TA token x 32*TB row tile of 32x32 blocks; a block
//     is four dependent MFMAs over a 128-K step followed by its 16 chain
//     updates per lane, and the scheduler overlaps one block's updates with
//     the next block's MFMAs;
//   * the unpacked weight operands of a step stay in registers, the
//     activation operands stream one 32-token block at a time;
//   * the work-group is WMW x WNW waves; a wave unpacks the packed weight
//     tiles of its own row blocks;
//   * per 128-K step the activation tile, the packed weight tiles and the
//     FP16 scales reach LDS through buffer loads straight into LDS, into a
//     ring of NST stages; every wave issues the same number of loads per
//     stage, so one vmcnt retires a stage, and one barrier per step both
//     publishes the next stage and frees the one refilled next;
//   * the pipeline runs across steps: the barrier sits before a step's last
//     block, the next step's first operands are read during that block, and
//     the last block's updates run under the next step's first MFMAs, so no
//     step starts or ends with the matrix core idle.
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
#include <utility>

namespace kxw4 {

constexpr int kG3GroupTT = 4;      // token tiles per raster group (option gemm3_raster)

#define KXW4_G3_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// Word 3 of a buffer descriptor for untyped loads: data format 32 (a zero
// format reads zeros), no swizzle, no index.
constexpr int kBufWord3 = 0x00020000;

// XB = 1: one more 32-row block column after the waves' own columns, of
// which each wave takes one 32x32 block (token block wn of its own token
// range; needs TA == WNW and TB == 1)
template <int TA, int TB, int WMW, int WNW, int UNIT, int XB = 0>
struct G3Shape {
    static constexpr int NW = WMW * WNW;
    static constexpr int NTH = 64 * NW;
    static constexpr int BM = WMW * 32 * TA;             // tokens per tile
    static constexpr int BNG = WNW * 2 * TB + 2 * XB;    // row-groups per tile
    static_assert(XB == 0 || (XB == 1 && TA == WNW && TB == 1), "extra column: one block per wave");
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

// f(integral_constant<int, I>) for each I of the sequence, in order
template <class F, int... I>
__device__ __forceinline__ void for_each_index(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}

// OCC: waves per SIMD the register budget is sized for
template <int TA, int TB, int WMW, int WNW, int UNIT, int NST, int OCC, int XB>
__global__ __launch_bounds__(64 * WMW * WNW)
__attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm3_kernel(const GemmArgs a) {
    using S = G3Shape<TA, TB, WMW, WNW, UNIT, XB>;
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
    const int GTT = a.raster_tt;
    const int group = L / (GTT * nnt);
    const int first = group * GTT;
    const int gsz = min(ntt - first, GTT);
    const int within = L % (GTT * nnt);
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

    // ---- load issue: buffer loads straight into LDS. A wave fills whole
    // 1 KB chunks, so the rows of each of its loads are the same for every
    // lane: a buffer descriptor per load holds the first row and the bytes of
    // the rows that exist, and rows past T (activations) or M (weights) read
    // as zero through the descriptor's range check (they are never stored).
    // The lane part of each offset is one 32-bit VGPR per kind of load, the K
    // step goes in the scalar offset (the launcher keeps T*K and M*K/2 below
    // 2^31). Activation chunk ch holds tile rows 8ch..8ch+7: lane l fills
    // row 8ch + 2(l/16) + (l/8)%2, 16-byte chunk (l%8) ^ ((4ch + l/16) % 8):
    // an odd chunk's lane offset is an even chunk's with byte bit 6 flipped.
    // With an even wave count a wave's chunks all have the wave's parity ----
    static_assert(S::A_CHUNKS % 2 == 0, "chunk parity follows the wave and load index");
    // Lane parts of the offsets: activations, weights, and scale granule
    // gi = (j * UPS + u) * 2 + half of this wave's slice (a slice never
    // wraps; row-groups past M repeat the last one).
    auto lane_offsets = [&](int ln, uint32_t &al, uint32_t &bl, uint32_t &so) {
        const int par = NW % 2 == 0 ? (wave & 1) : 0;
        al = (uint32_t)(2 * (ln >> 4) + ((ln >> 3) & 1)) * K +
             (uint32_t)(((ln & 7) ^ ((4 * par + (ln >> 4)) & 7)) * 16);
        bl = ln * 16;
        const int gi = (wave * S::S_LANES) % S::S_TOTAL + min(ln, S::S_LANES - 1);
        const int j = gi / (2 * UPS), u = (gi >> 1) % UPS, half = gi & 1;
        const int rg = min(rg0 + j, RG - 1);
        so = (((uint32_t)rg * G + u) * 16 + half * 8) * 2;
    };
    // With three waves per SIMD and more than one block per wave the
    // registers are short: the lane parts are recomputed at each issue
    // instead of held across the K loop.
    constexpr bool kLaneRecompute = OCC >= 3 && TA * TB > 1;
    uint32_t a_lane0 = 0, b_lane0 = 0, soff0 = 0;
    if constexpr (!kLaneRecompute) lane_offsets(lane, a_lane0, b_lane0, soff0);
    // The descriptors are built at each issue from scalars (a few SALU
    // operations): held in arrays, of descriptors or of their base pointers,
    // they make the host compilation pass drop the kernel without a
    // diagnostic. The base pointers are pinned in SGPRs, or the compiler
    // reloads them from the kernel arguments at every issue, and a pending
    // scalar load turns every LDS wait in the loop into lgkmcnt(0).
    const int8_t *qg = a.q;
    const uint8_t *cg = W.codes;
    const uint16_t *sg = W.scales;
    asm volatile("" : "+s"(qg), "+s"(cg), "+s"(sg));
    auto issue = [&](int kb, int st) {
        uint32_t a_lane = a_lane0, b_lane = b_lane0, soff = soff0;
        if constexpr (kLaneRecompute) {
            int ln = lane;
            asm volatile("" : "+v"(ln));          // (not loop-invariant, so not hoisted)
            lane_offsets(ln, a_lane, b_lane, soff);
        }
        uint8_t *base = smem + st * STAGE;
#pragma unroll
        for (int i = 0; i < S::A_LOADS; ++i) {
            const int r = t0 + 8 * ((wave + NW * i) % S::A_CHUNKS);
            // (computed outside the builtin's argument list: inside it, this
            // expression also makes the host pass drop the kernel)
            const uint32_t al = NW % 2 == 0 ? a_lane : a_lane ^ (64u * (((wave + NW * i) % S::A_CHUNKS) & 1));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                __builtin_amdgcn_make_buffer_rsrc((void *)(qg + (size_t)min(r, T - 1) * K), 0, max(T - r, 0) * K, kBufWord3),
                KXW4_G3_LDS(base + ((wave + NW * i) % S::A_CHUNKS) * 1024),
                16, al, kb * kTileK, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < S::B_LOADS; ++i) {
            const int rg = rg0 + (wave + NW * i) % BNG;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                __builtin_amdgcn_make_buffer_rsrc((void *)(cg + (size_t)min(rg, RG - 1) * NT * kTileBytes), 0,
                                                  rg < RG ? NT * kTileBytes : 0, kBufWord3),
                KXW4_G3_LDS(base + A_BYTES + ((wave + NW * i) % BNG) * 1024),
                16, b_lane, kb * kTileBytes, 0, 0);
        }
        // lanes past the wave's granules are masked off; the load still
        // counts once in vmcnt
        if (lane < S::S_LANES)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(__builtin_amdgcn_make_buffer_rsrc((void *)sg, 0, RG * G * 32, kBufWord3),
                                                     KXW4_G3_LDS(base + A_BYTES + B_BYTES + (wave * S::S_LANES) % S::S_TOTAL * 16),
                                                     16, soff, kb * UPS * 32, 0, 0);
        // with the first stage, the tile's token scales (64 per wave); the
        // later stages' loads are all younger, so the first wait retires it
        // (the DMA builtin takes a generic void pointer: with a typed pointer
        // the host compilation pass drops the kernel without a diagnostic)
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
    // extra column (XB): byte distances from this wave's weight and scale
    // offsets to the extra column's, and the activation offset of its token
    // block (wave-uniform)
    const int dxb = (WNW - wn) * 2 * TB * kTileBytes;
    const int dxs = (WNW - wn) * 2 * TB * UPS * 32;
    const int dxa = wn * 4096;
    // the same offsets inside the current step's stage, moved on each step
    // (so a read needs no address arithmetic)
    int ast[4], bst = boff, sst = soff_lds;
#pragma unroll
    for (int c = 0; c < 4; ++c) ast[c] = aoff[c];

    float f[TA][TB][16], fx[16];
#pragma unroll
    for (int i = 0; i < TA; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) f[i][j][r] = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) fx[r] = 0.0f;

    // Ring of NST stages; step k's loads go to stage k % NST. A wave reaches
    // arrive(k) just before the last 32x32 block of step k - 1 (before the
    // loop for k = 0): vmcnt retires its own loads of step k (those of the
    // stages issued after it may stay in flight), lgkmcnt(0) completes its
    // reads of step k - 1, whose operands are all in registers by then, and
    // the barrier makes both hold for every wave. Step k - 1's stage is then
    // free and takes step k - 1 + NST; the first operands of step k are read
    // while the last block of step k - 1 runs.
    static_assert(NST >= 2 && NST <= 4, "two to four stages");
    constexpr int LD = S::LOADS;
    static_assert(LD * (NST - 2) <= 63, "vmcnt field");
    auto arrive = [&](int k) {
        const int later = min(NST - 2, NT - 1 - k);
        if (NST >= 4 && later >= 2) KXW4_WAIT_VMCNT(2 * LD);
        else if (NST >= 3 && later >= 1) KXW4_WAIT_VMCNT(LD);
        else KXW4_WAIT_VMCNT(0);
        lds_sync_after_dma();
    };
    // operand reads from a stage (block jb's packed weight dwords, MFMA
    // c = 2h + half; its FP16 group scales; token block ib's activations)
    // (d: 0 for the current stage, else the byte distance to the next)
    auto read_b = [&](int d, int jb, v4u (&wd)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
            wd[h] = *reinterpret_cast<const v4u *>(smem + bst + d + jb * 2 * kTileBytes + h * 512);
    };
    auto unpack_b = [&](const v4u (&wd)[2], v4i (&Bj)[4]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            Bj[2 * h] = unpack_k64(wd[h].x, wd[h].y);
            Bj[2 * h + 1] = unpack_k64(wd[h].z, wd[h].w);
        }
    };
    auto read_w = [&](int d, float (&wv)[TB][UPS]) {
#pragma unroll
        for (int jb = 0; jb < TB; ++jb)
#pragma unroll
            for (int u = 0; u < UPS; ++u)
                wv[jb][u] = half_bits_to_float(
                    *reinterpret_cast<const uint16_t *>(smem + sst + d + (jb * 2 * UPS + u) * 32));
    };
    auto read_a = [&](int d, int ib, v4i (&A)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c) A[c] = *reinterpret_cast<const v4i *>(smem + ast[c] + d + ib * 4096);
    };

    // Software pipeline over the 32x32 blocks of all steps (row block jb
    // fastest within a step): block b issues its MFMAs interleaved with the
    // chain updates of the block before it (at a step's first block, the
    // previous step's last), so the updates run while the matrix core works.
    // Within a step, token block ib + 1's activations are read at block
    // (ib, 0) and weight block jb + 1 at block (0, jb), one block ahead. With
    // an extra column the step ends with its block: its packed weights and
    // scales are read two blocks ahead, unpacked and its activations read
    // one block ahead.
    constexpr int NBO = TA * TB, NB = NBO + XB;
    static_assert(XB == 0 || NBO >= 2, "extra column reads two blocks ahead");
    v4i B[TB][4];
    v4i Bx[4];
    v4u rawx[2];
    float wx[UPS];
    v4u raw[2];                        // TB = 1, NB > 1: the next step's packed tile
    v4i Bnext[4];                      // NB = 1: the next step's unpacked tile
    float w[TB][UPS], wnext[TB][UPS], wlast[UPS];
    v4i Acur[4], Anext[4];
    // acc[slot][u]: the 64-K group u of a block (one group per block at
    // group 128, where MFMAs 0-3 chain into acc[.][0]; at group 64 the
    // first 64-K half is MFMAs 0 and 2, the second 1 and 3); consecutive
    // blocks alternate slots across steps too
    v16i acc[2][UPS];
    const v16i zero = {};
    auto read_next_step = [&](int d) {
        if constexpr (TB > 1) {
            v4u wd[2];
            read_b(d, 0, wd);
            unpack_b(wd, B[0]);
        } else if constexpr (NB == 1) {
            v4u wd[2];
            read_b(d, 0, wd);
            unpack_b(wd, Bnext);
        } else {
            read_b(d, 0, raw);          // (no registers to unpack it ahead)
        }
        read_w(d, wnext);
        read_a(d, 0, Anext);
    };
    auto update = [&](int ib, int jb, const v16i (&p)[UPS], const float (&wv)[UPS]) {
#pragma unroll
        for (int u = 0; u < UPS; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                f[ib][jb][r] = __builtin_fmaf((float)p[u][r], wv[u], f[ib][jb][r]);
    };
    auto update_x = [&](const v16i (&p)[UPS]) {
#pragma unroll
        for (int u = 0; u < UPS; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) fx[r] = __builtin_fmaf((float)p[u][r], wx[u], fx[r]);
    };
    // LDS reads block b issues ahead of its MFMAs
    auto ds_reads = [](int b) {
        const int ib = b / TB, jb = b % TB;
        if (b == NB - 1) return 2 + TB * UPS + 4;
        return (jb == 0 && ib + 1 < TA ? 4 : 0) + (ib == 0 && jb + 1 < TB ? 2 : 0) +
               (XB && b == NBO - 2 ? 2 + UPS : 0) + (XB && b == NBO - 1 ? 4 : 0);
    };
    // (the group size must be a literal; the block loop is unrolled, so the
    // switch folds)
    auto ds_first = [](int n) {
        switch (n) {
        case 2: __builtin_amdgcn_sched_group_barrier(0x100, 2, 0); break;
        case 4: __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); break;
        case 6: __builtin_amdgcn_sched_group_barrier(0x100, 6, 0); break;
        case 7: __builtin_amdgcn_sched_group_barrier(0x100, 7, 0); break;
        case 8: __builtin_amdgcn_sched_group_barrier(0x100, 8, 0); break;
        case 10: __builtin_amdgcn_sched_group_barrier(0x100, 10, 0); break;
        default: break;
        }
    };

#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < NT) issue(s, s);
    arrive(0);
    if (NST - 1 < NT) issue(NST - 1, NST - 1);
    read_next_step(0);
    // With one block per step every read is of the next step's stage, so the
    // tracked offsets point there instead. A one-block step whose ring fits
    // the 16-bit offset field of an LDS read instead takes its stage as a
    // compile-time index (the loop unrolled over the ring and the slot
    // parity): the stage offset then folds into each read's immediate, and
    // no offsets are moved at all.
    constexpr bool kTrackNext = TA * TB == 1;
    constexpr bool kStaticStage = NB == 1 && NST * STAGE <= 65536;
    if constexpr (kTrackNext && !kStaticStage) {
#pragma unroll
        for (int c = 0; c < 4; ++c) ast[c] += STAGE;
        bst += STAGE;
        sst += STAGE;
    }
    // (complete here: the wait pass would otherwise assume them pending at
    // the loop head and wait on every step's first MFMA)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    // step 0's first block "updates" the last block of no step: a zero
    // product at a zero scale leaves its +0 chain unchanged
#pragma unroll
    for (int u = 0; u < UPS; ++u) acc[1][u] = zero;
#pragma unroll
    for (int jb = 0; jb < TB; ++jb)
#pragma unroll
        for (int u = 0; u < UPS; ++u) w[jb][u] = 0.0f;
#pragma unroll
    for (int u = 0; u < UPS; ++u) wx[u] = 0.0f;

    int st = 0;
    // (stc: the step's stage when compile-time, else -1 for the tracked one)
    auto step = [&](const int kb, auto par, auto stc) {
        constexpr int PAR = decltype(par)::value, SC = decltype(stc)::value;
        const int sc = SC >= 0 ? SC : st;
        const int stn = sc == NST - 1 ? 0 : sc + 1;
        const int dn = (stn - sc) * STAGE;
        // byte distances from the tracked offsets to this step's stage and
        // to the next one
        const int dcur = SC >= 0 ? SC * STAGE : 0;
        const int dnext = SC >= 0 ? stn * STAGE : kTrackNext ? 0 : dn;
        const bool more = kb + 1 < NT;
#pragma unroll
        for (int u = 0; u < UPS; ++u) wlast[u] = w[TB - 1][u];
#pragma unroll
        for (int jb = 0; jb < TB; ++jb)
#pragma unroll
            for (int u = 0; u < UPS; ++u) w[jb][u] = wnext[jb][u];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int ib = b / TB, jb = b % TB;
            const int slot = (PAR * NB + b) & 1;
            if (b == NB - 1) {
                if (more) {
                    arrive(kb + 1);
                    if (kb + NST < NT) issue(kb + NST, sc);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (jb == 0) {
#pragma unroll
                for (int c = 0; c < 4; ++c) Acur[c] = Anext[c];
            }
            if constexpr (TB == 1 && NB == 1) {
#pragma unroll
                for (int c = 0; c < 4; ++c) B[0][c] = Bnext[c];
            } else if constexpr (TB == 1) {
                if (b == 0) unpack_b(raw, B[0]);
            }
            if (b == NB - 1) {
                // the next step's first operands (after the last step: a
                // harmless read of a stale stage)
                read_next_step(dnext);
            } else {
                if (jb == 0 && ib + 1 < TA) read_a(dcur, ib + 1, Anext);
                if (ib == 0 && jb + 1 < TB) {
                    v4u wd[2];
                    read_b(dcur, jb + 1, wd);
                    unpack_b(wd, B[jb + 1]);
                }
                if (XB && b == NBO - 2) {
                    read_b(dcur + dxb, 0, rawx);
#pragma unroll
                    for (int u = 0; u < UPS; ++u)
                        wx[u] = half_bits_to_float(*reinterpret_cast<const uint16_t *>(smem + sst + dcur + dxs + u * 32));
                }
                if (XB && b == NBO - 1) {
                    read_a(dcur + dxa, 0, Anext);
                    unpack_b(rawx, Bx);
                }
            }
            const v4i (&Bo)[4] = b < NBO ? B[jb] : Bx;
            v16i (&p)[UPS] = acc[slot];
            if constexpr (UNIT == 128) {
                p[0] = mfma32(Acur[0], Bo[0], zero);
                p[0] = mfma32(Acur[1], Bo[1], p[0]);
                p[0] = mfma32(Acur[2], Bo[2], p[0]);
                p[0] = mfma32(Acur[3], Bo[3], p[0]);
            } else {
                static_assert(UNIT == 64, "per-token mode has unit = group in {64, 128}");
                p[0] = mfma32(Acur[0], Bo[0], zero);
                p[UPS - 1] = mfma32(Acur[1], Bo[1], zero);
                p[0] = mfma32(Acur[2], Bo[2], p[0]);
                p[UPS - 1] = mfma32(Acur[3], Bo[3], p[UPS - 1]);
            }
            if (XB && b == 0) {
                // the previous step's extra block
                update_x(acc[slot ^ 1]);
#pragma unroll
                for (int r = 0; r < 16; ++r) asm volatile("" ::"v"(fx[r]));
            } else {
                const int ub = b > 0 ? (b - 1) / TB : TA - 1, uj = b > 0 ? (b - 1) % TB : TB - 1;
                update(ub, uj, acc[slot ^ 1], b > 0 ? w[uj] : wlast);
                // keep the updates in this block: without a use here the
                // compiler sinks them past the barrier branch of the last block
#pragma unroll
                for (int r = 0; r < 16; ++r) asm volatile("" ::"v"(f[ub][uj][r]));
            }
            // the block's reads, then one MFMA and the VALU share of the
            // previous block's updates, four times
            ds_first(ds_reads(b));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 8 * UPS, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (SC < 0) {
            const int adv = kTrackNext ? ((stn == NST - 1 ? 0 : stn + 1) - stn) * STAGE : dn;
            st = stn;
#pragma unroll
            for (int c = 0; c < 4; ++c) ast[c] += adv;
            bst += adv;
            sst += adv;
        }
    };
    using Dyn = std::integral_constant<int, -1>;
    // the last block's updates after the last step
    auto update_last = [&](const v16i (&p)[UPS]) {
        if constexpr (XB) update_x(p);
        else update(TA - 1, TB - 1, p, w[TB - 1]);
    };
    // after the last step, its last block's updates
    constexpr int LAST0 = (NB - 1) & 1, LAST1 = (2 * NB - 1) & 1;
    if constexpr (kStaticStage) {
        // U steps per iteration (a multiple of the ring and, for an odd
        // block count, of the slot parity), then up to U - 1 more; step i of
        // an iteration has stage i % NST and parity i % 2
        constexpr int U = NB % 2 == 0 ? NST : (NST % 2 == 0 ? NST : 2 * NST);
        int kb = 0;
        auto one = [&](auto i) {
            constexpr int I = decltype(i)::value;
            step(kb + I, std::integral_constant<int, (NB & 1) * (I & 1)>{}, std::integral_constant<int, I % NST>{});
        };
        for (; kb + U <= NT; kb += U) for_each_index(one, std::make_integer_sequence<int, U>{});
        for_each_index([&](auto i) { if (kb + decltype(i)::value < NT) one(i); }, std::make_integer_sequence<int, U - 1>{});
        if (NB % 2 == 1 && ((NT - 1) & 1)) update_last(acc[LAST1]);
        else update_last(acc[LAST0]);
    } else if constexpr (NB % 2 == 0) {
        for (int kb = 0; kb < NT; ++kb) step(kb, std::integral_constant<int, 0>{}, Dyn{});
        update_last(acc[LAST0]);
    } else {
        // an odd block count flips the slot parity every step: two steps
        // per iteration keep the slots compile-time
        int kb = 0;
        for (; kb + 1 < NT; kb += 2) {
            step(kb, std::integral_constant<int, 0>{}, Dyn{});
            step(kb + 1, std::integral_constant<int, 1>{}, Dyn{});
        }
        if (kb < NT) {
            step(kb, std::integral_constant<int, 0>{}, Dyn{});
            update_last(acc[LAST0]);
        } else {
            update_last(acc[LAST1]);
        }
    }
    // ---- output ----
    // Each wave stages SB token blocks at a time in its own LDS slab (the
    // ring is free once every wave is past its last step) and writes whole
    // 16-byte row runs: register r of block (ib, jb) is token
    // 8(r/4) + 4kg + r%4 and row m32 of the block. The extra column's block
    // goes out the same way after the wave's own blocks.
    constexpr int EPS = S::EPS, SB = S::template slab_blocks<NST>();
    static_assert(TA % SB == 0, "slabs cover the wave tile");
    static_assert(S::template lds_bytes<NST>() <= 160 * 1024, "LDS");
    lds_sync();
    float *slab = reinterpret_cast<float *>(smem) + wave * (32 * SB * EPS);
    const float *tsc = reinterpret_cast<const float *>(smem + S::template body_bytes<NST>());
    // read back runs of CH rows of one token (CH = 8 BF16 or 4 FP32 outputs
    // = 16 bytes) from NBT token blocks x COLS rows of the slab; tok: the
    // first token relative to the tile, rgb: the first row-group relative to
    // the tile. The slab is this wave's own, and its LDS accesses complete in
    // order
    auto run = [&](auto ch, auto cols, auto nbt, int tok, int rgb) {
        constexpr int CH = decltype(ch)::value, COLS = decltype(cols)::value, NBT = decltype(nbt)::value;
        constexpr int PER_TOKEN = COLS / CH;
#pragma unroll
        for (int it = 0; it < 32 * NBT * PER_TOKEN / 64; ++it) {
            const int q = it * 64 + lane;
            const int tl = q / PER_TOKEN, rl = (q % PER_TOKEN) * CH;
            const int t = t0 + tok + tl;
            const int rg = rg0 + rgb + (rl >> 4);
            if (t >= T || rg >= RG) continue;
            const int row = rg * 16 + (rl & 15);
            const float sc = tsc[tok + tl] * 0.0625f;
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
    auto out_pass = [&](auto cols, auto nbt, int tok, int rgb) {
        if (a.y_bf16) run(std::integral_constant<int, 8>{}, cols, nbt, tok, rgb);
        else run(std::integral_constant<int, 4>{}, cols, nbt, tok, rgb);
    };
#pragma unroll
    for (int s0 = 0; s0 < TA; s0 += SB) {
#pragma unroll
        for (int ib = s0; ib < s0 + SB; ++ib)
#pragma unroll
            for (int jb = 0; jb < TB; ++jb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    slab[(32 * (ib - s0) + 8 * (r >> 2) + 4 * kg + (r & 3)) * EPS + 32 * jb + m32] = f[ib][jb][r];
        out_pass(std::integral_constant<int, 32 * TB>{}, std::integral_constant<int, SB>{}, tw + 32 * s0, wn * 2 * TB);
    }
    if constexpr (XB) {
#pragma unroll
        for (int r = 0; r < 16; ++r) slab[(8 * (r >> 2) + 4 * kg + (r & 3)) * EPS + m32] = fx[r];
        out_pass(std::integral_constant<int, 32>{}, std::integral_constant<int, 1>{}, tw + 32 * wn, WNW * 2 * TB);
    }
}

template <int TA, int TB, int WMW, int WNW, int UNIT, int NST, int OCC = 2, int XB = 0>
static int launch_g3(GemmArgs &a, hipStream_t st) {
    using S = G3Shape<TA, TB, WMW, WNW, UNIT, XB>;
    int nt = 0;
    for (int i = 0; i < a.count; ++i) {
        a.w[i].nt_begin = nt;
        nt += (a.w[i].M / 16 + S::BNG - 1) / S::BNG;
    }
    a.n_tiles = nt;
    a.t_tiles = (a.T + S::BM - 1) / S::BM;
    a.raster_tt = options().gemm3_raster > 0 ? options().gemm3_raster : kG3GroupTT;
    const dim3 grid(a.n_tiles * a.t_tiles), block(S::NTH);
    auto k = gemm3_kernel<TA, TB, WMW, WNW, UNIT, NST, OCC, XB>;
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

// Tile choice. Per SIMD the kernel is bound by the FP32 chain of its
// blocks, so each candidate is scored by the rounds of work-groups it needs
// over the CUs times the 32x32 blocks per K step its busiest SIMD carries
// per round (waves on that SIMD x blocks per wave); the small tile pays ~10%
// for its larger L2 traffic per MAC (measured):
//   256 x 256, 8 waves (2 per SIMD, 8 blocks each), one work-group per CU;
//   256 x 160 (G128) / 64 x 160 (G64), 10 waves (3 on the busiest SIMD),
//     one work-group per CU: fits the grid when the 256-row tile leaves
//     CUs idle;
//   256 x 160 at G128 as 8 waves of 4 + 1 blocks (each wave's four blocks
//     of its own 32-row column and one block of the fifth column): 10 blocks
//     on every SIMD (the waves of a work-group go to the SIMDs in turn, so
//     ten one-column waves put 12 on two SIMDs and 8 on the others);
//   128 x 64, 4 waves of 2 blocks, three work-groups per CU;
//   128 x 256 (G128), 4 waves of 8 blocks, two work-groups per CU: the same
//     16 blocks per SIMD and step as 256 x 256, but a SIMD's two waves
//     belong to different work-groups and never wait for each other at the
//     step barrier (with one 8-wave work-group the older wave of each SIMD
//     finishes its step ~1,700 cycles early and idles): 8% faster on cfg4
//     (measured), so it is preferred at an equal number of rounds.
static int choose_tile(const GemmArgs &a, int *bm) {
    const bool g128 = a.group == 128;
    struct Cand { int sel, bm, bng, wgs, simd_blocks; double penalty; };
    const Cand cands[4] = {
        {0, 256, g128 ? 16 : 8, 1, g128 ? 16 : 8, 1.0},
        {g128 ? 11 : 8, g128 ? 256 : 64, 10, 1, g128 ? 10 : 3, 1.0},
        {g128 ? 3 : 4, 128, 4, 3, 6, 1.1},
        {1, 128, 16, 2, 16, 0.92},
    };
    const long long cus = device_cus();
    double best = 0.0;
    int sel = -1;
    for (const Cand &c : cands) {
        if (c.sel == 1 && !g128) continue;                   // (tile 1 is 128 x 128 at G64)
        long long nt = 0;
        for (int i = 0; i < a.count; ++i) nt += (a.w[i].M / 16 + c.bng - 1) / c.bng;
        const long long tiles = nt * ((a.T + c.bm - 1) / c.bm);
        const long long rounds = (tiles + cus * c.wgs - 1) / (cus * c.wgs);
        const double cost = (double)rounds * c.simd_blocks * c.penalty;
        if (sel < 0 || cost < best) {
            best = cost;
            sel = c.sel;
            *bm = c.bm;
        }
    }
    return sel;
}

static int launch_tile(GemmArgs &a, int sel, hipStream_t st);

int launch_gemm3(GemmArgs &a, hipStream_t st) {
    // per-token activation scale, plain FP16 weight scales, one split per token
    if (a.block != 0 || a.scale_enc != 0 || (a.group != 64 && a.group != 128)) return 1;
    if ((long long)a.T * a.K >= (1ll << 31)) return 1;          // 32-bit activation offsets
    for (int i = 0; i < a.count; ++i) {
        if ((long long)a.w[i].M * a.K / 2 >= (1ll << 31)) return 1;
        for (int s = 0; s < a.seg_count; ++s)
            if (a.w[i].seg_split[s] != 1) return 1;
    }
    // the gemm3_tile option (0..11) picks one configuration (tests, tuning)
    const int forced = options().gemm3_tile;
    if (forced >= 0) return launch_tile(a, forced, st);
    int bm = 0;
    const int sel = choose_tile(a, &bm);
    return launch_tile(a, sel, st);
}

static int launch_tile(GemmArgs &a, int sel, hipStream_t st) {
    if (a.group == 128) {
        switch (sel) {
        case 8: return launch_g3<4, 1, 2, 5, 128, 3, 3>(a, st);   // 256 x 160, 10 waves
        case 10: return launch_g3<4, 1, 2, 4, 128, 3, 2, 1>(a, st);  // 256 x 160, 8 waves of 4 + 1 blocks
        case 11: return launch_g3<4, 1, 2, 4, 128, 2, 2, 1>(a, st);  // the same, 2 stages
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
