// kxw4_quant.hip — activation quantizers (kernels_dpas.cpp:188-223, 846-929,
// 1149-1207): rows spread over work-groups when few, else one work-group per
// row.
//
// A producer computes the fp32 value of element k (plain load, SiLU(g)*u, or
// (1+w) RMSNorm); the quantizer turns it into int8 with
//   s = absmax/127 (1 when the block max is not positive),
//   q = clamp(rint(v / s), -127, 127)          (IEEE division, NaN -> -127)
// over blocks of 32 K (reference mode) or the whole row (per-token mode), and
// writes exact int32 code sums per K32. Codes are stored in the MFMA slot
// order of each 64-element chunk (act_slot). The chunk kernels divide once
// per chunk or row and multiply by the reciprocal, taking the division only
// where that could round differently (rint_quot), so their codes are the
// division's.
//
// The element-loop fallback (rows not on 16 bytes, or per-token rows longer
// than the chunk kernels hold): in block 32 the 32 lanes of a half wave hold
// one block, so absmax and sums are half-wave shuffles and each element is
// produced once; per-token, a first pass reduces the row absmax across the
// work-group, a second pass quantizes (producers are recomputed,
// bit-identically).
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

namespace kxw4 {

enum Producer { kLoadF32 = 0, kLoadBF16 = 1, kSiluMul = 2, kRmsNorm = 3 };

constexpr int kQThreads = 256;

struct QuantArgs {
    const void *x;          // f32 / bf16 input, or gate (SiLU), or in (norm)
    const float *up;        // SiLU up operand
    const uint16_t *w;      // RMSNorm bf16 weight
    float *out;             // optional fp32 producer output [T][K]
    int8_t *q;
    float *scale;
    int32_t *sum;
    int T, K;
    float eps;
};

__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int half_wave_sum(int v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Lane reductions on DPP moves (no LDS round trip per step), for max and
// integer sums, whose result does not depend on the order: quad_perm
// [1,0,3,2] and [2,3,0,1] exchange the neighbours and pairs of a 4-lane
// group, row_half_mirror (lane i <-> 7-i of each 8) joins two groups,
// row_mirror (i <-> 15-i of each 16) two halves of a row, and lanes 0, 16,
// 32 and 48 then hold the four rows' results. Every lane of the group being
// reduced must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
    return fmaxf(v, dpp_f<kDppQuadXor2>(v));
}
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp_i<kDppQuadXor1>(v);
    return v + dpp_i<kDppQuadXor2>(v);
}
__device__ __forceinline__ float oct_max(float v) {
    v = quad_max(v);
    return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}
__device__ __forceinline__ int oct_sum(int v) {
    v = quad_sum(v);
    return v + dpp_i<kDppHalfMirror>(v);
}
__device__ __forceinline__ float wave_max(float v) {
    v = oct_max(v);
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    const int b = __float_as_int(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 0)), __int_as_float(__builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 32)), __int_as_float(__builtin_amdgcn_readlane(b, 48))));
}

__device__ __forceinline__ float block_reduce_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kQThreads / 64; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_reduce_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kQThreads / 64; ++i) r += red[i];
    __syncthreads();
    return r;
}

template <int P>
__device__ __forceinline__ float produce(const QuantArgs &a, int t, int k, float rms_inv) {
    const size_t i = (size_t)t * a.K + k;
    if constexpr (P == kLoadF32) {
        return static_cast<const float *>(a.x)[i];
    } else if constexpr (P == kLoadBF16) {
        return bf16_to_float(static_cast<const uint16_t *>(a.x)[i]);
    } else if constexpr (P == kSiluMul) {
        const float g = static_cast<const float *>(a.x)[i];
        return (g / (1.0f + expf(-g))) * a.up[i];
    } else {
        const float v = static_cast<const float *>(a.x)[i];
        return v * rms_inv * (1.0f + bf16_to_float(a.w[k]));
    }
}

__device__ __forceinline__ int8_t quantize_one(float v, float s) {
    return (int8_t)(int)clampf(rintf(v / s), -127.0f, 127.0f);
}

// rint(v / s) of N values, bit for bit, without a division per value:
// y = v * r with r the hardware reciprocal of s (within 1 ulp of 1/s; the
// bound below allows 2). Where |v| <= m and s is m / L rounded (the block or
// row absmax over the code limit L), |v / s| <= L (1 + 2^-23) and y differs
// from the rounded quotient fl(v / s) by at most |v / s| * 1.5 * 2^-22,
// 4.6e-5 at L = 127; so where y lies further than 2^-14 from every half-integer,
// fl(v / s) lies on the same side of it and both round to the same integer.
// The other values (about one in 8,000 for smooth data), and every value when
// s < 2^-120 (whose reciprocal could overflow), take the division itself. A
// NaN value gives NaN on both paths; an infinite one makes s infinite, r 0
// and y NaN as v / s is, and every finite value of its block 0 on both.
template <int N>
__device__ __forceinline__ void rint_quot(const float (&v)[N], float s, float (&k)[N]) {
    const float r = __builtin_amdgcn_rcpf(s);
    float d = 0.0f;   // largest distance of a y from its integer (NaN y: none)
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const float y = v[j] * r;
        k[j] = rintf(y);
        d = fmaxf(d, fabsf(y - k[j]));
    }
    if (!(s >= 0x1p-120f) || d > 0.5f - 0x1p-14f) {
#pragma unroll
        for (int j = 0; j < N; ++j) k[j] = rintf(v[j] / s);
    }
}

// The int8 codes of a chunk of 8 values at scale s, as quantize_one gives
// them, packed in element order, and their sum (two signed byte dot products
// with ones).
__device__ __forceinline__ uint2 quantize_chunk(const float (&v)[8], float s, int &sum) {
    float k[8];
    rint_quot(v, s, k);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int8_t q = (int8_t)(int)clampf(k[j], -127.0f, 127.0f);
        if (j < 4) lo |= (uint32_t)(uint8_t)q << (8 * j);
        else hi |= (uint32_t)(uint8_t)q << (8 * (j - 4));
    }
    sum = __builtin_amdgcn_sdot4((int)hi, 0x01010101, __builtin_amdgcn_sdot4((int)lo, 0x01010101, 0, false), false);
    return make_uint2(lo, hi);
}

// The element loops below take kQU elements per thread and pass: all kQU
// loads are issued (at indices clamped into the row) before any is used, so a
// pass costs one memory round trip instead of one per element; the values of
// clamped positions are never used, and the arithmetic and its order are the
// element loop's.
constexpr int kQU = 8;

// 1 / sqrt(mean(x^2) + eps) of row t, summed in a fixed order: thread tid
// adds x[k]^2 for k = tid, tid + kQThreads, ... in turn, then the work-group
// sum (the work-group must have kQThreads threads). The loads go 32 to a
// memory round trip (H = 17408: three round trips instead of nine); the
// adds keep their order.
__device__ __forceinline__ float row_rms_inv(const QuantArgs &a, int t, float *red) {
    constexpr int B = 32;
    const int K = a.K, tid = threadIdx.x;
    const float *row = static_cast<const float *>(a.x) + (size_t)t * K;
    float ss = 0.0f;
    for (int k0 = tid; k0 < K; k0 += kQThreads * B) {
        float x[B];
#pragma unroll
        for (int u = 0; u < B; ++u) x[u] = row[min(k0 + u * kQThreads, K - 1)];
#pragma unroll
        for (int u = 0; u < B; ++u)
            if (k0 + u * kQThreads < K) ss += x[u] * x[u];
    }
    ss = block_reduce_sum(ss, red);
    return 1.0f / sqrtf(ss / (float)K + a.eps);
}

template <int P, bool PER_TOKEN>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(QuantArgs a) {
    __shared__ float red[kQThreads / 64];
    const int t = blockIdx.x;
    const int K = a.K;
    const int tid = threadIdx.x;
    float rms_inv = 0.0f;
    if constexpr (P == kRmsNorm) rms_inv = row_rms_inv(a, t, red);
    int8_t *qrow = a.q + (size_t)t * K;
    float s_tok = 1.0f;
    if constexpr (PER_TOKEN) {
        float mx = -INFINITY;
        for (int k0 = tid; k0 < K; k0 += kQThreads * kQU) {
            float v[kQU];
#pragma unroll
            for (int u = 0; u < kQU; ++u) v[u] = produce<P>(a, t, min(k0 + u * kQThreads, K - 1), rms_inv);
#pragma unroll
            for (int u = 0; u < kQU; ++u) {
                const int k = k0 + u * kQThreads;
                if (k < K) {
                    if (a.out) a.out[(size_t)t * K + k] = v[u];
                    mx = fmaxf(mx, fabsf(v[u]));
                }
            }
        }
        mx = block_reduce_max(mx, red);
        s_tok = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
        if (tid == 0) a.scale[t] = s_tok;
    }
    // K % 32 == 0 and kQThreads % 32 == 0: each half wave walks whole blocks,
    // so a half wave's positions are all in the row or all past it (those
    // past it shuffle among themselves and store nothing).
    for (int k0 = tid; k0 < K; k0 += kQThreads * kQU) {
        float v[kQU];
#pragma unroll
        for (int u = 0; u < kQU; ++u) v[u] = produce<P>(a, t, min(k0 + u * kQThreads, K - 1), rms_inv);
#pragma unroll
        for (int u = 0; u < kQU; ++u) {
            const int k = k0 + u * kQThreads;
            const bool in = k < K;
            float s = s_tok;
            if constexpr (!PER_TOKEN) {
                if (a.out && in) a.out[(size_t)t * K + k] = v[u];
                const float mx = half_wave_max(fabsf(v[u]));
                s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
                if (in && (k & 31) == 0) a.scale[(size_t)t * (K / 32) + (k >> 5)] = s;
            }
            const int8_t q = quantize_one(v[u], s);
            if (in) qrow[(k & ~63) + act_slot(k)] = q;
            const int bsum = half_wave_sum((int)q);
            if (in && (k & 31) == 0 && a.sum) a.sum[(size_t)t * (K / 32) + (k >> 5)] = bsum;
        }
    }
}

// The values of this thread's NCH chunks of 8 consecutive elements of row t
// (chunk first + tid + c*NT), every chunk's inputs loaded before any is used,
// at chunk indices clamped into the row (a chunk past the row holds the last
// chunk's values and is not used); the per-element arithmetic is produce's.
template <int P, int NCH, int NT>
__device__ __forceinline__ void chunk_values(const QuantArgs &a, int t, float rms_inv, float (&v)[NCH][8],
                                             int first = 0) {
    const int nch = a.K / 8, tid = threadIdx.x;
    const size_t row0 = (size_t)t * a.K;
    uint4 raw[NCH][P == kLoadBF16 || P == kRmsNorm ? 1 : 2];
    float4 upv[P == kSiluMul ? NCH : 1][2];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = min(first + tid + c * NT, nch - 1);
        if constexpr (P == kLoadBF16) {
            raw[c][0] = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.x) + row0)[idx];
        } else {
            const float4 *xr = reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) + row0);
            const float4 x0 = xr[2 * idx], x1 = xr[2 * idx + 1];
            v[c][0] = x0.x; v[c][1] = x0.y; v[c][2] = x0.z; v[c][3] = x0.w;
            v[c][4] = x1.x; v[c][5] = x1.y; v[c][6] = x1.z; v[c][7] = x1.w;
            if constexpr (P == kSiluMul) {
                const float4 *ur = reinterpret_cast<const float4 *>(a.up + row0);
                upv[c][0] = ur[2 * idx];
                upv[c][1] = ur[2 * idx + 1];
            }
            if constexpr (P == kRmsNorm) raw[c][0] = reinterpret_cast<const uint4 *>(a.w)[idx];
        }
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if constexpr (P == kLoadBF16) {
            const uint32_t w[4] = {raw[c][0].x, raw[c][0].y, raw[c][0].z, raw[c][0].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[c][2 * j] = __uint_as_float(w[j] << 16);
                v[c][2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
            }
        } else if constexpr (P == kSiluMul) {
            const float u[8] = {upv[c][0].x, upv[c][0].y, upv[c][0].z, upv[c][0].w,
                                upv[c][1].x, upv[c][1].y, upv[c][1].z, upv[c][1].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[c][j] = (v[c][j] / (1.0f + expf(-v[c][j]))) * u[j];
        } else if constexpr (P == kRmsNorm) {
            const uint32_t w[4] = {raw[c][0].x, raw[c][0].y, raw[c][0].z, raw[c][0].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[c][2 * j] = v[c][2 * j] * rms_inv * (1.0f + bf16_to_float((uint16_t)(w[j] & 0xFFFFu)));
                v[c][2 * j + 1] = v[c][2 * j + 1] * rms_inv * (1.0f + bf16_to_float((uint16_t)(w[j] >> 16)));
            }
        }
    }
}

// the producer's fp32 value of chunk idx, when the caller asked for it
template <int NCH>
__device__ __forceinline__ void store_chunk_out(const QuantArgs &a, int t, int idx, const float (&v)[8]) {
    float4 *o = reinterpret_cast<float4 *>(a.out + (size_t)t * a.K) + 2 * idx;
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// One row per work-group: each thread holds chunks of 8 consecutive
// elements (16-byte bf16 / 32-byte f32 loads) in registers for the whole
// row, so the row is read once. The MFMA slot order keeps the 8 codes of a
// chunk contiguous: chunk c of 64-element chunk h lands at byte
// 64h + 16(c & 3) + 8((c >> 2) & 1), one 8-byte store. The four chunks of a
// K32 block sit in four consecutive lanes, so a block's absmax (K32 mode)
// and code sum are 4-lane shuffles; the per-token absmax is a work-group
// reduction.
template <int P, int NCH, int NT = kQThreads, bool PER_TOKEN = true>
__global__ __launch_bounds__(NT) void quantize_tok_kernel(QuantArgs a) {
    static_assert(P != kRmsNorm || NT == kQThreads, "the row sum's order assumes kQThreads threads");
    __shared__ float red[NT / 64];
    const int t = blockIdx.x, K = a.K, tid = threadIdx.x;
    const int nch = K / 8;
    float rms_inv = 0.0f;
    if constexpr (P == kRmsNorm) rms_inv = row_rms_inv(a, t, red);
    float v[NCH][8];
    chunk_values<P, NCH, NT>(a, t, rms_inv, v);
    float s = 1.0f;
    if constexpr (PER_TOKEN) {
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (tid + c * NT < nch) {
#pragma unroll
                for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[c][j]));
            }
        }
        // work-group max (order-free, so any thread count gives the same bits)
        mx = wave_max(mx);
        if ((tid & 63) == 0) red[tid >> 6] = mx;
        __syncthreads();
        mx = red[0];
#pragma unroll
        for (int i = 1; i < NT / 64; ++i) mx = fmaxf(mx, red[i]);
        s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
        if (tid == 0) a.scale[t] = s;
    }
    int8_t *qrow = a.q + (size_t)t * K;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = tid + c * NT;
        // whole K32 blocks (4 chunks) per 4-lane group: nch % 4 == 0
        if (idx - (tid & 3) < nch) {
            const bool in = idx < nch;
            if (P >= kSiluMul && a.out && in) store_chunk_out<NCH>(a, t, idx, v[c]);
            if constexpr (!PER_TOKEN) {
                float mx = fabsf(v[c][0]);
#pragma unroll
                for (int j = 1; j < 8; ++j) mx = fmaxf(mx, fabsf(v[c][j]));
                mx = quad_max(mx);
                s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
            }
            int sum = 0;
            const uint2 codes = quantize_chunk(v[c], s, sum);
            if (in) *reinterpret_cast<uint2 *>(qrow + 64 * (idx >> 3) + 16 * (idx & 3) + 8 * ((idx >> 2) & 1)) = codes;
            sum = quad_sum(sum);
            if (in && (idx & 3) == 0) {
                if (!PER_TOKEN) a.scale[(size_t)t * (K / 32) + (idx >> 2)] = s;
                if (a.sum) a.sum[(size_t)t * (K / 32) + (idx >> 2)] = sum;
            }
        }
    }
}

// Rows spread over work-groups: work-group b = t*G + g quantizes chunks
// [g*NT, (g+1)*NT) of row t (G = ceil(nch / NT)), one chunk per thread, so
// with few tokens a row's quantization runs on G CUs instead of one. K32
// blocks (4 chunks, 4 consecutive lanes) need only their own chunk: absmax
// and code sum are two lane shuffles each. A per-token scale needs the row's
// absmax, so each work-group of a row produces the whole row as the per-row
// kernel does (NCH chunks per thread, G <= NCH) and reduces it -- a max per
// element, against the quantization it leaves to the chunk's owner -- and
// keeps its own chunk, c = g, in registers. RMSNorm's row sum is likewise
// computed by every work-group of the row in the per-row kernel's order, so
// every work-group sees the same bits.
template <int P, int NCH, bool PER_TOKEN>
__global__ __launch_bounds__(kQThreads) void quantize_spread_kernel(QuantArgs a, int G) {
    static_assert(PER_TOKEN || NCH == 1, "K32 blocks: one chunk per thread");
    __shared__ float red[kQThreads / 64];
    const int t = blockIdx.x / G, g = blockIdx.x - t * G;
    const int K = a.K, tid = threadIdx.x, nch = K / 8;
    const int idx = g * kQThreads + tid;
    const bool in = idx < nch;   // a K32 block's four chunks are all in the row or all past it
    float rms_inv = 0.0f;
    if constexpr (P == kRmsNorm) rms_inv = row_rms_inv(a, t, red);
    float w[8];
    float s;
    if constexpr (PER_TOKEN) {
        float v[NCH][8];
        chunk_values<P, NCH, kQThreads>(a, t, rms_inv, v);
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (tid + c * kQThreads < nch) {
#pragma unroll
                for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[c][j]));
            }
        }
        mx = wave_max(mx);
        if ((tid & 63) == 0) red[tid >> 6] = mx;
        __syncthreads();
        mx = red[0];
#pragma unroll
        for (int i = 1; i < kQThreads / 64; ++i) mx = fmaxf(mx, red[i]);
        s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
        if (g == 0 && tid == 0) a.scale[t] = s;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (c == g) {
#pragma unroll
                for (int j = 0; j < 8; ++j) w[j] = v[c][j];
            }
        }
    } else {
        float v[1][8];
        chunk_values<P, 1, kQThreads>(a, t, rms_inv, v, g * kQThreads);
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = v[0][j];
        float mx = fabsf(w[0]);
#pragma unroll
        for (int j = 1; j < 8; ++j) mx = fmaxf(mx, fabsf(w[j]));
        mx = quad_max(mx);
        s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
    }
    if (P >= kSiluMul && a.out && in) store_chunk_out<1>(a, t, idx, w);
    int sum = 0;
    const uint2 codes = quantize_chunk(w, s, sum);
    if (in)
        *reinterpret_cast<uint2 *>(a.q + (size_t)t * K + 64 * (idx >> 3) + 16 * (idx & 3) + 8 * ((idx >> 2) & 1)) =
            codes;
    sum = quad_sum(sum);
    if (in && (idx & 3) == 0) {
        if (!PER_TOKEN) a.scale[(size_t)t * (K / 32) + (idx >> 2)] = s;
        if (a.sum) a.sum[(size_t)t * (K / 32) + (idx >> 2)] = sum;
    }
}

template <int P>
static int launch_q(const QuantArgs &a, int block, hipStream_t st) {
    // One pass with the chunks in registers: 16-byte vector loads and stores
    // of the rows and 8-byte code stores, so the rows must start on 16 bytes.
    // K32 blocks: rows spread over work-groups, one chunk per thread (RMSNorm
    // with many rows: one work-group per row, up to 20480 elements).
    // Per-token: spread as well while one work-group per row would leave CUs
    // idle (T below the CU count) and every work-group can hold its row (at
    // most 12 chunks per thread, K <= 24576), else one work-group per row (up
    // to 20480 elements; T=1, K=17408: 4.5 us on one 1024-thread work-group
    // before the rows were spread, 3.3 us spread).
    auto al = [](const void *p, uintptr_t m) { return ((uintptr_t)p & (m - 1)) == 0; };
    const int nch = a.K / 8;
    const int G = (nch + kQThreads - 1) / kQThreads;   // work-groups per spread row
    if (a.K % 32 == 0 && al(a.x, 16) && al(a.up, 16) && al(a.w, 16) && al(a.out, 16) && al(a.q, 8) &&
        (long long)a.T * G < (1ll << 31)) {
        auto spread = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((unsigned)(a.T * G)), dim3(kQThreads), 0, st, a, G);
            return hipGetLastError() == hipSuccess ? 0 : -6;
        };
        auto per_row = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(a.T), dim3(kQThreads), 0, st, a);
            return hipGetLastError() == hipSuccess ? 0 : -6;
        };
        const int cus = device_cus();
        if (block == 32) {
            // RMSNorm's row sum is computed by every work-group of a spread
            // row: with many rows, once per row instead (T=512, H=17408:
            // 50 us spread)
            if (P != kRmsNorm || a.T < cus) return spread(quantize_spread_kernel<P, 1, false>);
            if constexpr (P == kRmsNorm) {
                if (nch <= 2 * kQThreads) return per_row(quantize_tok_kernel<P, 2, kQThreads, false>);
                if (nch <= 3 * kQThreads) return per_row(quantize_tok_kernel<P, 3, kQThreads, false>);
                if (nch <= 4 * kQThreads) return per_row(quantize_tok_kernel<P, 4, kQThreads, false>);
                if (nch <= 10 * kQThreads) return per_row(quantize_tok_kernel<P, 10, kQThreads, false>);
            }
        } else {
            if (a.T < cus && G <= 12) {
                if (G <= 1) return spread(quantize_spread_kernel<P, 1, true>);
                if (G <= 2) return spread(quantize_spread_kernel<P, 2, true>);
                if (G <= 3) return spread(quantize_spread_kernel<P, 3, true>);
                if (G <= 5) return spread(quantize_spread_kernel<P, 5, true>);
                if (G <= 9) return spread(quantize_spread_kernel<P, 9, true>);
                return spread(quantize_spread_kernel<P, 12, true>);
            }
            // rows past 16384 elements: 1024 threads per row fill the CUs'
            // wave slots at a few hundred rows (T=512, K=17408: 7.9 against
            // 8.7 us); shorter rows would leave a third of those threads idle
            // (T=2048, K=5120: 13.3 against 9.5 us)
            if constexpr (P != kRmsNorm) {
                if (nch > 2048 && nch <= 3072) {
                    hipLaunchKernelGGL((quantize_tok_kernel<P, 3, 1024>), dim3(a.T), dim3(1024), 0, st, a);
                    return hipGetLastError() == hipSuccess ? 0 : -6;
                }
            }
            if (nch <= 2 * kQThreads) return per_row(quantize_tok_kernel<P, 2>);
            if (nch <= 3 * kQThreads) return per_row(quantize_tok_kernel<P, 3>);
            if (nch <= 4 * kQThreads) return per_row(quantize_tok_kernel<P, 4>);
            if (nch <= 10 * kQThreads) return per_row(quantize_tok_kernel<P, 10>);
        }
    }
    if (block == 32)
        hipLaunchKernelGGL((quantize_kernel<P, false>), dim3(a.T), dim3(kQThreads), 0, st, a);
    else
        hipLaunchKernelGGL((quantize_kernel<P, true>), dim3(a.T), dim3(kQThreads), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

// s4 activations of the W4A4 GEMM (x_quantize_act_chunk_s4,
// kernels_dpas.cpp:1492-1498 over quantize_act_chunk_subgroup<true>,
// 1149-1197): per (token, K64) block s = absmax/7 (1 when the max is not
// positive), q = clamp(rint(v / s), -7, 7) and the exact code sum. One thread
// per 8 consecutive elements: a K64 block is 8 consecutive lanes (3-step
// shuffles) and its 8 codes pack into one dword of the s4 tile layout, where
// chunk c (k = 128kb + 8c .. +7) of token t lands at dword
// (kb*T + t)*16 + 4(c & 3) + (c >> 2), codes 0..3 in the low nibbles of its
// bytes and 4..7 in the high nibbles. Scales and sums are [K/64][T].
template <int P>
__global__ __launch_bounds__(256) void quantize_s4_kernel(const void *x, int T, int K, uint32_t *q4,
                                                          float *scale, int32_t *sum) {
    const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int cpt = K / 8;                                   // chunks per token, a multiple of 16
    const bool live = id < (size_t)T * cpt;                  // 8-lane groups are live or dead as a whole
    const int t = live ? (int)(id / cpt) : 0;
    const int idx = live ? (int)(id % cpt) : 0;
    float v[8];
    if (live) {
        if constexpr (P == kLoadBF16) {
            const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + (size_t)t * K + 8 * idx);
            const uint32_t h[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = __uint_as_float(h[j] << 16);
                v[2 * j + 1] = __uint_as_float(h[j] & 0xFFFF0000u);
            }
        } else {
            const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + (size_t)t * K + 8 * idx);
            const float4 x0 = src[0], x1 = src[1];
            v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
            v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
    mx = oct_max(mx);
    const float s = (mx > 0.0f) ? (mx / 7.0f) : 1.0f;
    float k[8];
    rint_quot(v, s, k);
    uint32_t w = 0;
    int sm = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = (int)clampf(k[j], -7.0f, 7.0f);
        sm += q;
        w |= (uint32_t)(q & 0xF) << (j < 4 ? 8 * j : 8 * (j - 4) + 4);
    }
    sm = oct_sum(sm);
    if (live) {
        const int kb = idx >> 4, c = idx & 15;
        q4[((size_t)kb * T + t) * 16 + 4 * (c & 3) + (c >> 2)] = w;
        if ((idx & 7) == 0) {
            const size_t o = (size_t)(idx >> 3) * T + t;
            scale[o] = s;
            sum[o] = sm;
        }
    }
}

int launch_quantize_s4(const void *x, int x_dtype, int T, int K, uint8_t *q4, float *scale,
                       int32_t *sum, hipStream_t st) {
    const size_t threads = (size_t)T * (K / 8);
    const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    uint32_t *q = reinterpret_cast<uint32_t *>(q4);
    if (x_dtype == 1)
        hipLaunchKernelGGL((quantize_s4_kernel<kLoadBF16>), grid, block, 0, st, x, T, K, q, scale, sum);
    else
        hipLaunchKernelGGL((quantize_s4_kernel<kLoadF32>), grid, block, 0, st, x, T, K, q, scale, sum);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_quantize(const void *x, int x_dtype, int T, int K, int block, int8_t *q,
                    float *scale, int32_t *sum, hipStream_t st) {
    QuantArgs a{x, nullptr, nullptr, nullptr, q, scale, sum, T, K, 0.0f};
    return x_dtype == 1 ? launch_q<kLoadBF16>(a, block, st) : launch_q<kLoadF32>(a, block, st);
}

int launch_silu_mul_quant(float *out, const float *gate, const float *up, int T, int K,
                          int block, int8_t *q, float *scale, int32_t *sum, hipStream_t st) {
    QuantArgs a{gate, up, nullptr, out, q, scale, sum, T, K, 0.0f};
    return launch_q<kSiluMul>(a, block, st);
}

// x_rmsnorm_chunk (kernels_dpas.cpp:1124-1144): the (1+w) RMSNorm of
// x_rmsnorm_quant over T rows without the quantizer; the sum of squares and
// the scaling are the quantizer's own (same partial sums, same reduction), so
// both entry points write identical rows.
__global__ __launch_bounds__(kQThreads) void rmsnorm_kernel(QuantArgs a) {
    __shared__ float red[kQThreads / 64];
    const int t = blockIdx.x, K = a.K, tid = threadIdx.x;
    const float rms_inv = row_rms_inv(a, t, red);
    for (int k0 = tid; k0 < K; k0 += kQThreads * kQU) {
        float v[kQU];
#pragma unroll
        for (int u = 0; u < kQU; ++u) v[u] = produce<kRmsNorm>(a, t, min(k0 + u * kQThreads, K - 1), rms_inv);
#pragma unroll
        for (int u = 0; u < kQU; ++u)
            if (k0 + u * kQThreads < K) a.out[(size_t)t * K + k0 + u * kQThreads] = v[u];
    }
}

int launch_rmsnorm(float *out, const float *in, const uint16_t *w, int T, int H, float eps, hipStream_t st) {
    QuantArgs a{in, nullptr, w, out, nullptr, nullptr, nullptr, T, H, eps};
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(kQThreads), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_rmsnorm_quant(float *out, const float *in, const uint16_t *w, int T, int H, float eps,
                         int block, int8_t *q, float *scale, int32_t *sum, hipStream_t st) {
    QuantArgs a{in, nullptr, w, out, q, scale, sum, T, H, eps};
    return launch_q<kRmsNorm>(a, block, st);
}

}  // namespace kxw4
