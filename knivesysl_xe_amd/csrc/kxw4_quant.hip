// kxw4_quant.hip — activation quantizers (kernels_dpas.cpp:188-223, 846-929,
// 1149-1207), one work-group per token row.
//
// A producer computes the fp32 value of element k (plain load, SiLU(g)*u, or
// (1+w) RMSNorm); the quantizer turns it into int8 with
//   s = absmax/127 (1 when the block max is not positive),
//   q = clamp(rint(v / s), -127, 127)          (IEEE division, NaN -> -127)
// over blocks of 32 K (reference mode) or the whole row (per-token mode), and
// writes exact int32 code sums per K32. Codes are stored in the MFMA slot
// order of each 64-element chunk (act_slot).
//
// Block 32: the 32 lanes of a half wave hold one block, so absmax and sums are
// half-wave shuffles and each element is produced once. Per-token: a first pass
// reduces the row absmax across the work-group, a second pass quantizes
// (producers are recomputed, bit-identically).
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

// The element loops below take kQU elements per thread and pass: all kQU
// loads are issued (at indices clamped into the row) before any is used, so a
// pass costs one memory round trip instead of one per element; the values of
// clamped positions are never used, and the arithmetic and its order are the
// element loop's.
constexpr int kQU = 8;

// 1 / sqrt(mean(x^2) + eps) of row t, summed in a fixed order: thread tid
// adds x[k]^2 for k = tid, tid + kQThreads, ... in turn, then the work-group
// sum (the work-group must have kQThreads threads)
__device__ __forceinline__ float row_rms_inv(const QuantArgs &a, int t, float *red) {
    const int K = a.K, tid = threadIdx.x;
    const float *row = static_cast<const float *>(a.x) + (size_t)t * K;
    float ss = 0.0f;
    for (int k0 = tid; k0 < K; k0 += kQThreads * kQU) {
        float x[kQU];
#pragma unroll
        for (int u = 0; u < kQU; ++u) x[u] = row[min(k0 + u * kQThreads, K - 1)];
#pragma unroll
        for (int u = 0; u < kQU; ++u)
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
// (chunk tid + c*NT), every chunk's inputs loaded before any is used, at
// chunk indices clamped into the row (a chunk past the row holds the last
// chunk's values and is not used); the per-element arithmetic is produce's.
template <int P, int NCH, int NT>
__device__ __forceinline__ void chunk_values(const QuantArgs &a, int t, float rms_inv, float (&v)[NCH][8]) {
    const int nch = a.K / 8, tid = threadIdx.x;
    const size_t row0 = (size_t)t * a.K;
    uint4 raw[NCH][P == kLoadBF16 || P == kRmsNorm ? 1 : 2];
    float4 upv[P == kSiluMul ? NCH : 1][2];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = min(tid + c * NT, nch - 1);
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

// Per-token mode with plain loads, one pass: each thread holds chunks of 8
// consecutive elements (16-byte bf16 / 32-byte f32 loads) in registers for the
// whole row, so the row is read once. The MFMA slot order keeps the 8 codes of
// a chunk contiguous: chunk c of 64-element chunk h lands at byte
// 64h + 16(c & 3) + 8((c >> 2) & 1), one 8-byte store. The four chunks of a
// K32 block sit in four consecutive lanes, so their code sum is a 4-lane
// shuffle.
template <int P, int NCH, int NT = kQThreads>
__global__ __launch_bounds__(NT) void quantize_tok_kernel(QuantArgs a) {
    static_assert(P != kRmsNorm || NT == kQThreads, "the row sum's order assumes kQThreads threads");
    __shared__ float red[NT / 64];
    const int t = blockIdx.x, K = a.K, tid = threadIdx.x;
    const int nch = K / 8;
    float rms_inv = 0.0f;
    if constexpr (P == kRmsNorm) rms_inv = row_rms_inv(a, t, red);
    float v[NCH][8];
    chunk_values<P, NCH, NT>(a, t, rms_inv, v);
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (tid + c * NT < nch) {
            if (P >= kSiluMul && a.out) store_chunk_out<NCH>(a, t, tid + c * NT, v[c]);
#pragma unroll
            for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[c][j]));
        }
    }
    // work-group max (order-free, so any thread count gives the same bits)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) mx = fmaxf(mx, red[i]);
    const float s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
    if (tid == 0) a.scale[t] = s;
    int8_t *qrow = a.q + (size_t)t * K;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = tid + c * NT;
        // whole K32 blocks (4 chunks) per 4-lane group: nch % 4 == 0
        if (idx - (tid & 3) < nch) {
            uint32_t lo = 0, hi = 0;
            int sum = 0;
            if (idx < nch) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int8_t q = quantize_one(v[c][j], s);
                    sum += q;
                    if (j < 4) lo |= (uint32_t)(uint8_t)q << (8 * j);
                    else hi |= (uint32_t)(uint8_t)q << (8 * (j - 4));
                }
                *reinterpret_cast<uint2 *>(qrow + 64 * (idx >> 3) + 16 * (idx & 3) + 8 * ((idx >> 2) & 1)) =
                    make_uint2(lo, hi);
            }
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            if (a.sum && (idx & 3) == 0 && idx < nch) a.sum[(size_t)t * (K / 32) + (idx >> 2)] = sum;
        }
    }
}

// Reference mode (K32 blocks) in one pass: each thread holds chunks of 8
// consecutive elements, so a K32 block is 4 consecutive lanes and its absmax
// and code sum are two lane shuffles each (one element per lane would take
// five dependent shuffles per reduction and element). Every chunk's inputs
// are loaded before any is used, at chunk indices clamped into the row; the
// per-element arithmetic is the element loop's (produce), and the codes of a
// chunk are one 8-byte store in the slot order. RMSNorm keeps kQThreads
// threads for its fixed-order row sum.
template <int P, int NCH, int NT = kQThreads>
__global__ __launch_bounds__(NT) void quantize_blk_kernel(QuantArgs a) {
    static_assert(P != kRmsNorm || NT == kQThreads, "the row sum's order assumes kQThreads threads");
    __shared__ float red[kQThreads / 64];
    const int t = blockIdx.x, K = a.K, tid = threadIdx.x;
    const int nch = K / 8;
    float rms_inv = 0.0f;
    if constexpr (P == kRmsNorm) rms_inv = row_rms_inv(a, t, red);
    const size_t row0 = (size_t)t * K;
    float v[NCH][8];
    chunk_values<P, NCH, NT>(a, t, rms_inv, v);
    int8_t *qrow = a.q + row0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = tid + c * NT;
        // a K32 block's four chunks are all in the row or all past it
        const bool in = idx < nch;
        if (a.out && in) store_chunk_out<NCH>(a, t, idx, v[c]);
        float mx = fabsf(v[c][0]);
#pragma unroll
        for (int j = 1; j < 8; ++j) mx = fmaxf(mx, fabsf(v[c][j]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const float sc = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
        uint32_t lo = 0, hi = 0;
        int sum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int8_t q = quantize_one(v[c][j], sc);
            sum += q;
            if (j < 4) lo |= (uint32_t)(uint8_t)q << (8 * j);
            else hi |= (uint32_t)(uint8_t)q << (8 * (j - 4));
        }
        if (in) *reinterpret_cast<uint2 *>(qrow + 64 * (idx >> 3) + 16 * (idx & 3) + 8 * ((idx >> 2) & 1)) =
                    make_uint2(lo, hi);
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if (in && (idx & 3) == 0) {
            a.scale[(size_t)t * (K / 32) + (idx >> 2)] = sc;
            if (a.sum) a.sum[(size_t)t * (K / 32) + (idx >> 2)] = sum;
        }
    }
}

template <int P>
static int launch_q(const QuantArgs &a, int block, hipStream_t st) {
    // One pass with the row's chunks in registers, up to 20480 elements:
    // per-token (block 0) on quantize_tok_kernel, K32 blocks on
    // quantize_blk_kernel; 16-byte vector loads and stores of the rows and
    // 8-byte code stores, so the rows must start on 16 bytes. With few
    // tokens a row's work-group is most of the launch, so it takes 1024
    // threads (more loads in flight per row; T=1, K=17408: 6.3 -> 4.5 us);
    // RMSNorm keeps 256 for its fixed-order row sum.
    auto al = [](const void *p, uintptr_t m) { return ((uintptr_t)p & (m - 1)) == 0; };
    const int nch = a.K / 8;
    if (a.K % 32 == 0 && al(a.x, 16) && al(a.up, 16) && al(a.w, 16) && al(a.out, 16) && al(a.q, 8)) {
        auto run = [&](auto kernel1024_1, auto kernel1024_3, auto kernel2, auto kernel4, auto kernel10) {
            if (P != kRmsNorm && a.T < 64 && nch <= 3 * 1024) {
                if (nch <= 1024) hipLaunchKernelGGL(kernel1024_1, dim3(a.T), dim3(1024), 0, st, a);
                else hipLaunchKernelGGL(kernel1024_3, dim3(a.T), dim3(1024), 0, st, a);
                return true;
            }
            if (nch > 10 * kQThreads) return false;
            if (nch <= 2 * kQThreads) hipLaunchKernelGGL(kernel2, dim3(a.T), dim3(kQThreads), 0, st, a);
            else if (nch <= 4 * kQThreads) hipLaunchKernelGGL(kernel4, dim3(a.T), dim3(kQThreads), 0, st, a);
            else hipLaunchKernelGGL(kernel10, dim3(a.T), dim3(kQThreads), 0, st, a);
            return true;
        };
        // (RMSNorm has no 1024-thread instances: the null pointers are never launched)
        constexpr bool k1024 = P != kRmsNorm;
        bool done;
        if (block == 32)
            done = run(k1024 ? quantize_blk_kernel<P, 1, k1024 ? 1024 : kQThreads> : nullptr,
                       k1024 ? quantize_blk_kernel<P, 3, k1024 ? 1024 : kQThreads> : nullptr,
                       quantize_blk_kernel<P, 2>, quantize_blk_kernel<P, 4>, quantize_blk_kernel<P, 10>);
        else
            done = run(k1024 ? quantize_tok_kernel<P, 1, k1024 ? 1024 : kQThreads> : nullptr,
                       k1024 ? quantize_tok_kernel<P, 3, k1024 ? 1024 : kQThreads> : nullptr,
                       quantize_tok_kernel<P, 2>, quantize_tok_kernel<P, 4>, quantize_tok_kernel<P, 10>);
        if (done) return hipGetLastError() == hipSuccess ? 0 : -6;
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
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
    const float s = (mx > 0.0f) ? (mx / 7.0f) : 1.0f;
    uint32_t w = 0;
    int sm = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = (int)clampf(rintf(v[j] / s), -7.0f, 7.0f);
        sm += q;
        w |= (uint32_t)(q & 0xF) << (j < 4 ? 8 * j : 8 * (j - 4) + 4);
    }
    sm += __shfl_xor(sm, 1, 64);
    sm += __shfl_xor(sm, 2, 64);
    sm += __shfl_xor(sm, 4, 64);
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
