// kxw4_pack.hip — load-time weight kernels: pack natural int4 codes into the
// gfx950 tile layout, unpack it, import the reference's DPAS layout, and the
// E2M3 -> asymmetric int4 repack (kernels_dpas.cpp:229-344; K32, K16 and
// K64 groups), and the W8A8 tier's int8 pack and repack.
//
// Packed tile (16 rows x 128 K, 1024 bytes): lane l owns bytes [16l, 16l+16),
// row l%16; dword i of the lane holds k = 32i + 8(l/16) + b with b = 0..3 in
// the low nibbles of bytes 0..3 and b = 4..7 in the high nibbles, so one
// 16-byte load per lane feeds two K64 MFMAs (or four K32 MFMAs). The W8A8
// tier's int8 tiles (2048 bytes) follow the same K slots, below.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"

namespace kxw4 {

// Tile-local coordinates of packed dword `d` (0..255 within a tile).
struct DwordCoord {
    int row;   // row within the 16-row group
    int k0;    // first K of the dword, within the 128-K tile
};

__device__ __forceinline__ DwordCoord dword_coord(int d) {
    const int lane = d >> 2, i = d & 3;
    return {lane & 15, 32 * i + 8 * (lane >> 4)};
}

__global__ void pack_codes_kernel(const int8_t *__restrict__ codes, int M, int K,
                                  uint32_t *__restrict__ out) {
    const size_t total = (size_t)M * K / 8;
    const size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= total) return;
    const int NT = K / kTileK;
    const size_t tile = d >> 8;
    const DwordCoord c = dword_coord((int)(d & 255));
    const int rg = (int)(tile / NT), kb = (int)(tile % NT);
    const int8_t *src = codes + (size_t)(rg * 16 + c.row) * K + kb * kTileK + c.k0;
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t lo = (uint32_t)src[b] & 0xFu, hi = (uint32_t)src[b + 4] & 0xFu;
        w |= (lo | (hi << 4)) << (8 * b);
    }
    out[d] = w;
}

__global__ void unpack_codes_kernel(const uint32_t *__restrict__ in, int M, int K,
                                    int8_t *__restrict__ codes) {
    const size_t total = (size_t)M * K / 8;
    const size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= total) return;
    const int NT = K / kTileK;
    const size_t tile = d >> 8;
    const DwordCoord c = dword_coord((int)(d & 255));
    const int rg = (int)(tile / NT), kb = (int)(tile % NT);
    int8_t *dst = codes + (size_t)(rg * 16 + c.row) * K + kb * kTileK + c.k0;
    const uint32_t w = in[d];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        dst[b] = (int8_t)sext4(w >> (8 * b));
        dst[b + 4] = (int8_t)sext4(w >> (8 * b + 4));
    }
}

// scales [M][G] (natural) <-> [M/16][G][16] (row within row-group fastest).
__global__ void scales_to_tiled_kernel(const uint16_t *__restrict__ in, int M, int G,
                                       uint16_t *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * G) return;
    const int row = (int)(i / G), g = (int)(i % G);
    out[((size_t)(row >> 4) * G + g) * 16 + (row & 15)] = in[i];
}

__global__ void scales_to_natural_kernel(const uint16_t *__restrict__ in, int M, int G,
                                         uint16_t *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * G) return;
    const int row = (int)(i / G), g = (int)(i % G);
    out[i] = in[((size_t)(row >> 4) * G + g) * 16 + (row & 15)];
}

// Reference layout (kernels_dpas.cpp:327-342): tile (rg, kt32) of 256 bytes;
// row n owns bytes [16n, 16n+16); k = 32kt + 8i + 2b + h sits in dword i,
// byte b, low nibble for h = 0.
__device__ __forceinline__ uint32_t ref_nibble(const uint8_t *__restrict__ ref, int Kt, int row,
                                               int k) {
    const int rg = row >> 4, n = row & 15, kt = k >> 5, j = k & 31;
    const uint8_t v = ref[((size_t)rg * Kt + kt) * 256u + (size_t)(n * 4 + (j >> 3)) * 4u +
                          (size_t)((j & 7) >> 1)];
    return (j & 1) ? (uint32_t)(v >> 4) : (uint32_t)(v & 0xFu);
}

__global__ void import_ref_codes_kernel(const uint8_t *__restrict__ ref, int M, int K,
                                        uint32_t *__restrict__ out) {
    const size_t total = (size_t)M * K / 8;
    const size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= total) return;
    const int NT = K / kTileK, Kt = K / 32;
    const size_t tile = d >> 8;
    const DwordCoord c = dword_coord((int)(d & 255));
    const int rg = (int)(tile / NT), kb = (int)(tile % NT);
    const int row = rg * 16 + c.row, k = kb * kTileK + c.k0;
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t lo = ref_nibble(ref, Kt, row, k + b);
        const uint32_t hi = ref_nibble(ref, Kt, row, k + b + 4);
        w |= (lo | (hi << 4)) << (8 * b);
    }
    out[d] = w;
}

// ---- E2M3 -> asymmetric int4 (kernels_dpas.cpp:49-69, 229-344) -----------

__device__ __forceinline__ float e2m3f(uint32_t c) {
    const float m = (float)(c & 7u);
    const uint32_t e = (c >> 3) & 3u;
    const float v = (e == 0) ? m * 0.125f : (1.0f + m * 0.125f) * (float)(1u << (e - 1));
    return (c & 0x20u) ? -v : v;
}

__device__ __forceinline__ uint32_t e2m3_code_at(const uint8_t *__restrict__ payload, int Kt,
                                                 int row, int col) {
    const int mt = row >> 4;
    const int kt = col >> 5;
    const int lane = (((row & 15) >> 1) << 2) | ((col & 31) >> 3);
    const int idx = (((col >> 2) & 1) << 3) | ((row & 1) << 2) | (col & 3);
    const int bit = 6 * idx;
    const uint8_t *p = payload + ((size_t)mt * Kt + kt) * 384u + (size_t)lane * 12u;
    uint32_t bits = p[bit >> 3];
    if ((bit & 7) > 2) bits |= (uint32_t)p[(bit >> 3) + 1] << 8;
    return (bits >> (bit & 7)) & 0x3fu;
}

// fit_int4_asym with the least-squares sums evaluated as fused multiply-adds.
template <int N>
__device__ uint16_t fit_int4_asym(const float *wf, int *out_z) {
    float lo = 0.0f, hi = 0.0f;
    for (int j = 0; j < N; ++j) {
        lo = fminf(lo, wf[j]);
        hi = fmaxf(hi, wf[j]);
    }
    float s = (hi - lo) / 15.0f;
    if (!(s > 0.0f)) s = 1.0f;
    for (int iter = 0; iter < 3; ++iter) {
        const int zi = (int)clampf(rintf(-lo / s) - 8.0f, -8.0f, 7.0f);
        float num = 0.0f, den = 0.0f;
        for (int j = 0; j < N; ++j) {
            const float q = clampf(rintf(wf[j] / s + (float)zi), -8.0f, 7.0f);
            const float c = q - (float)zi;
            num = __builtin_fmaf(wf[j], c, num);
            den = __builtin_fmaf(c, c, den);
        }
        if (den > 0.0f) s = num / den;
    }
    *out_z = (int)clampf(rintf(-lo / s) - 8.0f, -8.0f, 7.0f);
    uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)s);
    sh = (uint16_t)((sh + 8u) & 0xFFF0u);
    return sh;
}

// One thread per (row, group): decode, fit, then write the group's packed
// dwords (a group of 32 or 64 K owns whole dwords in every lane group) and
// its FP16|zp scale.
template <int GROUP>
__global__ void repack_e2m3_kernel(const uint8_t *__restrict__ payload,
                                   const float *__restrict__ bs, int scale_cols, int M, int K,
                                   uint32_t *__restrict__ out_codes,
                                   uint16_t *__restrict__ out_scales) {
    const int G = K / GROUP, Kt = K / 32, NT = K / kTileK;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * G) return;
    const int row = (int)(i / G), g = (int)(i % G);
    const int mt = row >> 4;
    const int k0 = g * GROUP;
    float wf[GROUP];
#pragma unroll
    for (int j = 0; j < GROUP; ++j) {
        const int kt = (k0 + j) >> 5;
        const int sc = (scale_cols == Kt) ? kt : (kt >> 2);
        const float b = bs[(size_t)(mt >> 3) * scale_cols + sc];
        wf[j] = e2m3f(e2m3_code_at(payload, Kt, row, k0 + j)) * b;
    }
    int z = 0;
    const uint16_t sh = fit_int4_asym<GROUP>(wf, &z);
    out_scales[((size_t)mt * G + g) * 16 + (row & 15)] = (uint16_t)(sh | (z & 0xF));
    const float gs = half_bits_to_float(sh);
    uint8_t q4[GROUP];
#pragma unroll
    for (int j = 0; j < GROUP; ++j)
        q4[j] = (uint8_t)((int)clampf(rintf(wf[j] / gs + (float)z), -8.0f, 7.0f) & 0xF);
    // Dwords of this group: K32 unit u = (k0 + 32v) covers tile kb, dword
    // i = (u % 128) / 32, for the four lane groups gl (k = 32i + 8gl + b).
    const int n = row & 15;
#pragma unroll
    for (int v = 0; v < GROUP / 32; ++v) {
        const int k = k0 + 32 * v;
        const int kb = k / kTileK, di = (k % kTileK) / 32;
        uint32_t *tile = out_codes + ((size_t)mt * NT + kb) * 256;
#pragma unroll
        for (int gl = 0; gl < 4; ++gl) {
            uint32_t w = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 32 * v + 8 * gl + b;
                w |= ((uint32_t)q4[j] | ((uint32_t)q4[j + 4] << 4)) << (8 * b);
            }
            tile[(n + 16 * gl) * 4 + di] = w;
        }
    }
}

// ---- the W8A8 tier (kernels_dpas.cpp:346-399, 558-575) --------------------
//
// W8 tile (16 rows x 128 K, 2048 bytes): half h at byte 1024h; lane l owns
// bytes [1024h + 16l, +16), row l%16, holding K32 unit j = 2h (bytes 0..7)
// and j = 2h + 1 (bytes 8..15); byte b of a unit is k = 32j + 8(l/16) + b.
// So one 16-byte load per lane and half is the operand of two K32 MFMAs,
// with the same K slots the W4 unpack produces.
__device__ __forceinline__ DwordCoord dword_coord_s8(int d) {
    const int h = d >> 8, lane = (d >> 2) & 63, e = d & 3;
    return {lane & 15, 32 * (2 * h + (e >> 1)) + 8 * (lane >> 4) + 4 * (e & 1)};
}

__global__ void pack_s8_kernel(const int8_t *__restrict__ codes, int M, int K, uint32_t *__restrict__ out) {
    const size_t total = (size_t)M * K / 4;
    const size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= total) return;
    const int NT = K / kTileK;
    const size_t tile = d >> 9;
    const DwordCoord c = dword_coord_s8((int)(d & 511));
    const int rg = (int)(tile / NT), kb = (int)(tile % NT);
    const int8_t *src = codes + (size_t)(rg * 16 + c.row) * K + kb * kTileK + c.k0;
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) w |= ((uint32_t)(uint8_t)src[b]) << (8 * b);
    out[d] = w;
}

__global__ void unpack_s8_kernel(const uint32_t *__restrict__ in, int M, int K, int8_t *__restrict__ codes) {
    const size_t total = (size_t)M * K / 4;
    const size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= total) return;
    const int NT = K / kTileK;
    const size_t tile = d >> 9;
    const DwordCoord c = dword_coord_s8((int)(d & 511));
    const int rg = (int)(tile / NT), kb = (int)(tile % NT);
    int8_t *dst = codes + (size_t)(rg * 16 + c.row) * K + kb * kTileK + c.k0;
    const uint32_t w = in[d];
#pragma unroll
    for (int b = 0; b < 4; ++b) dst[b] = (int8_t)(w >> (8 * b));
}

// w8_repack_kernel's fit with the least-squares sums as fused multiply-adds:
// s = max(hi/127, neg/128), two refinements, FP16 by round to nearest even.
__device__ uint16_t fit_int8(const float *wf) {
    float hi = 0.0f, neg = 0.0f;
    for (int j = 0; j < 32; ++j) {
        hi = fmaxf(hi, wf[j]);
        neg = fmaxf(neg, -wf[j]);
    }
    float s = fmaxf(hi / 127.0f, neg / 128.0f);
    if (!(s > 0.0f)) s = 1.0f;
    for (int iter = 0; iter < 2; ++iter) {
        float num = 0.0f, den = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float q = clampf(rintf(wf[j] / s), -128.0f, 127.0f);
            num = __builtin_fmaf(wf[j], q, num);
            den = __builtin_fmaf(q, q, den);
        }
        if (den > 0.0f) s = num / den;
    }
    return __builtin_bit_cast(uint16_t, (_Float16)s);
}

// One thread per (row, K32): decode, fit, write the unit's 8 dwords (two per
// lane group) and its tiled FP16 scale.
__global__ void repack_e2m3_s8_kernel(const uint8_t *__restrict__ payload, const float *__restrict__ bs,
                                      int scale_cols, int M, int K, uint32_t *__restrict__ out_codes,
                                      uint16_t *__restrict__ out_scales) {
    const int Kt = K / 32, NT = K / kTileK;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * Kt) return;
    const int row = (int)(i / Kt), kt = (int)(i % Kt);
    const int mt = row >> 4, n = row & 15;
    const int sc = (scale_cols == Kt) ? kt : (kt >> 2);
    const float b = bs[(size_t)(mt >> 3) * scale_cols + sc];
    float wf[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) wf[j] = e2m3f(e2m3_code_at(payload, Kt, row, kt * 32 + j)) * b;
    const uint16_t sh = fit_int8(wf);
    out_scales[((size_t)mt * Kt + kt) * 16 + n] = sh;
    const float st = half_bits_to_float(sh);
    const int kb = kt >> 2, j = kt & 3;
    uint32_t *tile = out_codes + ((size_t)mt * NT + kb) * 512 + 256 * (j >> 1);
#pragma unroll
    for (int gl = 0; gl < 4; ++gl)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            uint32_t w = 0;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const int q = (int)clampf(rintf(wf[8 * gl + 4 * e + bb] / st), -128.0f, 127.0f);
                w |= (uint32_t)(uint8_t)q << (8 * bb);
            }
            tile[(n + 16 * gl) * 4 + 2 * (j & 1) + e] = w;
        }
}

// Mode 1, the K16 tier (kernels_dpas.cpp:287-296): one thread per (row, K32
// tile) fits its two K16 halves (FP16|zp each); half h owns dword kt % 4 of
// lane groups 2h and 2h + 1.
__global__ void repack_e2m3_k16_kernel(const uint8_t *__restrict__ payload,
                                       const float *__restrict__ bs, int scale_cols, int M, int K,
                                       uint32_t *__restrict__ out_codes,
                                       uint16_t *__restrict__ out_scales) {
    const int Kt = K / 32, NT = K / kTileK, G = K / 16;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * Kt) return;
    const int row = (int)(i / Kt), kt = (int)(i % Kt);
    const int mt = row >> 4, n = row & 15;
    const int sc = (scale_cols == Kt) ? kt : (kt >> 2);
    const float b = bs[(size_t)(mt >> 3) * scale_cols + sc];
    float wf[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) wf[j] = e2m3f(e2m3_code_at(payload, Kt, row, kt * 32 + j)) * b;
    uint8_t q4[32];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int z = 0;
        const uint16_t sh = fit_int4_asym<16>(wf + 16 * h, &z);
        out_scales[((size_t)mt * G + 2 * kt + h) * 16 + n] = (uint16_t)(sh | (z & 0xF));
        const float gs = half_bits_to_float(sh);
#pragma unroll
        for (int j = 16 * h; j < 16 * h + 16; ++j)
            q4[j] = (uint8_t)((int)clampf(rintf(wf[j] / gs + (float)z), -8.0f, 7.0f) & 0xF);
    }
    uint32_t *tile = out_codes + ((size_t)mt * NT + kt / 4) * 256;
#pragma unroll
    for (int gl = 0; gl < 4; ++gl) {
        uint32_t w = 0;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb)
            w |= ((uint32_t)q4[8 * gl + bb] | ((uint32_t)q4[8 * gl + bb + 4] << 4)) << (8 * bb);
        tile[(n + 16 * gl) * 4 + (kt & 3)] = w;
    }
}

static inline unsigned blocks_for(size_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

int launch_pack_s8(const int8_t *codes, const uint16_t *scales, int M, int K, uint8_t *out_codes,
                   uint16_t *out_scales, hipStream_t st) {
    const size_t nd = (size_t)M * K / 4, ns = (size_t)M * (K / 32);
    hipLaunchKernelGGL(pack_s8_kernel, dim3(blocks_for(nd, 256)), dim3(256), 0, st, codes, M, K,
                       reinterpret_cast<uint32_t *>(out_codes));
    hipLaunchKernelGGL(scales_to_tiled_kernel, dim3(blocks_for(ns, 256)), dim3(256), 0, st, scales, M,
                       K / 32, out_scales);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_unpack_s8(const uint8_t *codes, const uint16_t *scales, int M, int K, int8_t *out_codes,
                     uint16_t *out_scales, hipStream_t st) {
    const size_t nd = (size_t)M * K / 4, ns = (size_t)M * (K / 32);
    hipLaunchKernelGGL(unpack_s8_kernel, dim3(blocks_for(nd, 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t *>(codes), M, K, out_codes);
    if (out_scales)
        hipLaunchKernelGGL(scales_to_natural_kernel, dim3(blocks_for(ns, 256)), dim3(256), 0, st, scales,
                           M, K / 32, out_scales);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_repack_e2m3_s8(const uint8_t *payload, const float *bs, int scale_cols, int M, int K,
                          uint8_t *out_codes, uint16_t *out_scales, hipStream_t st) {
    const size_t n = (size_t)M * (K / 32);
    hipLaunchKernelGGL(repack_e2m3_s8_kernel, dim3(blocks_for(n, 128)), dim3(128), 0, st, payload, bs,
                       scale_cols, M, K, reinterpret_cast<uint32_t *>(out_codes), out_scales);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_pack(const int8_t *codes, const uint16_t *scales, int M, int K, int group,
                uint8_t *out_codes, uint16_t *out_scales, hipStream_t st) {
    const size_t nd = (size_t)M * K / 8, ns = (size_t)M * (K / group);
    hipLaunchKernelGGL(pack_codes_kernel, dim3(blocks_for(nd, 256)), dim3(256), 0, st, codes, M,
                       K, reinterpret_cast<uint32_t *>(out_codes));
    hipLaunchKernelGGL(scales_to_tiled_kernel, dim3(blocks_for(ns, 256)), dim3(256), 0, st,
                       scales, M, K / group, out_scales);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_unpack(const uint8_t *codes, const uint16_t *scales, int M, int K, int group,
                  int8_t *out_codes, uint16_t *out_scales, hipStream_t st) {
    const size_t nd = (size_t)M * K / 8, ns = (size_t)M * (K / group);
    hipLaunchKernelGGL(unpack_codes_kernel, dim3(blocks_for(nd, 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t *>(codes), M, K, out_codes);
    if (out_scales)
        hipLaunchKernelGGL(scales_to_natural_kernel, dim3(blocks_for(ns, 256)), dim3(256), 0, st,
                           scales, M, K / group, out_scales);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_import_ref(const uint8_t *ref_codes, const uint16_t *ref_scales, int M, int K,
                      int group, uint8_t *out_codes, uint16_t *out_scales, hipStream_t st) {
    const size_t nd = (size_t)M * K / 8, ns = (size_t)M * (K / group);
    hipLaunchKernelGGL(import_ref_codes_kernel, dim3(blocks_for(nd, 256)), dim3(256), 0, st,
                       ref_codes, M, K, reinterpret_cast<uint32_t *>(out_codes));
    if (hipMemcpyAsync(out_scales, ref_scales, ns * sizeof(uint16_t), hipMemcpyDeviceToDevice,
                       st) != hipSuccess)
        return -6;
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

int launch_repack_e2m3(const uint8_t *payload, const float *bs, int scale_cols, int M, int K,
                       int group, uint8_t *out_codes, uint16_t *out_scales, hipStream_t st) {
    const size_t n = (size_t)M * (K / group);
    uint32_t *oc = reinterpret_cast<uint32_t *>(out_codes);
    if (group == 16)
        hipLaunchKernelGGL(repack_e2m3_k16_kernel, dim3(blocks_for((size_t)M * (K / 32), 128)), dim3(128), 0,
                           st, payload, bs, scale_cols, M, K, oc, out_scales);
    else if (group == 32)
        hipLaunchKernelGGL(repack_e2m3_kernel<32>, dim3(blocks_for(n, 128)), dim3(128), 0, st,
                           payload, bs, scale_cols, M, K, oc, out_scales);
    else
        hipLaunchKernelGGL(repack_e2m3_kernel<64>, dim3(blocks_for(n, 128)), dim3(128), 0, st,
                           payload, bs, scale_cols, M, K, oc, out_scales);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace kxw4
