// kxw4_probe.hip — machine probes behind the roofline figures, the MI355X
// counterpart of the reference's xpu/probe/dpas_probe.cpp (DPAS rate table
// with all-ones operands, pure-read bandwidth; results in
// xpu/PROBE_RESULTS.md:8-33).
//
// MFMA rate: every wave runs four independent accumulator chains of one int8
// MFMA shape with all-ones operands, so each accumulator ends at iters * K
// exactly; the wave writes that value only when all of its accumulators hold
// it (else -1), which proves that every MFMA ran at the stated depth.
//
// Read rate: a grid-stride sweep of 16-byte loads, a ring of 2-8 of them in
// flight per lane, XOR-folded into one word per wave (every byte counts), in
// one of a few launch shapes; the caller times each shape and keeps the
// fastest (the grid-stride pattern measured fastest for a pure stream on
// this GPU).
//
// Issue mix: the per-token GEMM's inner work without memory. A "block" is
// four dependent v_mfma_i32_32x32x32_i8 (one 128-K step of a 32x32 output
// block) and/or its FP32 chain (16 int->float conversions and 16 FMAs per
// lane). Mode 0 runs only the MFMAs, 1 only the chain, 2 both in one wave as
// the GEMM interleaves them (block b's MFMAs with block b-1's chain), 3 both
// in different waves of a SIMD; timed and counted per mode and waves per
// SIMD, it gives what one SIMD can issue of each.
#include "kxw4_device.hpp"
#include "kxw4_internal.hpp"
#include "../../include/kxw4.h"

namespace kxw4 {

constexpr int kProbeWaves = 4;              // waves per work-group (one per SIMD)
constexpr int kProbeGroupsPerCu = 2;

template <int SHAPE>
__global__ __launch_bounds__(64 * kProbeWaves) void probe_mfma_kernel(int iters, int32_t *sink) {
    const int lane = threadIdx.x & 63;
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    int32_t want, ok = 1;
    if constexpr (SHAPE == 0) {
        // v_mfma_i32_32x32x32_i8: 16 results per lane, K = 32
        v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma32(ones, ones, c0);
            c1 = mfma32(ones, ones, c1);
            c2 = mfma32(ones, ones, c2);
            c3 = mfma32(ones, ones, c3);
        }
        want = iters * 32;
#pragma unroll
        for (int r = 0; r < 16; ++r) ok &= (c0[r] == want) & (c1[r] == want) & (c2[r] == want) & (c3[r] == want);
    } else {
        // v_mfma_i32_16x16x64_i8: 4 results per lane, K = 64
        v4i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma_k64(ones, ones, c0);
            c1 = mfma_k64(ones, ones, c1);
            c2 = mfma_k64(ones, ones, c2);
            c3 = mfma_k64(ones, ones, c3);
        }
        want = iters * 64;
#pragma unroll
        for (int r = 0; r < 4; ++r) ok &= (c0[r] == want) & (c1[r] == want) & (c2[r] == want) & (c3[r] == want);
    }
    // every lane must agree: the wave's result is want only if all 64 did
    const bool all = __all(ok != 0);
    if (lane == 0) sink[blockIdx.x * kProbeWaves + (threadIdx.x >> 6)] = all ? want : -1;
}

// A ring of U loads in flight per lane over the lane's grid-stride sequence:
// each slot is refilled right after it is consumed, so the lane never drains.
template <int U>
__global__ __launch_bounds__(1024) void probe_read_kernel(const v4u *p, size_t n16, uint32_t *sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t cnt = i0 < n16 ? (n16 - i0 + stride - 1) / stride : 0;
    const v4u zero = {0u, 0u, 0u, 0u};
    v4u r[U];
#pragma unroll
    for (int j = 0; j < U; ++j) r[j] = (size_t)j < cnt ? p[i0 + j * stride] : zero;
    v4u e = zero;
    for (size_t k = 0; k < cnt; k += U) {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const v4u v = r[j];
            const size_t nx = k + U + j;
            r[j] = nx < cnt ? p[i0 + nx * stride] : zero;
            e ^= v;
        }
    }
    uint32_t acc = e.x ^ e.y ^ e.z ^ e.w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) sink[((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6] = acc;
}

// One wave's share of the issue probe in mode M (0: MFMAs, 1: the chain, 2:
// both interleaved); returns the lane's sum of its accumulators.
template <int M>
__device__ __forceinline__ float issue_run(int iters, float w, int lane) {
    constexpr int NB = 4;                                  // blocks per iteration
    v4i a = {lane, lane + 1, lane + 2, lane + 3}, b = {3, 5, 7, 9};
    v16i acc[2] = {};
    float f[NB][16];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) f[j][r] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j <= NB; ++j) {
            if (j < NB && M != 1) {
                v16i &p = acc[j & 1];
                const v16i z = {};
                // (opaque operands, so the MFMAs are not hoisted)
#pragma unroll
                for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(a[e]));
                p = mfma32(a, b, M == 2 ? z : p);
                p = mfma32(b, a, p);
                p = mfma32(a, b, p);
                p = mfma32(b, a, p);
            }
            if (j > 0 && M != 0) {
                v16i &p = acc[(j - 1) & 1];
                if (M != 2) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(p[r]));
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) f[j - 1][r] = __builtin_fmaf((float)p[r], w, f[j - 1][r]);
            }
            if (M == 2 && j > 0 && j < NB) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += f[j][r];
#pragma unroll
    for (int r = 0; r < 16; ++r) s += (float)acc[0][r] + (float)acc[1][r];
    return s;
}

template <int MODE>
__global__ __launch_bounds__(1024) void probe_issue_kernel(int iters, float w, float *sink) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float s;
    if constexpr (MODE == 3) {
        // waves 0-3 of each group of eight (one per SIMD) run the MFMAs,
        // waves 4-7 the chain: two loops, so neither holds the other's
        // registers
        s = ((wave >> 2) & 1) == 0 ? issue_run<0>(iters, w, lane) : issue_run<1>(iters, w, lane);
    } else {
        s = issue_run<MODE>(iters, w, lane);
    }
    // one word per wave, summed in a fixed order (the same every run)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) sink[blockIdx.x * (blockDim.x >> 6) + wave] = s;
}

// launch shapes of the read probe: (work-groups per CU, threads, ring depth)
struct ReadShape { int per_cu, threads, ring; };
constexpr ReadShape kReadShapes[] = {
    {1, 512, 4}, {2, 512, 4}, {1, 1024, 4}, {2, 256, 8}, {4, 256, 4}, {1, 512, 8}, {8, 256, 2}, {2, 1024, 2},
};
constexpr int kReadShapeCount = sizeof(kReadShapes) / sizeof(kReadShapes[0]);

// A wave that holds its stream until the host sets *flag (host-pinned
// memory, read at system scope) or max_ticks of the constant-rate wall clock
// have passed, whichever comes first, then writes 1 (released by the flag)
// or 2 (timed out) to *status. A timing harness enqueues it before its start
// event and sets the flag once it has submitted the timed launches, so the
// start event is stamped with all of them queued (nvbench's blocking
// kernel). Every lane polls the same word; lane 0 writes the status.
__global__ __launch_bounds__(64) void probe_hold_kernel(const uint32_t *flag, long long max_ticks,
                                                        uint32_t *status) {
    const long long t0 = wall_clock64();
    uint32_t st = 1;
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 0) {
        if (wall_clock64() - t0 > max_ticks) {
            st = 2;
            break;
        }
        __builtin_amdgcn_s_sleep(8);
    }
    if (threadIdx.x == 0) *status = st;
}

}  // namespace kxw4

using namespace kxw4;

extern "C" int kxw4_probe_mfma_i8(int shape, int iters, int32_t *sink, int sink_words, double *ops,
                                  void *stream) {
    if ((shape != 0 && shape != 1) || iters < 1 || !sink) return KXW4_EARG;
    // accumulators reach iters * K: keep them inside int32
    if ((long long)iters * 64 > 0x7FFFFFFFLL) return KXW4_EARG;
    const int groups = device_cus() * kProbeGroupsPerCu;
    if (sink_words < groups * kProbeWaves) return KXW4_ESHAPE;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (shape == 0)
        hipLaunchKernelGGL(probe_mfma_kernel<0>, dim3(groups), dim3(64 * kProbeWaves), 0, st, iters, sink);
    else
        hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(groups), dim3(64 * kProbeWaves), 0, st, iters, sink);
    if (hipGetLastError() != hipSuccess) return KXW4_EHIP;
    // 2 * 32 * 32 * 32 and 2 * 16 * 16 * 64 operations per MFMA
    if (ops) *ops = (double)groups * kProbeWaves * 4.0 * iters * (shape == 0 ? 65536.0 : 32768.0);
    return groups * kProbeWaves;
}

extern "C" int kxw4_probe_read(const void *buf, size_t bytes, int shape, uint32_t *sink, int sink_words,
                               void *stream) {
    if (!buf || !sink || bytes < 16 || (bytes & 15) || (reinterpret_cast<uintptr_t>(buf) & 15)) return KXW4_EARG;
    if (shape < 0 || shape >= kReadShapeCount) return KXW4_EARG;
    const ReadShape &rs = kReadShapes[shape];
    const int groups = device_cus() * rs.per_cu;
    const int waves = groups * (rs.threads / 64);
    if (sink_words < waves) return KXW4_ESHAPE;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const v4u *p = static_cast<const v4u *>(buf);
    const size_t n16 = bytes / 16;
    switch (rs.ring) {
    case 2: hipLaunchKernelGGL(probe_read_kernel<2>, dim3(groups), dim3(rs.threads), 0, st, p, n16, sink); break;
    case 4: hipLaunchKernelGGL(probe_read_kernel<4>, dim3(groups), dim3(rs.threads), 0, st, p, n16, sink); break;
    default: hipLaunchKernelGGL(probe_read_kernel<8>, dim3(groups), dim3(rs.threads), 0, st, p, n16, sink); break;
    }
    return hipGetLastError() == hipSuccess ? waves : KXW4_EHIP;
}

extern "C" int kxw4_probe_read_shapes(void) { return kReadShapeCount; }

extern "C" int kxw4_probe_issue(int mode, int waves_per_simd, int iters, float *sink, int sink_words,
                                double *blocks, void *stream) {
    if (mode < 0 || mode > 3 || waves_per_simd < 1 || waves_per_simd > 4 || iters < 1 || !sink) return KXW4_EARG;
    // split roles need a wave of each role on every SIMD
    if (mode == 3 && waves_per_simd % 2) return KXW4_EARG;
    const int groups = device_cus(), threads = 256 * waves_per_simd;
    if (sink_words < groups * 4 * waves_per_simd) return KXW4_ESHAPE;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const float w = 1.0001f;
    switch (mode) {
    case 0: hipLaunchKernelGGL(probe_issue_kernel<0>, dim3(groups), dim3(threads), 0, st, iters, w, sink); break;
    case 1: hipLaunchKernelGGL(probe_issue_kernel<1>, dim3(groups), dim3(threads), 0, st, iters, w, sink); break;
    case 2: hipLaunchKernelGGL(probe_issue_kernel<2>, dim3(groups), dim3(threads), 0, st, iters, w, sink); break;
    default: hipLaunchKernelGGL(probe_issue_kernel<3>, dim3(groups), dim3(threads), 0, st, iters, w, sink); break;
    }
    if (hipGetLastError() != hipSuccess) return KXW4_EHIP;
    // blocks per SIMD: 4 per iteration and wave (split roles: per role pair)
    if (blocks) *blocks = 4.0 * iters * (mode == 3 ? waves_per_simd / 2 : waves_per_simd);
    return groups * 4 * waves_per_simd;
}

extern "C" int kxw4_probe_hold(const uint32_t *flag, int max_us, uint32_t *status, void *stream) {
    using namespace kxw4;
    if (!flag || !status || max_us <= 0 || max_us > 1000000) return KXW4_EARG;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        return KXW4_EHIP;
    const long long ticks = (long long)max_us * khz / 1000;
    hipLaunchKernelGGL(probe_hold_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), flag, ticks,
                       status);
    return hipGetLastError() == hipSuccess ? 0 : KXW4_EHIP;
}
