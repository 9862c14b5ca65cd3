// kxw4_noalloc.hip — kxw4_gemv_x_noalloc: the reference's x_gemv_w4a8 /
// x_gemv_w4a8_add (kernels_dpas.cpp:1662-1680, quantize FP32 activations
// into library-allocated grow-only scratch, then the GEMV) for callers that
// cannot allocate: the quantized activations live in a fixed device array of
// this file instead.
//
// `scratch` is a file-scope __device__ array. In host code its name is only
// a stand-in for the device symbol, never a device address, so the host side
// asks the runtime for the array's address on each device once
// (hipGetSymbolAddress with that device current) and passes that pointer to
// the kernels. Each GPU holds its own copy of the array for the life of the
// process; every call on a GPU shares it, so calls that overlap on one GPU
// (two streams, two host threads) race. The quantizer writes every byte the
// GEMV reads, so nothing is cleared between calls.
#include "../../include/kxw4.h"
#include "kxw4_internal.hpp"

#include <mutex>

namespace kxw4 {

// Largest activation the array holds: T <= 16 tokens of K <= 32768, i.e.
// q[T][K] int8, then scale[T][K/32] f32 and sum[T][K/32] i32 (640 KiB).
constexpr int kNoAllocMaxT = 16;
constexpr int kNoAllocMaxK = 32768;
constexpr size_t kNoAllocQ = (size_t)kNoAllocMaxT * kNoAllocMaxK;
constexpr size_t kNoAllocS = (size_t)kNoAllocMaxT * (kNoAllocMaxK / 32) * 4;
constexpr size_t kNoAllocBytes = kNoAllocQ + 2 * kNoAllocS;

static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device; nullptr if the runtime cannot give it.
void *scratch_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_ptr[dev] = p;
    }
    return g_ptr[dev];
}

}  // namespace
}  // namespace kxw4

extern "C" int kxw4_gemv_x_noalloc(const kxw4_weight_t *w, const void *x, int x_dtype, int T, void *y,
                                   int y_dtype, const float *residual, void *stream) {
    using namespace kxw4;
    if (!w || !x || !y) return KXW4_EARG;
    if (x_dtype != KXW4_F32 && x_dtype != KXW4_BF16) return KXW4_ESHAPE;
    // the array's limits, checked before anything is enqueued
    if (T < 1 || T > kNoAllocMaxT || w->K <= 0 || w->K > kNoAllocMaxK || w->K % 128) return KXW4_ESHAPE;
    uint8_t *base = static_cast<uint8_t *>(scratch_ptr());
    if (!base) return KXW4_EHIP;
    const int K = w->K;
    int8_t *q = reinterpret_cast<int8_t *>(base);
    float *scale = reinterpret_cast<float *>(base + kNoAllocQ);
    int32_t *sum = reinterpret_cast<int32_t *>(base + kNoAllocQ + kNoAllocS);
    int rc = kxw4_quantize_act(x, x_dtype, T, K, 32, q, scale, sum, stream);
    if (rc) return rc;
    kxw4_act_t a;
    a.T = T;
    a.K = K;
    a.block = 32;
    a.q = q;
    a.scale = scale;
    a.sum = sum;
    return kxw4_gemv(w, &a, y, y_dtype, residual, 0, stream);
}
