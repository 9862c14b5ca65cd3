// kxw4_device.hpp — device helpers shared by the gfx950 kernels.
//
// Operand contract of the int8 MFMAs used here (checked on the MI355X with a
// one-hot/random probe): for v_mfma_i32_16x16x64_i8 and _16x16x32_i8 the A
// and B operands have the same register layout — lane l supplies row
// (A) / column (B) l%16 and the K slots of lane group l/16 — and the 16x16
// int32 result puts D[4*(l/16) + r][l%16] in register r of lane l.
//
// A operand = activations (rows = tokens), B operand = weights (columns =
// output rows), so a lane holds one output row n = l%16 and four tokens.
//
// Weight nibbles are unpacked to int8 as 16*q: a nibble in the high half of a
// byte read as int8 is 16*q exactly, so `w & 0xF0F0F0F0` and
// `(w << 4) & 0xF0F0F0F0` yield four int8 operands each with no sign fix-up.
// Every int32 MFMA result is therefore 16x the unit partial; the factor is
// exact (|16 P| < 2^22 for every unit) and is divided back out exactly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kxw4 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kTileK = 128;        // K extent of one packed weight tile
constexpr int kTileBytes = 1024;   // 16 rows x 128 K x 4 bits

__device__ __forceinline__ uint32_t nib_lo16(uint32_t w) { return (w << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t nib_hi16(uint32_t w) { return w & 0xF0F0F0F0u; }

// B operand of the K64 MFMA over chunk c (0/1) of a 128-K tile held as four
// packed dwords: slots 0..7 = dword 2c, slots 8..15 = dword 2c+1.
__device__ __forceinline__ v4i unpack_k64(uint32_t d0, uint32_t d1) {
    v4i b;
    b.x = (int)nib_lo16(d0);
    b.y = (int)nib_hi16(d0);
    b.z = (int)nib_lo16(d1);
    b.w = (int)nib_hi16(d1);
    return b;
}

// B operand of the K32 MFMA for one packed dword (one K32 unit).
__device__ __forceinline__ long unpack_k32(uint32_t d) {
    const uint64_t lo = nib_lo16(d), hi = nib_hi16(d);
    return (long)(lo | (hi << 32));
}

// v_mfma_i32_32x32x32_i8: lane l supplies row (A) / column (B) l%32 and the
// 16 K slots of K group l/32 (the same slots for both operands); result
// register r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l%32] (checked on the
// MI355X against a host product of random operands).
__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i mfma_k64(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i mfma_k32(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Reference f32 -> bf16 (integer round-to-nearest-even, kernels_core.cpp:21-24).
__device__ __forceinline__ uint16_t float_to_bf16(float x) {
    const uint32_t b = __float_as_uint(x);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16_to_float(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ int sext4(uint32_t v) {
    const int z = (int)(v & 0xFu);
    return z >= 8 ? z - 16 : z;
}

// DPP row_ror:8 -- lane i of each 16-lane row takes lane (i+8)%16.
__device__ __forceinline__ v4i rotate8(v4i v) {
    v4i r;
    r.x = __builtin_amdgcn_mov_dpp(v.x, 0x128, 0xF, 0xF, false);
    r.y = __builtin_amdgcn_mov_dpp(v.y, 0x128, 0xF, 0xF, false);
    r.z = __builtin_amdgcn_mov_dpp(v.z, 0x128, 0xF, 0xF, false);
    r.w = __builtin_amdgcn_mov_dpp(v.w, 0x128, 0xF, 0xF, false);
    return r;
}

// s_waitcnt immediate that waits until at most n vector-memory operations of
// this wave are outstanding and leaves expcnt and lgkmcnt alone. The gfx9
// encoding splits vmcnt over bits [3:0] and [15:14] (six bits, n <= 63);
// expcnt is bits [6:4] (7 = no wait), lgkmcnt bits [11:8] (15 = no wait).
constexpr int waitcnt_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
static_assert(waitcnt_vmcnt(0) == 0x0F70 && waitcnt_vmcnt(15) == 0x0F7F &&
              waitcnt_vmcnt(16) == 0x4F70 && waitcnt_vmcnt(63) == 0xCF7F, "vmcnt encoding");
#define KXW4_WAIT_VMCNT(n)                                                     \
    do {                                                                       \
        static_assert((n) >= 0 && (n) <= 63, "vmcnt holds six bits");          \
        __builtin_amdgcn_s_waitcnt(::kxw4::waitcnt_vmcnt(n));                  \
    } while (0)

// Barrier for LDS traffic only: waits for this wave's LDS accesses, not for
// its outstanding global loads, so a prefetch ring stays in flight.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Barrier after direct global->LDS loads: the caller has already waited for
// them with an explicit vmcnt (they were issued before the loads still in
// flight); this waits for the wave's own LDS accesses and synchronises. The
// empty asm statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_sync_after_dma() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0); vmcnt, expcnt untouched
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Byte offset of element k inside its 64-element activation chunk.
__host__ __device__ __forceinline__ int act_slot(int k) {
    return 16 * ((k >> 3) & 3) + 8 * ((k >> 5) & 1) + (k & 7);
}

// sycl::clamp semantics: fmin(fmax(x, lo), hi), so NaN lands on lo.
__device__ __forceinline__ float clampf(float x, float lo, float hi) {
    return fminf(fmaxf(x, lo), hi);
}

}  // namespace kxw4
