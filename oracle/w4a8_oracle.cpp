// w4a8_oracle.cpp — CPU restatement of the reference W4A8 projection path.
//
// TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the reported
// CPU baseline. Nothing in the product links it. Built with
// -ffp-contract=off so every fused multiply-add below is an explicit fmaf()
// and every other operation rounds on its own, in the order written.
//
// Citations are reference paths (SRSWTI/knivesysl-xe) with line numbers.

#include "w4a8_oracle.h"

#include <cmath>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

inline uint32_t f2u(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }
inline float u2f(uint32_t u) { float x; std::memcpy(&x, &u, 4); return x; }

// sycl::clamp(x, lo, hi) for floats is fmin(fmax(x, lo), hi); a NaN input
// therefore lands on lo. Spelled out so the NaN rule is visible.
inline float clampf(float x, float lo, float hi) { return std::fmin(std::fmax(x, lo), hi); }

inline int sext4(uint32_t v) { int z = (int)(v & 0xFu); return z >= 8 ? z - 16 : z; }

// Round an unsigned magnitude right by `shift` bits, nearest-even.
inline uint32_t rne_shift(uint32_t m, int shift) {
    if (shift <= 0) return m << (-shift);
    if (shift >= 32) return 0;
    const uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    return (rem > half || (rem == half && (q & 1u))) ? q + 1 : q;
}

}  // namespace

extern "C" {

// IEEE binary32 -> binary16, round to nearest even (what sycl::half(float)
// does in fit_int4_asym, kernels_dpas.cpp:253). Overflow goes to infinity.
uint16_t orc_f32_to_f16(float x) {
    const uint32_t b = f2u(x);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const uint32_t exp = (b >> 23) & 0xFFu;
    const uint32_t man = b & 0x7FFFFFu;
    if (exp == 0xFFu) {
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));   // quiet NaN
    }
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        // Half subnormal: value = m * 2^-24 with m = (1.man) * 2^(exp-126+23).
        if (exp == 0) return (uint16_t)sign;   // float zero/subnormal -> 0
        const uint32_t full = man | 0x800000u;
        const int shift = 126 - (int)exp;      // >= 14
        return (uint16_t)(sign | rne_shift(full, shift));
    }
    const uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    const uint32_t r = (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ? q + 1 : q;
    return (uint16_t)(sign | r);               // a carry may produce infinity
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        return sign ? -std::ldexp((float)man, -24) : std::ldexp((float)man, -24);
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

// kernels_core.cpp:21-24 (the reference's f32 -> bf16, RNE by integer add).
uint16_t orc_f32_to_bf16(float x) {
    const uint32_t bits = f2u(x);
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

// kernels_core.cpp:27-29 / kernels_dpas.cpp:44-46.
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

// kernels_dpas.cpp:49-54: E2M3 = 1 sign, 2 exponent (bias 1), 3 mantissa.
float orc_e2m3(uint32_t c) {
    const float m = (float)(c & 7u);
    const uint32_t e = (c >> 3) & 3u;
    const float v = (e == 0) ? m * 0.125f : (1.0f + m * 0.125f) * (float)(1u << (e - 1));
    return (c & 0x20u) ? -v : v;
}

// kernels_dpas.cpp:58-69: (row, col) -> 6-bit code inside the 384-byte
// m16k32 fragment tile of the dense-E2M3 payload.
uint32_t orc_e2m3_code_at(const uint8_t *payload, int Kt, int row, int col) {
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

void orc_f32_to_f16_n(const float *x, uint16_t *h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_n(const uint16_t *h, float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_f16_to_f32(h[i]);
}
void orc_f32_to_bf16_n(const float *x, uint16_t *b, size_t n) {
    for (size_t i = 0; i < n; ++i) b[i] = orc_f32_to_bf16(x[i]);
}

// ---- activation quantizers ------------------------------------------------

// One symmetric int8 block: kernels_dpas.cpp:203-206 (quantize_act_s8) and
// 1172-1184 (quantize_act_chunk_subgroup<false>): s = absmax/127 (1 when the
// block max is not positive), q = clamp(rint(v/s), -127, 127). The absmax is
// an fmax reduction, which skips NaN (kernels_dpas.cpp:1175).
static void quantize_block(const float *v, int n, int8_t *q, float *scale) {
    float mx = -INFINITY;
    for (int j = 0; j < n; ++j) mx = std::fmax(mx, std::fabs(v[j]));
    const float s = (mx > 0.0f) ? (mx / 127.0f) : 1.0f;
    for (int j = 0; j < n; ++j)
        q[j] = (int8_t)(int32_t)clampf(std::rint(v[j] / s), -127.0f, 127.0f);
    *scale = s;
}

// Per-(token, K32) mode restates x_quantize_act_chunk (kernels_dpas.cpp:
// 1149-1207) and quantize_act_s8 (188-218); block 0 applies the same formula
// once over the whole token row (the per-token mode of the projection path).
// Sums are exact per K32 (the chunk quantizer's full-block sum, 1186-1192; the
// GEMV quantizer's two K16 halves add to the same integer, 636).
int orc_quantize_act(const float *x, int T, int K, int block, int8_t *q,
                     float *scale, int32_t *sum) {
    if (!x || !q || !scale || T <= 0 || K <= 0 || (K % 32) != 0) return -1;
    if (block != 0 && block != 32) return -1;
    for (int t = 0; t < T; ++t) {
        const float *xr = x + (size_t)t * K;
        int8_t *qr = q + (size_t)t * K;
        if (block == 32) {
            for (int b = 0; b < K / 32; ++b)
                quantize_block(xr + b * 32, 32, qr + b * 32, scale + (size_t)t * (K / 32) + b);
        } else {
            quantize_block(xr, K, qr, scale + t);
        }
        if (sum) {
            for (int b = 0; b < K / 32; ++b) {
                int32_t s = 0;
                for (int j = 0; j < 32; ++j) s += qr[b * 32 + j];
                sum[(size_t)t * (K / 32) + b] = s;
            }
        }
    }
    return 0;
}

// x_quantize_act_chunk_s4 (kernels_dpas.cpp:1492-1498 over
// quantize_act_chunk_subgroup<true>, 1149-1197): per (token, K64) block
// s = absmax/7 (1 when the block max is not positive), q = clamp(rint(v/s),
// -7, 7), and the exact code sum of the block. Codes are natural order
// [T][K]; scales and sums [T][K/64].
int orc_quantize_act_s4(const float *x, int T, int K, int8_t *q, float *scale, int32_t *sum) {
    if (!x || !q || !scale || !sum || T <= 0 || K <= 0 || (K % 64) != 0) return -1;
    for (int t = 0; t < T; ++t)
        for (int b = 0; b < K / 64; ++b) {
            const float *v = x + (size_t)t * K + (size_t)b * 64;
            int8_t *qb = q + (size_t)t * K + (size_t)b * 64;
            float mx = -INFINITY;
            for (int j = 0; j < 64; ++j) mx = std::fmax(mx, std::fabs(v[j]));
            const float s = (mx > 0.0f) ? (mx / 7.0f) : 1.0f;
            int32_t sm = 0;
            for (int j = 0; j < 64; ++j) {
                qb[j] = (int8_t)(int32_t)clampf(std::rint(v[j] / s), -7.0f, 7.0f);
                sm += qb[j];
            }
            scale[(size_t)t * (K / 64) + b] = s;
            sum[(size_t)t * (K / 64) + b] = sm;
        }
    return 0;
}

// w8_repack_kernel's fit (kernels_dpas.cpp:346-399): s = max(hi/127, neg/128)
// (1 when not positive), two least-squares refinements s = sum(w q)/sum(q q)
// with q = clamp(rint(w/s), -128, 127), then the FP16 (round to nearest even)
// of s; no zero point, no reserved nibble.
uint16_t orc_fit_int8(const float *wf, int n, int contract) {
    float hi = 0.0f, neg = 0.0f;
    for (int j = 0; j < n; ++j) {
        hi = std::fmax(hi, wf[j]);
        neg = std::fmax(neg, -wf[j]);
    }
    float s = std::fmax(hi / 127.0f, neg / 128.0f);
    if (!(s > 0.0f)) s = 1.0f;
    for (int iter = 0; iter < 2; ++iter) {
        float num = 0.0f, den = 0.0f;
        for (int j = 0; j < n; ++j) {
            const float q = clampf(std::rint(wf[j] / s), -128.0f, 127.0f);
            if (contract) {
                num = std::fma(wf[j], q, num);
                den = std::fma(q, q, den);
            } else {
                num = num + wf[j] * q;
                den = den + q * q;
            }
        }
        if (den > 0.0f) s = num / den;
    }
    return orc_f32_to_f16(s);
}

// kernels_dpas.cpp:197-199 (quantize_act_s8<true>): v = (g/(1+exp(-g)))*u.
void orc_silu_mul(const float *gate, const float *up, float *out, int n) {
    for (int i = 0; i < n; ++i) {
        const float g = gate[i];
        out[i] = (g / (1.0f + std::exp(-g))) * up[i];
    }
}

// kernels_dpas.cpp:866-929 (x_rmsnorm_quant): per-256 partial sums of x^2,
// summed in work-group order, rms_inv = rsqrt(sum/H + eps), and
// v = x * rms_inv * (1 + bf16(w)), multiplied left to right.
void orc_rmsnorm(const float *in, const uint16_t *w_bf16, int H, float eps, float *out) {
    float sum_sq = 0.0f;
    for (int b = 0; b < H; b += 256) {
        float part = 0.0f;
        for (int i = b; i < H && i < b + 256; ++i) part = part + in[i] * in[i];
        sum_sq = sum_sq + part;
    }
    const float rms_inv = 1.0f / std::sqrt(sum_sq / (float)H + eps);
    for (int i = 0; i < H; ++i)
        out[i] = in[i] * rms_inv * (1.0f + orc_bf16_to_f32(w_bf16[i]));
}

// ---- weight side ----------------------------------------------------------

// kernels_dpas.cpp:229-256 (fit_int4_asym). contract=1 evaluates the two
// least-squares accumulations as fused multiply-adds.
uint16_t orc_fit_int4_asym(const float *wf, int n, int reserve_nibble, int contract,
                           int *out_z) {
    float lo = 0.0f, hi = 0.0f;
    for (int j = 0; j < n; ++j) {
        lo = std::fmin(lo, wf[j]);
        hi = std::fmax(hi, wf[j]);
    }
    float s = (hi - lo) / 15.0f;
    if (!(s > 0.0f)) s = 1.0f;
    for (int iter = 0; iter < 3; ++iter) {
        const int zi = (int)clampf(std::rint(-lo / s) - 8.0f, -8.0f, 7.0f);
        float num = 0.0f, den = 0.0f;
        for (int j = 0; j < n; ++j) {
            const float q = clampf(std::rint(wf[j] / s + (float)zi), -8.0f, 7.0f);
            const float c = q - (float)zi;
            if (contract) {
                num = std::fma(wf[j], c, num);
                den = std::fma(c, c, den);
            } else {
                num = num + wf[j] * c;
                den = den + c * c;
            }
        }
        if (den > 0.0f) s = num / den;
    }
    *out_z = (int)clampf(std::rint(-lo / s) - 8.0f, -8.0f, 7.0f);
    uint16_t sh = orc_f32_to_f16(s);
    if (reserve_nibble) sh = (uint16_t)((sh + 8u) & 0xFFF0u);
    return sh;
}

// kernels_dpas.cpp:266-344 (w4_repack_kernel) for mode 0 (one scale per K32)
// and mode 2 (one per K64): decode E2M3 x block scale, fit, then quantize
// every weight against the STORED scale: q = clamp(rint(w/s + z), -8, 7).
// Output is natural order: codes[M][K], scales[M][K/group] (FP16|zp nibble).
int orc_repack_e2m3(const uint8_t *payload, const float *bs, int scale_cols, int M,
                    int K, int mode, int contract, int8_t *codes, uint16_t *scales) {
    if (!payload || !bs || !codes || !scales) return -1;
    if (M % 16 || K % 128) return -2;
    if (mode != 0 && mode != 1 && mode != 2) return -4;
    const int Kt = K / 32;
    const int group = mode == 2 ? 64 : mode == 1 ? 16 : 32;   // mode 1: K16 halves (kernels_dpas.cpp:287-296)
    const int G = K / group;
    for (int row = 0; row < M; ++row) {
        const int mt = row >> 4;
        for (int g = 0; g < G; ++g) {
            float wf[64];
            const int k0 = g * group;
            for (int j = 0; j < group; ++j) {
                const int kt = (k0 + j) >> 5;
                const int sc = (scale_cols == Kt) ? kt : (kt >> 2);
                const float b = bs[(size_t)(mt >> 3) * scale_cols + sc];
                wf[j] = orc_e2m3(orc_e2m3_code_at(payload, Kt, row, k0 + j)) * b;
            }
            int z = 0;
            const uint16_t sh = orc_fit_int4_asym(wf, group, 1, contract, &z);
            scales[(size_t)row * G + g] = (uint16_t)(sh | (z & 0xF));
            const float gs = orc_f16_to_f32(sh);
            for (int j = 0; j < group; ++j) {
                const float r = std::rint(wf[j] / gs + (float)z);
                codes[(size_t)row * K + k0 + j] = (int8_t)(int)clampf(r, -8.0f, 7.0f);
            }
        }
    }
    return 0;
}

// Reference DPAS weight layout (kernels_dpas.cpp:327-342 and tq_common.hpp:
// 62-72): codes [M/16][Kt][256 B]; row n of a row-group owns bytes
// [16n, 16n+16) of a tile; dword i holds k = 8i..8i+7; byte b holds k = 8i+2b
// (low nibble) and 8i+2b+1 (high). Scales [M/16][K/group][16], row fastest.
// x_w8_repack_weight (kernels_dpas.cpp:346-399, 558-575): dense-E2M3 payload ->
// int8 codes [M][K] and plain FP16 scales [M][K/32], per (row, K32).
int orc_repack_e2m3_s8(const uint8_t *payload, const float *bs, int scale_cols, int M, int K,
                       int contract, int8_t *codes, uint16_t *scales) {
    if (!payload || !bs || !codes || !scales) return -1;
    if (M % 16 || K % 128) return -2;
    const int Kt = K / 32;
    for (int row = 0; row < M; ++row) {
        const int mt = row >> 4;
        for (int kt = 0; kt < Kt; ++kt) {
            const int sc = (scale_cols == Kt) ? kt : (kt >> 2);
            const float b = bs[(size_t)(mt >> 3) * scale_cols + sc];
            float wf[32];
            for (int j = 0; j < 32; ++j)
                wf[j] = orc_e2m3(orc_e2m3_code_at(payload, Kt, row, kt * 32 + j)) * b;
            const uint16_t sh = orc_fit_int8(wf, 32, contract);
            scales[(size_t)row * Kt + kt] = sh;
            const float st = orc_f16_to_f32(sh);
            for (int j = 0; j < 32; ++j)
                codes[(size_t)row * K + kt * 32 + j] =
                    (int8_t)(int)clampf(std::rint(wf[j] / st), -128.0f, 127.0f);
        }
    }
    return 0;
}

int orc_pack_ref_layout(const int8_t *codes, const uint16_t *scales, int M, int K,
                        int group, uint8_t *ref_codes, uint16_t *ref_scales) {
    if (M % 16 || K % 32 || (group != 32 && group != 64)) return -2;
    const int Kt = K / 32, G = K / group;
    std::memset(ref_codes, 0, (size_t)M * K / 2);
    for (int row = 0; row < M; ++row) {
        const int rg = row >> 4, n = row & 15;
        for (int k = 0; k < K; ++k) {
            const int kt = k >> 5, j = k & 31;
            const size_t byte = ((size_t)rg * Kt + kt) * 256u + (size_t)(n * 4 + (j >> 3)) * 4u +
                                (size_t)((j & 7) >> 1);
            const uint8_t nib = (uint8_t)(codes[(size_t)row * K + k] & 0xF);
            ref_codes[byte] |= (j & 1) ? (uint8_t)(nib << 4) : nib;
        }
        for (int g = 0; g < G; ++g)
            ref_scales[((size_t)rg * G + g) * 16u + n] = scales[(size_t)row * G + g];
    }
    return 0;
}

int orc_unpack_ref_layout(const uint8_t *ref_codes, const uint16_t *ref_scales, int M,
                          int K, int group, int8_t *codes, uint16_t *scales) {
    if (M % 16 || K % 32 || (group != 32 && group != 64)) return -2;
    const int Kt = K / 32, G = K / group;
    for (int row = 0; row < M; ++row) {
        const int rg = row >> 4, n = row & 15;
        for (int k = 0; k < K; ++k) {
            const int kt = k >> 5, j = k & 31;
            const size_t byte = ((size_t)rg * Kt + kt) * 256u + (size_t)(n * 4 + (j >> 3)) * 4u +
                                (size_t)((j & 7) >> 1);
            const uint32_t v = (j & 1) ? (ref_codes[byte] >> 4) : (ref_codes[byte] & 0xFu);
            codes[(size_t)row * K + k] = (int8_t)sext4(v);
        }
        for (int g = 0; g < G; ++g)
            scales[(size_t)row * G + g] = ref_scales[((size_t)rg * G + g) * 16u + n];
    }
    return 0;
}

// ---- split plans ----------------------------------------------------------

// kernels_dpas.cpp:170-173 (choose_gemv_splits).
int orc_gemv_splits(int groups) {
    if (groups <= 4) return 16;
    return groups >= 4096 ? 1 : 8;
}

// kernels_dpas.cpp:1226-1250 (choose_gemm_splits); `forced` stands for the
// TQ_XPU_GEMM_SPLITS override (0 = heuristic; 1/2/4/8/16 accepted).
int orc_gemm_splits(int rgroups, int tgroups, int ktiles, int forced) {
    if (forced != 1 && forced != 2 && forced != 4 && forced != 8 && forced != 16) forced = 0;
    const long tasks = (long)rgroups * tgroups;
    if (tasks <= 0) return 1;
    if (forced) {
        int s = forced;
        while (s > 1 && s > ktiles) s >>= 1;
        return s;
    }
    const long want = 128L * 16;
    if (tasks >= want) return 1;
    for (int s = 2; s <= 16; s <<= 1) {
        if (s > ktiles) break;
        if (tasks * s >= want) return s;
    }
    int s = 16;
    while (s > 1 && s > ktiles) s >>= 1;
    return s;
}

// kernels_dpas.cpp:1343-1367: one split count per packed segment, from that
// segment's own 8-row group count. Segments of any positive length are
// accepted here (row counts are rounded up to 8-row groups); the reference
// additionally requires multiples of 8.
int orc_segment_splits(const int *offsets, int segments, int T, int M, int K, int forced,
                       int *split_per_token) {
    if (T <= 0 || M % 16 || K % 32) return -2;
    const int rgroups = M / 16, Kt = K / 32;
    if (!offsets) {
        if (segments != 0) return -2;
        const int s = orc_gemm_splits(rgroups, (T + 7) / 8, Kt, forced);
        for (int t = 0; t < T; ++t) split_per_token[t] = s;
        return 0;
    }
    if (segments < 1 || segments > 8 || offsets[0] != 0 || offsets[segments] != T) return -2;
    for (int i = 0; i < segments; ++i)
        if (offsets[i + 1] <= offsets[i]) return -2;
    for (int i = 0; i < segments; ++i) {
        const int len = offsets[i + 1] - offsets[i];
        const int s = orc_gemm_splits(rgroups, (len + 7) / 8, Kt, forced);
        for (int t = offsets[i]; t < offsets[i + 1]; ++t) split_per_token[t] = s;
    }
    return 0;
}

// ---- projection -----------------------------------------------------------

static int unit_of(const orc_weight_t *w, const orc_act_t *a) {
    if (w->group == 16) return 16;   // the K16 tier: one partial per K16 half
    return a->block == 32 ? 32 : a->block == 64 ? 64 : w->group;
}

// K extent of one activation scale / code-sum block
static int act_block_of(const orc_act_t *a) { return a->block == 64 ? 64 : 32; }

static int check_args(const orc_weight_t *w, const orc_act_t *a) {
    if (!w || !a || !w->codes || !w->scales || !a->q || !a->scale) return -1;
    if (w->M <= 0 || w->M % 16 || w->K <= 0 || w->K % 128 || w->K != a->K) return -2;
    if (w->group != 16 && w->group != 32 && w->group != 64 && w->group != 128) return -2;
    // the K16 tier (kernels_dpas.cpp:677-760): FP16|zp scales per K16 and
    // block-32 activations
    if (w->group == 16 && (w->scale_enc != ORC_SCALE_FP16_ZP4 || a->block != 32)) return -1;
    if (a->block != 0 && a->block != 32 && a->block != 64) return -2;
    // block 64 = s4 activations of the W4A4 GEMM (kernels_dpas.cpp:1503-1504):
    // K64-tier weights with FP16|zp scales only
    if (a->block == 64 && (w->group != 64 || w->scale_enc != ORC_SCALE_FP16_ZP4)) return -1;
    if (w->scale_enc == ORC_SCALE_FP16_ZP4 && !a->sum) return -1;
    // the W8A8 tier (kernels_dpas.cpp:771-844, 1578-1629): int8 codes, plain
    // FP16 scales per K32, block-32 activations only
    if (w->scale_enc == ORC_SCALE_S8 && (w->group != 32 || a->block != 32)) return -1;
    if (w->scale_enc != ORC_SCALE_FP16 && w->scale_enc != ORC_SCALE_FP16_ZP4 &&
        w->scale_enc != ORC_SCALE_S8)
        return -2;
    return 0;
}

// The exact integer of one unit: sum (q_w - z) * q_a over the unit
// (kernels_dpas.cpp:636, 1320, 1467: d - z * asum).
static inline int32_t unit_partial(const orc_weight_t *w, const orc_act_t *a, int t, int n,
                                   int u, int unit, int *zero_point) {
    const int K = w->K;
    const int8_t *wr = w->codes + (size_t)n * K + (size_t)u * unit;
    const int8_t *ar = a->q + (size_t)t * K + (size_t)u * unit;
    int32_t d = 0;
    for (int j = 0; j < unit; ++j) d += (int32_t)wr[j] * (int32_t)ar[j];
    int z = 0;
    if (w->scale_enc == ORC_SCALE_FP16_ZP4) {
        const int g = (u * unit) / w->group;
        z = sext4(w->scales[(size_t)n * (K / w->group) + g]);
        const int ab = act_block_of(a);
        int32_t s = 0;
        if (unit < ab) {
            // a K16 half: its own code sum (the reference's per-K16 d_sum,
            // kernels_dpas.cpp:208-214)
            for (int j = 0; j < unit; ++j) s += ar[j];
        } else {
            for (int b = (u * unit) / ab; b < ((u + 1) * unit) / ab; ++b)
                s += a->sum[(size_t)t * (K / ab) + b];
        }
        d -= z * s;
    }
    *zero_point = z;
    return d;
}

int orc_partials(const orc_weight_t *w, const orc_act_t *a, int32_t *P) {
    const int rc = check_args(w, a);
    if (rc) return rc;
    const int unit = unit_of(w, a), Nu = w->K / unit, M = w->M, T = a->T;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < M; ++n)
        for (int t = 0; t < T; ++t)
            for (int u = 0; u < Nu; ++u) {
                int z;
                P[((size_t)t * M + n) * Nu + u] = unit_partial(w, a, t, n, u, unit, &z);
            }
    return 0;
}

// Float epilogue per unit and per kernel variant:
//   GEMV and fan-out (kernels_dpas.cpp:636, 1061, 1072):
//       term = ((float)P * ws) * as, accumulated into acc  (contract: fma of
//       the second product into the accumulator)
//   GEMM (kernels_dpas.cpp:1320, 1467): acc += (float)P * (ws * as)
//   per-token activation scale (config mode): acc += (float)P * ws, with the
//       token scale applied once after the split reduction.
// Chains: GEMV alternates two accumulators over the split's units
// (kernels_dpas.cpp:644-652); fan-out and GEMM run one serial accumulator
// (1030-1074, 1313-1321, 1450-1468). Splits cover units [Nu*s/S, Nu*(s+1)/S);
// S == 1 stores the chain directly, otherwise 0 + partial_0 + ... in split
// order (663-672, 1092-1101, 1477-1486).
// K16 tier (x_gemv_w4a8_core_k16, 683-760): GEMV only, one serial
// accumulator, splits over K32 tiles [Kt*s/S, Kt*(s+1)/S) each covering both
// K16 halves, as per K32.
int orc_project(const orc_weight_t *w, const orc_act_t *a, int variant,
                const int *split_per_token, int contract, const float *residual,
                int out_bf16, void *y, int row_begin, int row_end) {
    const int rc = check_args(w, a);
    if (rc) return rc;
    if (!split_per_token || !y) return -1;
    if (variant != ORC_VAR_GEMV && variant != ORC_VAR_FANOUT && variant != ORC_VAR_GEMM)
        return -2;
    if (variant == ORC_VAR_FANOUT && residual) return -2;
    // W4A4: the GEMM variant, one chain per output (kernels_dpas.cpp:1540-1568)
    if (a->block == 64 && variant != ORC_VAR_GEMM) return -2;
    // K16: GEMV only (x_gemm_w4a8 rejects it, kernels_dpas.cpp:1337)
    if (w->group == 16 && variant != ORC_VAR_GEMV) return -1;
    const bool k16 = w->group == 16;
    const int M = w->M, K = w->K, T = a->T;
    if (row_begin < 0 || row_end > M || row_begin > row_end) return -2;
    const int unit = unit_of(w, a), Nu = K / unit, G = K / w->group;
    const bool per_token = a->block == 0;
    for (int t = 0; t < T; ++t)
        if (split_per_token[t] < 1) return -2;

#pragma omp parallel
    {
        std::vector<int32_t> P(Nu);
#pragma omp for schedule(static)
        for (int n = row_begin; n < row_end; ++n) {
            for (int t = 0; t < T; ++t) {
                for (int u = 0; u < Nu; ++u) {
                    int z;
                    P[u] = unit_partial(w, a, t, n, u, unit, &z);
                }
                const int S = split_per_token[t];
                float sum = 0.0f;
                for (int s = 0; s < S; ++s) {
                    const int step = k16 ? 2 : 1;   // K16: splits on K32 tiles
                    const int u0 = step * (int)((long long)(Nu / step) * s / S);
                    const int u1 = step * (int)((long long)(Nu / step) * (s + 1) / S);
                    float acc0 = 0.0f, acc1 = 0.0f;
                    for (int u = u0; u < u1; ++u) {
                        const uint16_t raw = w->scales[(size_t)n * G + (u * unit) / w->group];
                        const float ws = orc_f16_to_f32(
                            w->scale_enc == ORC_SCALE_FP16_ZP4 ? (uint16_t)(raw & 0xFFF0u) : raw);
                        const float p = (float)P[u];
                        float &acc = (variant == ORC_VAR_GEMV && !k16 && ((u - u0) & 1)) ? acc1 : acc0;
                        if (per_token) {
                            acc = contract ? std::fma(p, ws, acc) : acc + p * ws;
                        } else {
                            const float as = a->scale[(size_t)t * (K / act_block_of(a)) +
                                                      (u * unit) / act_block_of(a)];
                            if (variant == ORC_VAR_GEMM) {
                                const float wa = ws * as;
                                acc = contract ? std::fma(p, wa, acc) : acc + p * wa;
                            } else {
                                const float x = p * ws;
                                acc = contract ? std::fma(x, as, acc) : acc + x * as;
                            }
                        }
                    }
                    const float partial = (variant == ORC_VAR_GEMV) ? acc0 + acc1 : acc0;
                    if (S == 1) sum = partial;
                    else sum = sum + partial;
                }
                const float v = per_token ? sum * a->scale[t] : sum;
                const float r = residual ? residual[(size_t)t * M + n] : 0.0f;
                float out;
                if (variant == ORC_VAR_GEMV && S > 1) out = v + r;   // 670-671
                else out = residual ? v + r : v;
                if (out_bf16) ((uint16_t *)y)[(size_t)t * M + n] = orc_f32_to_bf16(out);
                else ((float *)y)[(size_t)t * M + n] = out;
            }
        }
    }
    return 0;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

}  // extern "C"
