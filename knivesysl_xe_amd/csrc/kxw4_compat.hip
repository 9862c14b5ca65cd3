// kxw4_compat.hip — the reference's C++ projection functions
// (xpu/src/tq_common.hpp:385-461) as shims over the C ABI. Host code only.
#include <hip/hip_runtime.h>

#include "../../include/kxw4_compat.hpp"

namespace {

hipStream_t g_stream = nullptr;

void dfree(void *p) {
    if (p) (void)hipFree(p);
}

// Prepared single-token activation: the counterpart of the reference's
// library-global grow-only scratch (kernels_dpas.cpp:133-149).
struct Prepared {
    int8_t *q = nullptr;
    float *scale = nullptr;
    int32_t *sum = nullptr;
    int cap = 0;      // capacity in K
    int K = 0;        // K of the last prepare (0 = none)
} g_act;

bool ensure_act(int K) {
    if (K <= g_act.cap) return true;
    dfree(g_act.q);
    dfree(g_act.scale);
    dfree(g_act.sum);
    g_act = Prepared{};
    if (hipMalloc(&g_act.q, (size_t)K) != hipSuccess ||
        hipMalloc(&g_act.scale, (size_t)(K / 32) * sizeof(float)) != hipSuccess ||
        hipMalloc(&g_act.sum, (size_t)(K / 32) * sizeof(int32_t)) != hipSuccess) {
        dfree(g_act.q);
        dfree(g_act.scale);
        dfree(g_act.sum);
        g_act = Prepared{};
        return false;
    }
    g_act.cap = K;
    return true;
}

kxw4_weight_t w4_of(const tq_qmma_weight_t *w) {
    kxw4_weight_t d;
    d.M = w->M;
    d.K = w->K;
    d.group = w->s4_k64 ? 64 : w->s4_k16 ? 16 : 32;
    d.scale_enc = KXW4_SCALE_FP16_ZP4;
    d.codes = w->d_s4;
    d.scales = w->d_s4_scale;
    return d;
}

kxw4_act_t prepared_act() {
    kxw4_act_t a;
    a.T = 1;
    a.K = g_act.K;
    a.block = 32;
    a.q = g_act.q;
    a.scale = g_act.scale;
    a.sum = g_act.sum;
    return a;
}

bool w4_ready(const tq_qmma_weight_t *w) {
    return w && w->s4_ready && !w->s4_k16 && w->d_s4 && w->d_s4_scale;
}

bool w8_ready(const tq_qmma_weight_t *w) { return w && w->s8_ready && w->d_s8 && w->d_s8_scale; }

kxw4_weight_t w8_of(const tq_qmma_weight_t *w) {
    kxw4_weight_t d;
    d.M = w->M;
    d.K = w->K;
    d.group = 32;
    d.scale_enc = KXW4_SCALE_W8;
    d.codes = w->d_s8;
    d.scales = w->d_s8_scale;
    return d;
}

}  // namespace

extern "C" void kxw4_compat_set_stream(void *stream) { g_stream = static_cast<hipStream_t>(stream); }

int x_w4_repack_weight_mode(tq_qmma_weight_t *w, int mode) {
    if (!w || !w->d_A || !w->d_block_scale_inv || !w->block_scaled || !w->e2m3) return -1;
    if (w->M % 16 || w->K % 128) return -2;
    if (mode == 2 && (w->Kt & 1)) return -3;
    if (mode != 0 && mode != 1 && mode != 2) return KXW4_ESHAPE;
    const int group = mode == 2 ? 64 : mode == 1 ? 16 : 32;
    uint8_t *codes = nullptr;
    uint16_t *scales = nullptr;
    if (hipMalloc(&codes, kxw4_code_bytes(w->M, w->K)) != hipSuccess) return KXW4_EHIP;
    if (hipMalloc(&scales, kxw4_scale_count(w->M, w->K, group) * sizeof(uint16_t)) != hipSuccess) {
        dfree(codes);
        return KXW4_EHIP;
    }
    int rc = kxw4_repack_e2m3(w->d_A, w->d_block_scale_inv, w->scale_cols, w->M, w->K, mode, codes,
                              scales, g_stream);
    if (rc == 0 && hipStreamSynchronize(g_stream) != hipSuccess) rc = KXW4_EHIP;
    if (rc != 0) {
        dfree(codes);
        dfree(scales);
        return rc;
    }
    dfree(w->d_A);
    dfree(w->d_block_scale_inv);
    w->d_A = nullptr;
    w->d_block_scale_inv = nullptr;
    w->d_s4 = codes;
    w->d_s4_scale = scales;
    w->s4_k16 = mode == 1 ? 1 : 0;
    w->s4_k64 = mode == 2 ? 1 : 0;
    w->s4_ready = 1;
    return 0;
}

int x_w4_repack_weight(tq_qmma_weight_t *w) { return x_w4_repack_weight_mode(w, 0); }

int x_w8_repack_weight(tq_qmma_weight_t *w) {
    if (!w || !w->d_A || !w->d_block_scale_inv || !w->block_scaled || !w->e2m3) return -1;
    if (w->M % 16 || w->K % 128) return -2;
    uint8_t *codes = nullptr;
    uint16_t *scales = nullptr;
    if (hipMalloc(&codes, (size_t)w->M * w->K) != hipSuccess) return KXW4_EHIP;
    if (hipMalloc(&scales, kxw4_scale_count(w->M, w->K, 32) * sizeof(uint16_t)) != hipSuccess) {
        dfree(codes);
        return KXW4_EHIP;
    }
    int rc = kxw4_repack_e2m3_s8(w->d_A, w->d_block_scale_inv, w->scale_cols, w->M, w->K, codes, scales,
                                 g_stream);
    if (rc == 0 && hipStreamSynchronize(g_stream) != hipSuccess) rc = KXW4_EHIP;
    if (rc != 0) {
        dfree(codes);
        dfree(scales);
        return rc;
    }
    dfree(w->d_A);
    dfree(w->d_block_scale_inv);
    w->d_A = nullptr;
    w->d_block_scale_inv = nullptr;
    w->d_s8 = codes;
    w->d_s8_scale = scales;
    w->s8_ready = 1;
    return 0;
}

void x_quantize_act_s8(const float *d_x, int K, int8_t *d_q, float *d_scale, int32_t *d_sum) {
    kxw4_quantize_act(d_x, KXW4_F32, 1, K, 32, d_q, d_scale, d_sum, g_stream);
}

void x_prepare_gemv_act_s8(const float *d_x, int K) {
    if (!d_x || K <= 0 || K % 128 || !ensure_act(K)) return;
    if (kxw4_quantize_act(d_x, KXW4_F32, 1, K, 32, g_act.q, g_act.scale, g_act.sum, g_stream) == 0)
        g_act.K = K;
}

void x_silu_mul_quant(float *d_out, const float *d_gate, const float *d_up, int K) {
    if (!d_gate || !d_up || K <= 0 || K % 128 || !ensure_act(K)) return;
    if (kxw4_silu_mul_quant(d_out, d_gate, d_up, 1, K, 32, g_act.q, g_act.scale, g_act.sum,
                            g_stream) == 0)
        g_act.K = K;
}

void x_rmsnorm_quant(float *d_out, const float *d_in, const uint16_t *d_w, int H, float eps) {
    if (!d_in || !d_w || H <= 0 || H % 128 || !ensure_act(H)) return;
    if (kxw4_rmsnorm_quant(d_out, d_in, d_w, 1, H, eps, 32, g_act.q, g_act.scale, g_act.sum,
                           g_stream) == 0)
        g_act.K = H;
}

void x_rmsnorm_chunk(float *d_out, const float *d_in, const uint16_t *d_w, int H, int T, float eps) {
    kxw4_rmsnorm(d_out, d_in, d_w, T, H, eps, g_stream);
}

int x_gemv_w4a8_prepared(const tq_qmma_weight_t *w, float *d_y, const float *d_residual) {
    // every W4 tier, K16 included (kernels_dpas.cpp:1647-1653)
    if (!w || !w->s4_ready || !w->d_s4 || !w->d_s4_scale || !d_y) return -1;
    // -2 when no activation of this K is prepared. The reference checks only
    // the scratch capacity (kernels_dpas.cpp:1636), so after a prepare of a
    // different K within that capacity it returns 0 and reads the stale
    // codes; this shim refuses that case with the same -2.
    if (g_act.K != w->K) return -2;
    const kxw4_weight_t d = w4_of(w);
    const kxw4_act_t a = prepared_act();
    return kxw4_gemv(&d, &a, d_y, KXW4_F32, d_residual, 0, g_stream);
}

int x_gemv_w4a8(const tq_qmma_weight_t *w, const float *d_x, float *d_y) {
    if (!w || !d_x) return -1;
    x_prepare_gemv_act_s8(d_x, w->K);
    return x_gemv_w4a8_prepared(w, d_y, nullptr);
}

int x_gemv_w4a8_add(const tq_qmma_weight_t *w, const float *d_x, const float *d_residual, float *d_y) {
    if (!w || !d_x || !d_residual) return -1;
    x_prepare_gemv_act_s8(d_x, w->K);
    return x_gemv_w4a8_prepared(w, d_y, d_residual);
}

int x_gemv_w4a8_fanout(const tq_qmma_weight_t *const *ws, float *const *ys, int count) {
    if (!ws || !ys || count <= 0 || count > 4) return -1;
    kxw4_weight_t d[4];
    const kxw4_weight_t *dp[4];
    void *yp[4];
    for (int i = 0; i < count; ++i) {
        const tq_qmma_weight_t *w = ws[i];
        if (!w4_ready(w) || !ys[i] || w->K != ws[0]->K || w->M % 16 || w->s4_k64 != ws[0]->s4_k64)
            return -2;
        d[i] = w4_of(w);
        dp[i] = &d[i];
        yp[i] = ys[i];
    }
    if (g_act.K != ws[0]->K) return -3;
    const kxw4_act_t a = prepared_act();
    return kxw4_gemv_fanout(dp, yp, count, &a, KXW4_F32, g_stream);
}

void x_quantize_act_chunk(const float *d_x, int K, int T, int8_t *d_aq, float *d_as, int32_t *d_asum) {
    kxw4_quantize_act(d_x, KXW4_F32, T, K, 32, d_aq, d_as, d_asum, g_stream);
}

// x_gemm_w4a8's checks (kernels_dpas.cpp:1337-1367): -1 for a weight that
// is not a K32/K64 W4 tier, -2 for missing operands, T not a positive
// multiple of 8, and offsets that do not partition [0, T) in multiples of 8
// (at most 8 segments). Ragged segments stay on the C ABI (kxw4_gemm).
int x_gemm_w4a8(const tq_qmma_weight_t *w, const int8_t *d_aq, const float *d_as,
                const int32_t *d_asum, float *d_y, int T, const int *offsets, int segments) {
    if (!w4_ready(w)) return -1;
    if (!d_aq || !d_as || !d_asum || !d_y || T <= 0 || (T % 8) != 0) return -2;
    if (offsets) {
        if (segments < 1 || segments > 8 || offsets[0] != 0 || offsets[segments] != T) return -2;
        for (int i = 0; i < segments; ++i)
            if (offsets[i] < 0 || offsets[i + 1] <= offsets[i] || offsets[i + 1] > T || offsets[i] % 8 ||
                offsets[i + 1] % 8)
                return -2;
    } else if (segments != 0) {
        return -2;
    }
    const kxw4_weight_t d = w4_of(w);
    kxw4_act_t a;
    a.T = T;
    a.K = w->K;
    a.block = 32;
    a.q = d_aq;
    a.scale = d_as;
    a.sum = d_asum;
    return kxw4_gemm(&d, &a, d_y, KXW4_F32, nullptr, offsets, segments, 0, g_stream);
}

void x_quantize_act_chunk_s4(const float *d_x, int K, int T, uint8_t *d_aq4, float *d_as4,
                             int32_t *d_asum4) {
    kxw4_quantize_act_s4(d_x, KXW4_F32, T, K, d_aq4, d_as4, d_asum4, g_stream);
}

int x_gemm_w4a4(const tq_qmma_weight_t *w, const uint8_t *d_aq4, const float *d_as4,
                const int32_t *d_asum4, float *d_y, int T) {
    if (!w || !w->s4_ready || !w->s4_k64 || !w->d_s4 || !w->d_s4_scale) return -1;
    if (!d_aq4 || !d_as4 || !d_asum4 || !d_y || T <= 0 || (T % 8) != 0) return -2;
    const kxw4_weight_t d = w4_of(w);
    return kxw4_gemm_w4a4(&d, d_aq4, d_as4, d_asum4, T, d_y, KXW4_F32, nullptr, g_stream);
}

int x_gemv_w8a8_prepared(const tq_qmma_weight_t *w, float *d_y, const float *d_residual) {
    if (!w8_ready(w) || !d_y) return -1;
    if (g_act.K != w->K) return -2;
    const kxw4_weight_t d = w8_of(w);
    const kxw4_act_t a = prepared_act();
    return kxw4_gemv(&d, &a, d_y, KXW4_F32, d_residual, 0, g_stream);
}

int x_gemv_w8a8(const tq_qmma_weight_t *w, const float *d_x, float *d_y) {
    if (!w || !d_x) return -1;
    x_prepare_gemv_act_s8(d_x, w->K);
    return x_gemv_w8a8_prepared(w, d_y, nullptr);
}

int x_gemv_w8a8_add(const tq_qmma_weight_t *w, const float *d_x, const float *d_residual, float *d_y) {
    if (!w || !d_x || !d_residual) return -1;
    x_prepare_gemv_act_s8(d_x, w->K);
    return x_gemv_w8a8_prepared(w, d_y, d_residual);
}

int x_gemm_w8a8(const tq_qmma_weight_t *w, const int8_t *d_aq, const float *d_as, float *d_y, int T) {
    if (!w8_ready(w)) return -1;
    if (!d_aq || !d_as || !d_y || T <= 0 || (T % 8) != 0) return -2;
    const kxw4_weight_t d = w8_of(w);
    kxw4_act_t a;
    a.T = T;
    a.K = w->K;
    a.block = 32;
    a.q = d_aq;
    a.scale = d_as;
    a.sum = nullptr;
    return kxw4_gemm(&d, &a, d_y, KXW4_F32, nullptr, nullptr, 0, 1, g_stream);
}

// kernels_core.cpp:235-252: W8A8 first, then W4A8.
int x_gemv_qmma_prepared(const tq_qmma_weight_t *w, const float *d_x, float *d_y,
                         const float *d_residual) {
    if (!w || !d_x || !d_y) return -1;
    if (w->s8_ready) return x_gemv_w8a8_prepared(w, d_y, d_residual);
    if (w->s4_ready) return x_gemv_w4a8_prepared(w, d_y, d_residual);
    return KXW4_ETIER;
}

int x_gemv_qmma_add(const tq_qmma_weight_t *w, const float *d_x, const float *d_residual, float *d_y) {
    if (!w || !d_x || !d_residual || !d_y) return -1;
    if (w->s8_ready) return x_gemv_w8a8_add(w, d_x, d_residual, d_y);
    if (w->s4_ready) return x_gemv_w4a8_add(w, d_x, d_residual, d_y);
    return KXW4_ETIER;
}
