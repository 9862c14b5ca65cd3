// kxw4_compat.hpp — the reference's C++ projection interface over libkxw4.so.
//
// Code written against knivesysl-xe's projection functions
// (xpu/src/tq_common.hpp:385-461) compiles and links unchanged against this
// header: same names, same signatures, same return codes. The functions are
// shims over the C ABI in kxw4.h. Differences a caller sees:
//   * d_s4 / d_s4_scale hold the CDNA4 tile layout of kxw4.h, produced by
//     x_w4_repack_weight[_mode] (or kxw4_import_ref_weight from the Xe2
//     layout), not the Xe2 DPAS layout;
//   * activation codes written by x_quantize_act_s8 / x_quantize_act_chunk
//     follow kxw4_act_t's slot order, and sums are per K32 block (the
//     buffers the reference sizes K/16 or [K/32][T] are large enough);
//   * s4 codes written by x_quantize_act_chunk_s4 follow kxw4.h's s4 tile
//     order (T*K/2 bytes, as the reference sizes aq4); scales and sums keep
//     the reference's [K/64][T] layout;
//   * every call runs on the stream set by kxw4_compat_set_stream (the null
//     stream by default), the counterpart of the reference's one in-order
//     queue per rank (decode.cpp:86-99);
//   * x_gemv_w4a8_prepared / x_gemv_w8a8_prepared return -2 unless the last
//     prepare had the weight's K; the reference checks only the scratch
//     capacity (kernels_dpas.cpp:1636) and would read a stale activation.
// Like the reference, the prepared activation (x_prepare_gemv_act_s8,
// x_silu_mul_quant, x_rmsnorm_quant) lives in library-owned grow-only scratch
// and stays valid until the next prepare; these calls are not thread-safe.
#ifndef KXW4_COMPAT_HPP
#define KXW4_COMPAT_HPP

#include <stddef.h>
#include <stdint.h>

#include "kxw4.h"

// The W4-relevant members of the reference descriptor (tq_common.hpp:49-76),
// field names kept. Members of tiers this library does not build (e2m1,
// row_major, ...) are present so code that sets them compiles; they are
// ignored.
typedef struct {
    int M, K, Mt, Kt;          // Mt = M/16, Kt = K/32
    float inv_scale;
    uint8_t *d_A;              // dense-E2M3 payload [Mt][Kt][384 B] (input of the repack)
    float *d_block_scale_inv;  // [scale_rows][scale_cols]
    int block_scaled;
    int row_major;
    int word_major;
    int e2m3;
    int e2m1;
    int e2m3_byte;
    int scale_rows;
    int scale_cols;
    uint8_t *d_s4;             // packed codes, kxw4.h layout
    uint16_t *d_s4_scale;      // [M/16][K/group][16] FP16|zp
    int s4_ready;
    int s4_k16;
    int s4_k64;                // 1 = one scale per K64 group
    uint8_t *d_s8;             // W8A8 tier: int8 codes, kxw4.h W8 tile layout
    uint16_t *d_s8_scale;      // [M/16][K/32][16] FP16
    int s8_ready;
} tq_qmma_weight_t;

extern "C" void kxw4_compat_set_stream(void *stream);

// kernels_dpas.cpp:403-424. mode 0 = K32 groups, 1 = K16 groups (the K16
// tier: GEMV only), 2 = K64 groups. Allocates d_s4/d_s4_scale, frees d_A and
// d_block_scale_inv, synchronizes.
int x_w4_repack_weight(tq_qmma_weight_t *w);
int x_w4_repack_weight_mode(tq_qmma_weight_t *w, int mode);
// kernels_dpas.cpp:558-575: the W8A8 tier (d_s8 / d_s8_scale in the W8 tile
// layout of kxw4.h); allocates, frees d_A and d_block_scale_inv, synchronizes.
int x_w8_repack_weight(tq_qmma_weight_t *w);
// kernels_dpas.cpp:220-223: one token, block 32.
void x_quantize_act_s8(const float *d_x, int K, int8_t *d_q, float *d_scale, int32_t *d_sum);
// kernels_dpas.cpp:1631-1680 and 846-849.
int x_gemv_w4a8(const tq_qmma_weight_t *w, const float *d_x, float *d_y);
int x_gemv_w4a8_add(const tq_qmma_weight_t *w, const float *d_x, const float *d_residual, float *d_y);
void x_prepare_gemv_act_s8(const float *d_x, int K);
// kernels_dpas.cpp:851-855, 866-929.
void x_silu_mul_quant(float *d_out, const float *d_gate, const float *d_up, int K);
void x_rmsnorm_quant(float *d_out, const float *d_in, const uint16_t *d_w, int H, float eps);
// kernels_dpas.cpp:1124-1144: T rows, no quantization.
void x_rmsnorm_chunk(float *d_out, const float *d_in, const uint16_t *d_w, int H, int T, float eps);
// kernels_dpas.cpp:945-1102.
int x_gemv_w4a8_fanout(const tq_qmma_weight_t *const *ws, float *const *ys, int count);
// kernels_dpas.cpp:1149-1207: T token rows, block 32.
void x_quantize_act_chunk(const float *d_x, int K, int T, int8_t *d_aq, float *d_as, int32_t *d_asum);
// kernels_dpas.cpp:1334-1490.
int x_gemm_w4a8(const tq_qmma_weight_t *w, const int8_t *d_aq, const float *d_as,
                const int32_t *d_asum, float *d_y, int T, const int *offsets = nullptr,
                int segments = 0);
int x_gemv_w4a8_prepared(const tq_qmma_weight_t *w, float *d_y, const float *d_residual = nullptr);
// kernels_dpas.cpp:1492-1498: s4 activations of the W4A4 GEMM.
void x_quantize_act_chunk_s4(const float *d_x, int K, int T, uint8_t *d_aq4, float *d_as4,
                             int32_t *d_asum4);
// kernels_dpas.cpp:1500-1571: -1 unless the weight is the K64 tier, -2 for a
// missing operand or T % 8 != 0.
int x_gemm_w4a4(const tq_qmma_weight_t *w, const uint8_t *d_aq4, const float *d_as4,
                const int32_t *d_asum4, float *d_y, int T);
// kernels_dpas.cpp:1682-1725 (W8A8 GEMV on the prepared activation) and
// 1578-1629 (W8A8 GEMM, T % 8 == 0, block-32 chunk activations).
int x_gemv_w8a8_prepared(const tq_qmma_weight_t *w, float *d_y, const float *d_residual = nullptr);
int x_gemv_w8a8(const tq_qmma_weight_t *w, const float *d_x, float *d_y);
int x_gemv_w8a8_add(const tq_qmma_weight_t *w, const float *d_x, const float *d_residual, float *d_y);
int x_gemm_w8a8(const tq_qmma_weight_t *w, const int8_t *d_aq, const float *d_as, float *d_y, int T);
// kernels_core.cpp:235-252: W8A8 when s8_ready, else W4A8 when s4_ready,
// otherwise KXW4_ETIER.
int x_gemv_qmma_prepared(const tq_qmma_weight_t *w, const float *d_x, float *d_y,
                         const float *d_residual = nullptr);
int x_gemv_qmma_add(const tq_qmma_weight_t *w, const float *d_x, const float *d_residual, float *d_y);

#endif  // KXW4_COMPAT_HPP
