/*
 * w4a8_oracle.h — CPU restatement of the reference W4A8 projection arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product (knivesysl_xe_amd/) never links or calls it.
 *
 * Every function cites the reference file:line it restates; paths are relative
 * to the reference repository root (SRSWTI/knivesysl-xe). Names follow the
 * reference: a weight has M output rows and K columns, a batch has T tokens,
 * outputs are y[T][M].
 *
 * Arithmetic modes
 *   reference mode : activation block 32 (one FP32 scale per (token, K32)),
 *                    weight group 32 or 64, FP16 scale with the signed zero
 *                    point in its low nibble (ORC_SCALE_FP16_ZP4).
 *   config mode    : per-token activation scale (block 0), weight group 64 or
 *                    128, plain FP16 scale, zero point 0 (ORC_SCALE_FP16).
 *   W8A8 mode      : int8 weight codes with plain FP16 scales per K32
 *                    (ORC_SCALE_S8) and block-32 activations: the reference
 *                    mode arithmetic with zero point 0 (kernels_dpas.cpp:
 *                    771-844 GEMV, 1578-1629 GEMM).
 *   K16 tier       : FP16|zp scales per K16 half, block-32 activations, the
 *                    GEMV only: per K32 tile two half partials, one serial
 *                    accumulator, splits on K32 tiles (kernels_dpas.cpp:
 *                    683-760).
 *   W4A4 mode      : s4 activations (block 64: codes in [-7, 7], one FP32
 *                    scale and one code sum per (token, K64)), K64 weights
 *                    with FP16|zp scales, the GEMM variant (x_gemm_w4a4,
 *                    kernels_dpas.cpp:1500-1571).
 * The int32 "unit" partial is taken over min(weight group, activation block);
 * it is exact in every mode.
 *
 * Pinning (what checks each function against something other than itself):
 *   conversions      numpy IEEE RNE, all 65536 FP16 codes, BF16 ties
 *   quantizers       golden vectors written from numpy (the reference's
 *                    chunk_quant_bench edge pattern), round-half-even ties;
 *                    the s4 quantizer by its closed-form properties (|q| <= 7,
 *                    the absmax element at +-7, |v - q s| <= s/2, zero and
 *                    NaN blocks, exact sums)
 *   partials         numpy int64 matrix products
 *   projection       exact-rational cases, hand-derived accumulation-order
 *                    cases per variant, all-ones => K, GEMM-vs-GEMV cosine gate;
 *                    W4A4: all-ones => K, zero-point cases, and the reference's
 *                    W4A4-vs-W4A8 cosine gate (kernels_dpas.cpp:2346-2409)
 *   split plans      the reference's stated values for the BASELINE shapes
 *   orc_e2m3         the OCP FP6 E2M3 closed form
 *   orc_e2m3_code_at parity unpinned beyond structure: tests show every
 *                    (row, col) owns a distinct contiguous 6-bit field of its
 *                    384-byte tile, and that each lane's 16 codes are one
 *                    little-endian 96-bit stream in its own 12 bytes (what
 *                    kernels_core.cpp:55-57 states); the (row, col) ->
 *                    (lane, index) map restates kernels_core.cpp:58-75 and no
 *                    reference vector checks it
 *   orc_fit_int8     hand-derived known answers (tests/test_oracle.py):
 *                    a group whose scale moves in both refinements (one or
 *                    three refinements, or the negative side over 127, give
 *                    other bits), grid-exact groups, the -128/127 clamp
 *                    asymmetry, all-zero => 1.0; plus invariants
 *   orc_fit_int4_asym hand-derived known answers: the (sh + 8) & 0xFFF0
 *                    nibble round-up (nibbles 7, 8, 9: truncation and
 *                    round-to-even fail), a group whose scale moves in all
 *                    three refinements (two or four fail), all-positive and
 *                    all-negative groups whose range must start at 0 (a
 *                    range seeded from the data fails); plus invariants
 *   contract         selects how a chain step `acc += x*y` (and the fit's
 *                    least-squares sums) round: 1 = one fused multiply-add,
 *                    what icpx's default contraction makes of the
 *                    reference's source and what the HIP kernels implement;
 *                    0 = separate multiply and add, the literal source. Both
 *                    are restated; which one Intel's compiled reference
 *                    produces is parity unpinned (no reference output pins it)
 *   division         every division here (v/s in the quantizers, (hi-lo)/15
 *                    and num/den in the fits, absmax/127) is IEEE correctly
 *                    rounded. The reference is built with plain
 *                    `icpx -fsycl -O2` (xpu/build.sh:13), whose default
 *                    floating-point model may replace a division by a
 *                    reciprocal approximation; which rounding Intel's
 *                    compiled reference produces is parity unpinned
 *   NaN in the GEMV  quantize_act_s8 reduces |v| with sycl::maximum
 *   quantizer        (kernels_dpas.cpp:203-204), whose result on a NaN input
 *                    depends on the sub-group's reduction order; the chunk
 *                    quantizer takes a NaN-skipping fmax per lane first
 *                    (1170-1172). The oracle applies fmax (NaN skipped) to
 *                    both; the GEMV quantizer's NaN behaviour is parity
 *                    unpinned (finite inputs are unaffected)
 */
#ifndef W4A8_ORACLE_H
#define W4A8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ORC_SCALE_S8: the W8A8 tier, int8 codes in [-128, 127] with plain FP16
 * scales per (row, K32) */
enum { ORC_SCALE_FP16 = 0, ORC_SCALE_FP16_ZP4 = 1, ORC_SCALE_S8 = 2 };
enum { ORC_VAR_GEMV = 0, ORC_VAR_FANOUT = 1, ORC_VAR_GEMM = 2 };

/* ---- scalar conversions ---------------------------------------------- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t b);
float orc_e2m3(uint32_t code);
uint32_t orc_e2m3_code_at(const uint8_t *payload, int Kt, int row, int col);
/* element-wise array forms of the conversions above */
void orc_f32_to_f16_n(const float *x, uint16_t *h, size_t n);
void orc_f16_to_f32_n(const uint16_t *h, float *x, size_t n);
void orc_f32_to_bf16_n(const float *x, uint16_t *b, size_t n);

/* ---- activation quantizers ------------------------------------------- */
/* x[T][K] fp32 -> q[T][K] int8, scale[T][K/block] (block 32) or [T] (block 0),
 * sum[T][K/32] (exact int32 code sums per K32; may be NULL). */
int orc_quantize_act(const float *x, int T, int K, int block, int8_t *q,
                     float *scale, int32_t *sum);
/* x[T][K] fp32 -> s4 codes q[T][K] (int8 holding [-7, 7]), scale and code
 * sum [T][K/64] (x_quantize_act_chunk_s4). */
int orc_quantize_act_s4(const float *x, int T, int K, int8_t *q, float *scale, int32_t *sum);
/* out[i] = (g/(1+exp(-g))) * up[i] */
void orc_silu_mul(const float *gate, const float *up, float *out, int n);
/* out[i] = in[i] * rsqrt(mean(in^2)+eps) * (1 + bf16(w[i])) */
void orc_rmsnorm(const float *in, const uint16_t *w_bf16, int H, float eps,
                 float *out);

/* ---- weight side ------------------------------------------------------ */
uint16_t orc_fit_int4_asym(const float *wf, int n, int reserve_nibble,
                           int contract, int *out_z);
/* E2M3 fragment payload + block scales -> natural int4 codes [M][K] and
 * packed FP16|zp scales [M][K/group]; mode 0 = K32 groups, 1 = K16 (the K16
 * tier), 2 = K64. */
int orc_repack_e2m3(const uint8_t *payload, const float *block_scale_inv,
                    int scale_cols, int M, int K, int mode, int contract,
                    int8_t *codes, uint16_t *scales);
/* W8A8 tier: the int8 fit of w8_repack_kernel and the E2M3 -> int8 repack
 * (natural codes [M][K], FP16 scales [M][K/32]). */
uint16_t orc_fit_int8(const float *wf, int n, int contract);
int orc_repack_e2m3_s8(const uint8_t *payload, const float *block_scale_inv,
                       int scale_cols, int M, int K, int contract,
                       int8_t *codes, uint16_t *scales);
/* natural codes/scales <-> the reference's lane-major K32 DPAS layout */
int orc_pack_ref_layout(const int8_t *codes, const uint16_t *scales, int M,
                        int K, int group, uint8_t *ref_codes,
                        uint16_t *ref_scales);
int orc_unpack_ref_layout(const uint8_t *ref_codes, const uint16_t *ref_scales,
                          int M, int K, int group, int8_t *codes,
                          uint16_t *scales);

/* ---- split plans ------------------------------------------------------ */
int orc_gemv_splits(int groups);
int orc_gemm_splits(int rgroups, int tgroups, int ktiles, int forced);
/* Per-token split count for a packed GEMM; offsets has segments+1 entries
 * (NULL for a single segment of T tokens). Returns 0 or -2. */
int orc_segment_splits(const int *offsets, int segments, int T, int M, int K,
                       int forced, int *split_per_token);

/* ---- projection ------------------------------------------------------- */
typedef struct {
    int M, K, group, scale_enc;
    const int8_t *codes;     /* [M][K], values in [-8, 7] */
    const uint16_t *scales;  /* [M][K/group] */
} orc_weight_t;

typedef struct {
    int T, K, block;         /* block: 32, 64 (s4, W4A4) or 0 (per token) */
    const int8_t *q;         /* [T][K] */
    const float *scale;      /* [T][K/block] or [T] */
    const int32_t *sum;      /* [T][K/32], or [T][K/64] for block 64 */
} orc_act_t;

/* Exact int32 unit partials P[T][M][K/unit]. */
int orc_partials(const orc_weight_t *w, const orc_act_t *a, int32_t *P);

/* y[T][M] (fp32 or bf16) for rows [row_begin, row_end); other rows untouched.
 * split_per_token[T] gives each token's split count. residual is [T][M] fp32
 * or NULL. */
int orc_project(const orc_weight_t *w, const orc_act_t *a, int variant,
                const int *split_per_token, int contract,
                const float *residual, int out_bf16, void *y, int row_begin,
                int row_end);

int orc_num_threads(void);
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
