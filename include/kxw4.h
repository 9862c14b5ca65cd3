/*
 * kxw4.h — C ABI of libkxw4.so, the MI355X (gfx950) W4A8 projection library.
 *
 * Drop-in boundary for the projection path of knivesysl-xe: every entry point
 * below replaces one C++-linkage function of the reference's projection
 * interface (xpu/src/tq_common.hpp:385-461), with the stream and every scratch
 * buffer made explicit so the library holds no hidden state. Plain pointers
 * and sizes only; `stream` is a hipStream_t passed as void* (NULL = the null
 * stream). All device pointers must be 16-byte aligned. Calls enqueue work and
 * return without synchronizing (as the reference's in-order queue does).
 *
 * Names follow the reference: a weight has M output rows and K columns; a
 * batch has T tokens; outputs are y[T][M] row-major.
 *
 * Return codes: 0 on success, negative on rejected arguments. The reference's
 * numbers keep their meaning: -1 missing/unprepared operand or wrong tier,
 * -2 bad shape, offsets or split plan (kernels_dpas.cpp:1336-1367, 1633-1636),
 * -3 activation not prepared and -4 split plan the fused reduction cannot
 * close (fan-out, 947-967). -5 names a tier this library does not build and
 * -6 a HIP runtime error.
 */
#ifndef KXW4_H
#define KXW4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KXW4_ABI_VERSION 1

enum {
    KXW4_OK = 0,
    KXW4_EARG = -1,
    KXW4_ESHAPE = -2,
    KXW4_EPREP = -3,
    KXW4_ESPLIT = -4,
    KXW4_ETIER = -5,
    KXW4_EHIP = -6
};

/* Scale encodings. FP16_ZP4 is the reference's packing: FP16 scale whose low
 * four mantissa bits carry a signed zero point (kernels_dpas.cpp:253-255,
 * decode 630-634). FP16 is a plain FP16 scale with zero point 0. W8 marks the
 * W8A8 tier (kernels_dpas.cpp:346-399, 771-844, 1578-1629): int8 codes in
 * the W8 tile layout below with a plain FP16 scale per (row, K32); group 32
 * and block-32 activations only. */
enum { KXW4_SCALE_FP16 = 0, KXW4_SCALE_FP16_ZP4 = 1, KXW4_SCALE_W8 = 2 };

/* Element types of activations, residuals and outputs. */
enum { KXW4_F32 = 0, KXW4_BF16 = 1 };

/* One packed W4 projection (the W4 fields of tq_qmma_weight_t,
 * tq_common.hpp:49-76).
 *   codes : M*K/2 bytes. Tiles of 16 rows x 128 K = 1024 bytes, tile
 *           (rg, kb) at byte (rg*(K/128) + kb)*1024. Inside a tile, lane
 *           l in [0,64) owns bytes [16l, 16l+16): row rg*16 + l%16, and
 *           dword i (0..3) holds k = kb*128 + 32i + 8(l/16) + b for
 *           b = 0..3 in the low nibbles of bytes 0..3 and b = 4..7 in the
 *           high nibbles. Nibbles are two's-complement int4.
 *   scales: [M/16][K/group][16] uint16 (row within the row-group fastest).
 * W8 weights (scale_enc KXW4_SCALE_W8): codes are M*K bytes, tiles of 16 rows
 * x 128 K = 2048 bytes at (rg*(K/128) + kb)*2048; half h at byte 1024h, lane
 * l owns bytes [1024h + 16l, +16) of row rg*16 + l%16, holding K32 units
 * j = 2h (bytes 0..7) and 2h+1 (bytes 8..15), byte b of unit j being
 * k = kb*128 + 32j + 8(l/16) + b (the K slots the W4 unpack produces).
 * Requires M % 16 == 0, K % 128 == 0, group in {16, 32, 64, 128} (32 for W8;
 * 16 is the K16 tier: FP16|zp scales, GEMV only). */
typedef struct kxw4_weight {
    int32_t M, K, group, scale_enc;
    const uint8_t *codes;
    const uint16_t *scales;
} kxw4_weight_t;

/* Quantized activations.
 *   q     : [T][K] int8. Inside every 64-element chunk, byte 16g + 8h + b
 *           holds k = 32h + 8g + b (g in 0..3, h in 0..1, b in 0..7), the
 *           operand order of the int8 MFMA.
 *   scale : [T][K/32] (block 32) or [T] (block 0 = one scale per token).
 *   sum   : [T][K/32] exact int32 code sums (needed by zero-point weights).
 * Requires K % 128 == 0. */
typedef struct kxw4_act {
    int32_t T, K, block;
    const int8_t *q;
    const float *scale;
    const int32_t *sum;
} kxw4_act_t;

int kxw4_abi_version(void);
const char *kxw4_error_string(int code);

/* Kernel-selection options, process-wide, for A/B timing and tests (the
 * counterpart of the reference's once-per-process TQ_XPU_GEMM_SPLITS read,
 * kernels_dpas.cpp:1227-1233; the split override itself is the explicit
 * `forced_splits` argument of kxw4_gemm). Each option starts from the
 * environment variable KXW4_<NAME> read once per process; the defaults pick
 * the kernels measured fastest and the results are the same bits either way.
 *   decode_kernel      0 auto, 1 K-parallel kernel only, 2 row-wave kernel
 *                      wherever it applies
 *   rowwave_spw        row slices per row-wave work-group, 0 = launcher's plan
 *   rowwave_k          row-wave work-groups per CU, 0 = launcher's plan
 *   rowwave_ring       8 = eight weight tiles in flight per wave (else 4)
 *   gemm_kernel        0 auto, 1 the general GEMM for every prefill shape
 *   gemm3_tile         -1 cost model, 0..11 one 32x32x32 GEMM tile
 *   gemmr_tile         -1 default, 0..9 one reference-mode (K32 activation
 *                      block) GEMM tile
 *   gemm3_raster       0 default (4), 1..64 token tiles per XCD raster
 *                      group of the per-token large-tile GEMM
 *   w4a4_tile          -1 default rule, 0..4 one W4A4 GEMM tile
 * Returns 0, -1 for an unknown name, -2 for a value out of range; *previous
 * (may be NULL) receives the old value. Not synchronised with launches in
 * flight on other host threads. */
int kxw4_set_option(const char *name, int value, int *previous);

/* Bytes of packed codes and number of scale entries of one weight. */
size_t kxw4_code_bytes(int M, int K);
size_t kxw4_scale_count(int M, int K, int group);

/* Split plans. choose_gemv_splits, kernels_dpas.cpp:170-173. */
int kxw4_gemv_splits(int groups);
/* choose_gemm_splits, kernels_dpas.cpp:1226-1250; forced in {1,2,4,8,16}
 * replaces the TQ_XPU_GEMM_SPLITS override, anything else = heuristic. */
int kxw4_gemm_splits(int rgroups, int tgroups, int ktiles, int forced);

/* ---- weights (load time) ------------------------------------------------ */

/* Natural int4 codes [M][K] (int8 values in [-8,7]) and scales [M][K/group]
 * -> packed layout. Replaces the packing half of x_w4_repack_weight_mode
 * (kernels_dpas.cpp:403-424) for callers that already hold integer codes. */
int kxw4_pack_weight(const int8_t *codes, const uint16_t *scales, int M, int K,
                     int group, uint8_t *out_codes, uint16_t *out_scales,
                     void *stream);

/* Inverse of kxw4_pack_weight (tests and export). */
int kxw4_unpack_weight(const kxw4_weight_t *w, int8_t *codes, uint16_t *scales,
                       void *stream);

/* W8A8 tier: natural int8 codes [M][K] and FP16 scales [M][K/32] -> the W8
 * tile layout (KXW4_SCALE_W8). kxw4_unpack_weight inverts it. */
int kxw4_pack_weight_s8(const int8_t *codes, const uint16_t *scales, int M,
                        int K, uint8_t *out_codes, uint16_t *out_scales,
                        void *stream);

/* x_w8_repack_weight (kernels_dpas.cpp:346-399, 558-575): dense-E2M3
 * fragment payload and FP32 block scales -> int8 codes (per (row, K32):
 * s = max(hi/127, neg/128), two least-squares refinements, FP16 scale,
 * codes rint(w/s) clamped to [-128, 127]) in the W8 tile layout. */
int kxw4_repack_e2m3_s8(const uint8_t *payload, const float *block_scale_inv,
                        int scale_cols, int M, int K, uint8_t *out_codes,
                        uint16_t *out_scales, void *stream);

/* Reference DPAS layout (lane-major K32 tiles and FP16|zp scales
 * [M/16][K/group][16], kernels_dpas.cpp:294-342) -> packed layout. Scales are
 * copied bit for bit; group is 16 (s4_k16), 32 or 64 (s4_k64). */
int kxw4_import_ref_weight(const uint8_t *ref_codes, const uint16_t *ref_scales,
                           int M, int K, int group, uint8_t *out_codes,
                           uint16_t *out_scales, void *stream);

/* x_w4_repack_weight_mode (kernels_dpas.cpp:266-344, 403-424): dense-E2M3
 * fragment payload [M/16][K/32][384 B] and FP32 block scales
 * [ceil(M/128)][scale_cols] -> asymmetric int4 fit per group with the zero
 * point in the FP16 scale nibble. mode 0 = K32 groups, 1 = K16 groups (the
 * K16 tier, kernels_dpas.cpp:287-296), 2 = K64 groups. Outputs use
 * KXW4_SCALE_FP16_ZP4. */
int kxw4_repack_e2m3(const uint8_t *payload, const float *block_scale_inv,
                     int scale_cols, int M, int K, int mode, uint8_t *out_codes,
                     uint16_t *out_scales, void *stream);

/* ---- activations ---------------------------------------------------------- */

/* x[T][K] (KXW4_F32 or KXW4_BF16) -> q, scale, sum. block 32 restates
 * x_quantize_act_s8 / x_quantize_act_chunk (kernels_dpas.cpp:188-223,
 * 1149-1207); block 0 applies the same formula once per token row. */
int kxw4_quantize_act(const void *x, int x_dtype, int T, int K, int block,
                      int8_t *q, float *scale, int32_t *sum, void *stream);

/* x_silu_mul_quant (kernels_dpas.cpp:851-855): hidden = silu(gate)*up
 * written to out[T][K] (may be NULL), then quantized as kxw4_quantize_act. */
int kxw4_silu_mul_quant(float *out, const float *gate, const float *up, int T,
                        int K, int block, int8_t *q, float *scale, int32_t *sum,
                        void *stream);

/* x_rmsnorm_quant (kernels_dpas.cpp:866-929), batched over T rows:
 * out = in * rsqrt(mean(in^2) + eps) * (1 + bf16 w), written to out[T][H]
 * (may be NULL), then quantized as kxw4_quantize_act. */
int kxw4_rmsnorm_quant(float *out, const float *in, const uint16_t *w, int T,
                       int H, float eps, int block, int8_t *q, float *scale,
                       int32_t *sum, void *stream);

/* x_rmsnorm_chunk (kernels_dpas.cpp:1124-1144): out[t][i] = in[t][i] *
 * rsqrt(mean(in[t]^2) + eps) * (1 + bf16(w[i])) over T rows of H, the same
 * rows kxw4_rmsnorm_quant writes to its `out`, without the quantizer. */
int kxw4_rmsnorm(float *out, const float *in, const uint16_t *w, int T, int H,
                 float eps, void *stream);

/* s4 activations of the W4A4 GEMM: x_quantize_act_chunk_s4
 * (kernels_dpas.cpp:1492-1498 over 1149-1197). x[T][K] (KXW4_F32 or
 * KXW4_BF16) -> per (token, K64) block s = absmax/7 (1 when the block max is
 * not positive), codes clamp(rint(v/s), -7, 7) and their exact sum.
 *   q4    : T*K/2 bytes, [K/128][T][64 B]: the 64 bytes of (128-K step kb,
 *           token t) have the nibble order of a packed weight tile row —
 *           dword i of 16-byte lane group g holds k = 128kb + 32i + 8g + b,
 *           b = 0..3 in the low nibbles of bytes 0..3, b = 4..7 in the high
 *           nibbles (two's complement).
 *   scale : [K/64][T] FP32, sum: [K/64][T] int32 (the reference's layout).
 * Requires K % 128 == 0. Buffer sizes equal the reference's (aq4, as4, asum4). */
int kxw4_quantize_act_s4(const void *x, int x_dtype, int T, int K, uint8_t *q4,
                         float *scale, int32_t *sum, void *stream);

/* ---- projections -------------------------------------------------------- */

/* x_gemv_w4a8_core arithmetic (kernels_dpas.cpp:586-675) with the
 * x_gemv_w4a8_prepared dispatch (1631-1680): per token row, K split in
 * `splits` parts (0 = choose_gemv_splits(M/16)), two alternating
 * accumulators per split, ordered split sum, optional FP32 residual[T][M].
 * T in [1, 64]. y is [T][M] of y_dtype. A W8 weight runs x_gemv_w8a8_core's
 * arithmetic (kernels_dpas.cpp:771-844, the same chain with zero point 0) for
 * T in [1, 16]. A K16 weight (group 16) runs x_gemv_w4a8_core_k16
 * (683-760): block-32 activations, two K16 half partials per K32 tile, one
 * serial accumulator per split, splits on K32 tiles; T in [1, 16]. W8 and
 * K16 stage every token's activation row in one work-group's LDS: where T
 * rows do not fit (long K: at K = 17408 from T = 7 for W8, from 2-4 tokens
 * for K16 depending on M) the tokens run in chunks that do, each streaming
 * the weights again (same bits, more weight traffic). W4 weights never
 * chunk: a shape whose rows do not fit runs on the K-parallel kernel, which
 * reads the weight once for all T tokens. */
int kxw4_gemv(const kxw4_weight_t *w, const kxw4_act_t *a, void *y, int y_dtype,
              const float *residual, int splits, void *stream);

/* x_gemv_w4a8_fanout (kernels_dpas.cpp:945-1102): up to 4 weights with one K
 * and one group/encoding, one launch, serial accumulator, one split count
 * choose_gemv_splits(total row-groups). T in [1, 64]. W8 weights return
 * KXW4_ETIER (the reference has no W8 fan-out), K16 weights -2 (956-959). */
int kxw4_gemv_fanout(const kxw4_weight_t *const *ws, void *const *ys, int count,
                     const kxw4_act_t *a, int y_dtype, void *stream);

/* x_gemm_w4a8 (kernels_dpas.cpp:1334-1490): serial accumulator, split count
 * per packed segment from choose_gemm_splits(M/16, ceil(rows/8), K/32),
 * ordered split sum. offsets[segments+1] is host memory (NULL with
 * segments 0 for one segment); segments may have any positive length (the
 * reference requires multiples of 8). Optional FP32 residual[T][M] is added
 * after the projection. A W8 weight runs x_gemm_w8a8's arithmetic
 * (kernels_dpas.cpp:1578-1629) on block-32 activations. */
int kxw4_gemm(const kxw4_weight_t *w, const kxw4_act_t *a, void *y, int y_dtype,
              const float *residual, const int *offsets, int segments,
              int forced_splits, void *stream);

/* Up to 4 weights sharing one activation in one launch (gate+up), each with
 * its own split plan; otherwise as kxw4_gemm. No counterpart in the
 * reference, which issues one x_gemm_w4a8 per weight (decode.cpp:1861-1862). */
int kxw4_gemm_fanout(const kxw4_weight_t *const *ws, void *const *ys, int count,
                     const kxw4_act_t *a, int y_dtype, const int *offsets,
                     int segments, int forced_splits, void *stream);

/* x_gemm_w4a4 (kernels_dpas.cpp:1500-1571): s4 activations from
 * kxw4_quantize_act_s4 against a K64 weight with FP16|zp scales (group 64,
 * KXW4_SCALE_FP16_ZP4, else -1). One serial FP32 chain per output over the
 * K64 groups, acc += (float)(d - zp*sum) * (ws*as); y[T][M] FP32 or BF16,
 * plus residual[T][M] (may be NULL). Any T >= 1 (the reference requires
 * T % 8 == 0; its shim keeps that check). */
int kxw4_gemm_w4a4(const kxw4_weight_t *w, const uint8_t *q4, const float *scale,
                   const int32_t *sum, int T, void *y, int y_dtype,
                   const float *residual, void *stream);

/* No counterpart in the reference. For callers that cannot allocate (code
 * under HIP graph capture, tight serving loops): x[T][K] (KXW4_F32 or
 * KXW4_BF16) is quantized per K32 block into a fixed device array of this
 * library (640 KiB per GPU, held until the process ends), then projected as
 * kxw4_gemv with the default split plan, plus residual (may be NULL).
 * Limits: T in [1, 16], K <= 32768 (else -2). Allocates nothing; calls that
 * overlap on one GPU race on the array. */
int kxw4_gemv_x_noalloc(const kxw4_weight_t *w, const void *x, int x_dtype, int T, void *y,
                        int y_dtype, const float *residual, void *stream);

/* ---- TQF1 ingest (host side) ---------------------------------------------
 * The reference's model container (tqf_loader.cpp:393-626): kxw4_tqf_open
 * validates the header as the reference does (BF16 non-quant tensors, dense
 * block-scaled E2M3 QMMA payloads, header size, layer types) and walks the
 * whole tensor sequence, reading no payload; the file must end exactly where
 * the sequence does. Each QMMA record (186-255) can then be repacked straight
 * into caller-owned device buffers: mode 0 / 1 / 2 as kxw4_repack_e2m3 (W4,
 * K32 / K16 / K64 groups), mode 8 as kxw4_repack_e2m3_s8 (W8A8). Errors: -1
 * unreadable file, bad magic or index, -2 bad header or shapes, -5 a payload
 * encoding this library does not ingest, -6 HIP. No counterpart in the
 * reference's projection interface: it replaces the read_qmma +
 * x_w4_repack_weight_mode pair of qwn_load. */
typedef struct kxw4_tqf kxw4_tqf_t;
enum { KXW4_TQF_BF16 = 0, KXW4_TQF_F32 = 1, KXW4_TQF_QMMA = 2 };
typedef struct kxw4_tqf_tensor {
    char name[64];            /* "lm_head", "layer3.mlp_down", "mtp.fc", ... */
    int32_t kind;             /* KXW4_TQF_* */
    int32_t M, K;             /* QMMA: rows, cols; vectors: element count, 1 */
    int32_t scale_rows, scale_cols;   /* QMMA block scales */
    uint64_t offset, bytes;   /* the record's byte range in the file */
} kxw4_tqf_tensor_t;
int kxw4_tqf_open(const char *path, kxw4_tqf_t **out);
void kxw4_tqf_close(kxw4_tqf_t *t);
int kxw4_tqf_count(const kxw4_tqf_t *t);
/* u[16], fl[3] and tail[8] of the header (any may be NULL) */
int kxw4_tqf_header(const kxw4_tqf_t *t, uint32_t *u16, float *f3, uint32_t *tail8);
int kxw4_tqf_tensor(const kxw4_tqf_t *t, int index, kxw4_tqf_tensor_t *out);
/* index of the tensor named `name`, or -1 */
int kxw4_tqf_find(const kxw4_tqf_t *t, const char *name);
/* out_codes: kxw4_code_bytes(M, K) (M*K for mode 8); out_scales:
 * kxw4_scale_count(M, K, group) entries. Synchronizes `stream`. */
int kxw4_tqf_load_qmma(const kxw4_tqf_t *t, int index, int mode,
                       uint8_t *out_codes, uint16_t *out_scales, void *stream);

/* Machine probes (xpu/probe/dpas_probe.cpp, results xpu/PROBE_RESULTS.md:
 * 8-33: DPAS rates with all-ones operands, pure-read bandwidth), the ceilings
 * the roofline fractions are read against besides the published peaks. They
 * enqueue one kernel on `stream`; the caller times it.
 * kxw4_probe_mfma_i8: shape 0 = v_mfma_i32_32x32x32_i8, 1 = _16x16x64_i8,
 * four independent all-ones chains per wave; each wave writes iters * K to
 * its sink word when every accumulator holds exactly that, else -1. *ops
 * receives the launch's integer operation count. kxw4_probe_read: a
 * grid-stride read of `bytes` (16-byte aligned, multiple of 16) in launch
 * shape `shape` (0 .. kxw4_probe_read_shapes() - 1: work-groups per CU,
 * threads, loads in flight per lane), one XOR checksum word per wave. Both
 * return the number of sink words written (sink_words must be at least
 * that: 64K words cover any GPU), or -1 / -2 (sink too small) / -6. */
int kxw4_probe_mfma_i8(int shape, int iters, int32_t *sink, int sink_words, double *ops,
                       void *stream);
int kxw4_probe_read(const void *buf, size_t bytes, int shape, uint32_t *sink, int sink_words,
                    void *stream);
int kxw4_probe_read_shapes(void);
/* kxw4_probe_issue: the per-token GEMM's inner work without memory, one
 * work-group of 4 * waves_per_simd waves (1-4 per SIMD) per CU. A block is
 * four dependent v_mfma_i32_32x32x32_i8 (a 128-K step of a 32x32 output
 * block) and/or its FP32 chain (16 int-to-float conversions and 16 FMAs per
 * lane). mode 0: MFMAs only; 1: chain only; 2: both in one wave, block b's
 * MFMAs interleaved with block b-1's chain; 3: MFMA waves and chain waves
 * side by side on each SIMD (waves_per_simd even). *blocks receives the
 * blocks each SIMD runs. One float per wave (deterministic; 0 for mode 1).
 * No counterpart in the reference's probe: it separates the MFMA and VALU
 * issue ceilings that bound the GEMM. Returns the words written, or -1 / -2 /
 * -6. */
int kxw4_probe_issue(int mode, int waves_per_simd, int iters, float *sink, int sink_words,
                     double *blocks, void *stream);
/* kxw4_probe_hold: one wave that holds `stream` until the host sets *flag
 * (host-pinned memory, e.g. hipHostMalloc) to nonzero or max_us (1 ..
 * 1000000) microseconds have passed, then writes 1 (released) or 2 (timed
 * out) to *status (device memory). A timing harness enqueues it before its
 * start event and sets the flag after submitting the timed launches, so the
 * host's submission time stays out of the timed region (nvbench's blocking
 * kernel). No counterpart in the reference. Returns 0, -1 or -6. */
int kxw4_probe_hold(const uint32_t *flag, int max_us, uint32_t *status, void *stream);

/* Debug: exact int32 unit partials P[T][M][K/unit] (unit = 32 for block 32,
 * else group), from the same unpack and MFMA code as the projections. */
int kxw4_partials(const kxw4_weight_t *w, const kxw4_act_t *a, int32_t *P,
                  void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KXW4_H */
