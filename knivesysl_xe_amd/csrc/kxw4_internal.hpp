// kxw4_internal.hpp — launch interfaces between the C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kxw4 {

enum { kVarGemv = 0, kVarFanout = 1, kVarGemm = 2 };
constexpr int kMaxWeights = 4;
constexpr int kMaxSegments = 8;

struct DecodeWeight {
    const uint8_t *codes;
    const uint16_t *scales;
    void *y;
    int M;
    int rg_begin;                     // first row-group of this weight over all weights (set by the launcher)
    int seg_split[kMaxSegments];      // split count per packed segment
};

struct DecodeArgs {
    DecodeWeight w[kMaxWeights];
    int count;
    const int8_t *q;
    const float *ascale;
    const int32_t *asum;
    const float *residual;
    int32_t *dbg;
    int T, K, group, block, scale_enc, y_bf16, variant;
    int w8;                           // int8 weight codes (the W8A8 tier)
    int seg_count;
    int seg_end[kMaxSegments];        // exclusive token end of each segment
    int ts;                           // tokens per work-group slice (set by the launcher)
    int smax;                         // largest split count of any token (set by the launcher)
    int total_rg;                     // row-groups over all weights (set by the launcher)
    // row-wave kernel plan (set by its launcher): split count, waves per
    // slice, slices per work-group, 8-row halves over all weights, most
    // row-groups one work-group touches
    int rw_S, rw_wrg, rw_spw, rw_halves, rw_grmax;
};

struct GemmWeight {
    const uint8_t *codes;
    const uint16_t *scales;
    void *y;
    int M;
    int nt_begin;                     // first 128-row n-tile (set by the launcher)
    int seg_split[kMaxSegments];      // split count per packed segment
};

struct GemmArgs {
    GemmWeight w[kMaxWeights];
    int count;
    const int8_t *q;
    const float *ascale;
    const int32_t *asum;
    const float *residual;
    int32_t *dbg;
    int T, K, group, block, scale_enc, y_bf16;
    int w8;                           // int8 weight codes (the W8A8 tier)
    int seg_count;
    int seg_end[kMaxSegments];        // exclusive token end of each segment
    int n_tiles, t_tiles;             // set by the launcher
    int raster_tt;                    // token tiles per raster group (set by the launcher)
};

int launch_pack(const int8_t *codes, const uint16_t *scales, int M, int K, int group,
                uint8_t *out_codes, uint16_t *out_scales, hipStream_t st);
int launch_unpack(const uint8_t *codes, const uint16_t *scales, int M, int K, int group,
                  int8_t *out_codes, uint16_t *out_scales, hipStream_t st);
int launch_import_ref(const uint8_t *ref_codes, const uint16_t *ref_scales, int M, int K,
                      int group, uint8_t *out_codes, uint16_t *out_scales, hipStream_t st);
int launch_repack_e2m3(const uint8_t *payload, const float *bs, int scale_cols, int M, int K,
                       int group, uint8_t *out_codes, uint16_t *out_scales, hipStream_t st);

int launch_pack_s8(const int8_t *codes, const uint16_t *scales, int M, int K, uint8_t *out_codes,
                   uint16_t *out_scales, hipStream_t st);
int launch_unpack_s8(const uint8_t *codes, const uint16_t *scales, int M, int K, int8_t *out_codes,
                     uint16_t *out_scales, hipStream_t st);
int launch_repack_e2m3_s8(const uint8_t *payload, const float *bs, int scale_cols, int M, int K,
                          uint8_t *out_codes, uint16_t *out_scales, hipStream_t st);

int launch_quantize(const void *x, int x_dtype, int T, int K, int block, int8_t *q,
                    float *scale, int32_t *sum, hipStream_t st);
int launch_silu_mul_quant(float *out, const float *gate, const float *up, int T, int K,
                          int block, int8_t *q, float *scale, int32_t *sum, hipStream_t st);
int launch_rmsnorm(float *out, const float *in, const uint16_t *w, int T, int H, float eps, hipStream_t st);
int launch_rmsnorm_quant(float *out, const float *in, const uint16_t *w, int T, int H, float eps,
                         int block, int8_t *q, float *scale, int32_t *sum, hipStream_t st);

// s4 activations of the W4A4 GEMM: q4 [K/128][T][64 B], scale and sum [K/64][T]
int launch_quantize_s4(const void *x, int x_dtype, int T, int K, uint8_t *q4, float *scale,
                       int32_t *sum, hipStream_t st);

struct W4a4Args {
    const uint8_t *q4;                // [K/128][T][64 B] s4 tiles
    const float *as4;                 // [K/64][T]
    const uint8_t *codes;             // packed K64 weight, FP16|zp scales
    const uint16_t *scales;
    void *y;
    const float *residual;
    int M, K, T, y_bf16;
    int n_tiles, t_tiles;             // set by the launcher
};
int launch_w4a4(W4a4Args &a, hipStream_t st);

// compute units of the current device (cached per device)
int device_cus();

int launch_decode(DecodeArgs &a, bool debug, hipStream_t st);
// Return 1 (nothing launched) when the shape is outside the kernel's range.
int launch_rowwave(DecodeArgs &a, hipStream_t st);
int launch_gemm(GemmArgs &a, bool debug, hipStream_t st);
// Returns 1 (nothing launched) outside the per-token, one-split-per-token mode.
int launch_gemm3(GemmArgs &a, hipStream_t st);
// Returns 1 (nothing launched) outside the reference mode (K32 activation
// blocks, W4 codes) with one split per token.
int launch_gemmr(GemmArgs &a, hipStream_t st);

// Kernel-selection options (kxw4_set_option): process-wide, read by the
// launchers. Defaults select the kernels measured fastest; the others keep
// every kernel reachable for tests and A/B timing. Initialised once per
// process from the KXW4_* environment variables of the same names.
enum { kDecodeAuto = 0, kDecodeKParallel = 1, kDecodeRowwave = 2 };
enum { kGemmAuto = 0, kGemmGeneral = 1 };
struct Options {
    int decode_kernel = kDecodeAuto;  // KXW4_DECODE_KERNEL: auto / kparallel / rowwave
    int rowwave_spw = 0;              // KXW4_ROWWAVE_SPW: row slices per work-group, 0 = launcher's plan
    int rowwave_ring = 0;             // KXW4_ROWWAVE_RING: weight tiles in flight per wave, 8 (else 4)
    int rowwave_k = 0;                // KXW4_ROWWAVE_K: work-groups per CU, 0 = launcher's plan
    int gemm_kernel = kGemmAuto;      // KXW4_GEMM_KERNEL: auto / general
    int gemm3_tile = -1;              // KXW4_GEMM3_TILE: 0..11, -1 = cost model
    int gemm3_raster = 0;             // KXW4_GEMM3_RASTER: token tiles per raster group, 0 = 4
    int gemmr_tile = -1;              // KXW4_GEMMR_TILE: 0..9, -1 = default
    int w4a4_tile = -1;               // KXW4_W4A4_TILE: 0..4, -1 = default rule
};
const Options &options();

}  // namespace kxw4
