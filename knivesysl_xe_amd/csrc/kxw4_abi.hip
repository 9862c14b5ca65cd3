// kxw4_abi.hip — the C ABI of libkxw4.so (declared in include/kxw4.h):
// argument checks with the reference's return codes, split plans, and
// dispatch to the kernels.
#include "../../include/kxw4.h"
#include "kxw4_internal.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>

using namespace kxw4;

namespace kxw4 {

namespace {

struct OptionDesc {
    const char *name;
    int Options::*field;
    int lo, hi;
};

const OptionDesc kOptions[] = {
    {"decode_kernel", &Options::decode_kernel, kDecodeAuto, kDecodeRowwave},
    {"rowwave_spw", &Options::rowwave_spw, 0, 16},
    {"gemm_kernel", &Options::gemm_kernel, kGemmAuto, kGemmGeneral},
    {"gemm3_tile", &Options::gemm3_tile, -1, 11},
    {"gemmr_tile", &Options::gemmr_tile, -1, 9},
    {"gemm3_raster", &Options::gemm3_raster, 0, 64},
    {"w4a4_tile", &Options::w4a4_tile, -1, 4},
    {"rowwave_ring", &Options::rowwave_ring, 0, 8},
    {"rowwave_k", &Options::rowwave_k, 0, 64},
};

// The environment is read once, when the library first selects a kernel.
Options from_env() {
    Options o;
    if (const char *e = getenv("KXW4_DECODE_KERNEL")) {
        if (!strcmp(e, "kparallel")) o.decode_kernel = kDecodeKParallel;
        else if (!strcmp(e, "rowwave")) o.decode_kernel = kDecodeRowwave;
    }
    auto num = [](const char *name, int lo, int hi, int &dst) {
        const char *e = getenv(name);
        if (!e || !*e) return;
        const int v = atoi(e);
        if (v >= lo && v <= hi) dst = v;
    };
    num("KXW4_ROWWAVE_SPW", 0, 16, o.rowwave_spw);
    num("KXW4_ROWWAVE_RING", 0, 8, o.rowwave_ring);
    num("KXW4_ROWWAVE_K", 0, 64, o.rowwave_k);
    if (const char *e = getenv("KXW4_GEMM_KERNEL"))
        if (!strcmp(e, "general")) o.gemm_kernel = kGemmGeneral;
    num("KXW4_GEMM3_TILE", -1, 11, o.gemm3_tile);
    num("KXW4_GEMMR_TILE", -1, 9, o.gemmr_tile);
    num("KXW4_GEMM3_RASTER", 0, 64, o.gemm3_raster);
    num("KXW4_W4A4_TILE", -1, 4, o.w4a4_tile);
    return o;
}

Options &mutable_options() {
    static Options o = from_env();
    return o;
}

}  // namespace

const Options &options() { return mutable_options(); }

}  // namespace kxw4

namespace {

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// 16 is the K16 tier (FP16|zp scales, GEMV only)
bool valid_group(int g) { return g == 16 || g == 32 || g == 64 || g == 128; }

// Shape of one packed weight (x_w4_repack_weight_mode, kernels_dpas.cpp:406).
bool valid_shape(int M, int K, int group) {
    return M > 0 && K > 0 && M % 16 == 0 && K % 128 == 0 && valid_group(group);
}

int check_weight(const kxw4_weight_t *w) {
    if (!w || !w->codes || !w->scales) return KXW4_EARG;
    if (!valid_shape(w->M, w->K, w->group)) return KXW4_ESHAPE;
    if (w->scale_enc != KXW4_SCALE_FP16 && w->scale_enc != KXW4_SCALE_FP16_ZP4 &&
        w->scale_enc != KXW4_SCALE_W8)
        return KXW4_ETIER;
    // the W8A8 tier keeps one scale per K32 (kernels_dpas.cpp:346-399), the
    // K16 tier FP16|zp scales (287-296)
    if (w->scale_enc == KXW4_SCALE_W8 && w->group != 32) return KXW4_ESHAPE;
    if (w->group == 16 && w->scale_enc != KXW4_SCALE_FP16_ZP4) return KXW4_ESHAPE;
    return KXW4_OK;
}

int check_act(const kxw4_act_t *a, int K, int scale_enc) {
    if (!a || !a->q || !a->scale) return KXW4_ESHAPE;
    if (a->K != K || a->T <= 0 || (a->block != 0 && a->block != 32)) return KXW4_ESHAPE;
    if (scale_enc == KXW4_SCALE_FP16_ZP4 && !a->sum) return KXW4_EPREP;
    // W8A8 runs on block-32 activations only (kernels_dpas.cpp:771-844, 1578-1629)
    if (scale_enc == KXW4_SCALE_W8 && a->block != 32) return KXW4_EARG;
    return KXW4_OK;
}

bool valid_split(int s) { return s == 1 || s == 2 || s == 4 || s == 8 || s == 16; }

template <class Args>
void fill_act(Args &args, const kxw4_act_t *a, int group, int scale_enc, int y_dtype) {
    args.q = a->q;
    args.ascale = a->scale;
    args.asum = a->sum;
    args.T = a->T;
    args.K = a->K;
    args.group = group;
    args.block = a->block;
    args.scale_enc = scale_enc;
    args.w8 = scale_enc == KXW4_SCALE_W8 ? 1 : 0;
    args.y_bf16 = y_dtype == KXW4_BF16 ? 1 : 0;
}

// Token counts up to this take the decode kernel (kxw4_decode.hip), larger
// ones the LDS-tiled GEMM (kxw4_gemm.hip).
constexpr int kDecodeMaxT = 64;

template <class Args>
void fill_plan(Args &args, const kxw4_weight_t *const *ws, void *const *ys, int count,
               const kxw4_act_t *a, int y_dtype, const float *residual, int32_t *dbg,
               const int *ends, const int (*splits)[kMaxSegments], int nseg) {
    args.count = count;
    for (int i = 0; i < count; ++i) {
        args.w[i].codes = ws[i]->codes;
        args.w[i].scales = ws[i]->scales;
        args.w[i].y = ys[i];
        args.w[i].M = ws[i]->M;
        for (int s = 0; s < nseg; ++s) args.w[i].seg_split[s] = splits[i][s];
    }
    fill_act(args, a, ws[0]->group, ws[0]->scale_enc, y_dtype);
    args.residual = residual;
    args.dbg = dbg;
    args.seg_count = nseg;
    for (int s = 0; s < nseg; ++s) args.seg_end[s] = ends[s];
}

// Per-segment split counts of one weight (kernels_dpas.cpp:1343-1367).
int segment_plan(int M, int K, int T, const int *offsets, int segments, int forced, int *ends,
                 int *splits, int *count) {
    const int rgroups = M / 16, Kt = K / 32;
    if (!offsets) {
        if (segments != 0) return KXW4_ESHAPE;
        *count = 1;
        ends[0] = T;
        splits[0] = kxw4_gemm_splits(rgroups, (T + 7) / 8, Kt, forced);
        return KXW4_OK;
    }
    if (segments < 1 || segments > kMaxSegments || offsets[0] != 0 || offsets[segments] != T)
        return KXW4_ESHAPE;
    for (int i = 0; i < segments; ++i) {
        if (offsets[i + 1] <= offsets[i]) return KXW4_ESHAPE;
        ends[i] = offsets[i + 1];
        splits[i] = kxw4_gemm_splits(rgroups, (offsets[i + 1] - offsets[i] + 7) / 8, Kt, forced);
    }
    *count = segments;
    return KXW4_OK;
}

int gemm_common(const kxw4_weight_t *const *ws, void *const *ys, int count, const kxw4_act_t *a,
                int y_dtype, const float *residual, const int *offsets, int segments, int forced,
                int32_t *dbg, hipStream_t st) {
    if (!ws || !ys || count <= 0 || count > kMaxWeights) return KXW4_EARG;
    for (int i = 0; i < count; ++i) {
        const int rc = check_weight(ws[i]);
        if (rc) return rc;
        if (!ys[i] && !dbg) return KXW4_EARG;
        if (ws[i]->K != ws[0]->K || ws[i]->group != ws[0]->group ||
            ws[i]->scale_enc != ws[0]->scale_enc)
            return KXW4_ESHAPE;
        // the K16 tier has no GEMM (x_gemm_w4a8 returns -1, kernels_dpas.cpp:1337)
        if (ws[i]->group == 16) return KXW4_EARG;
    }
    if (y_dtype != KXW4_F32 && y_dtype != KXW4_BF16) return KXW4_ESHAPE;
    const int rc = check_act(a, ws[0]->K, ws[0]->scale_enc);
    if (rc) return rc;
    const int T = a->T, K = a->K;
    int ends[kMaxSegments], nseg = 0;
    int splits[kMaxWeights][kMaxSegments];
    for (int i = 0; i < count; ++i) {
        const int prc = segment_plan(ws[i]->M, K, T, offsets, segments, forced, ends, splits[i], &nseg);
        if (prc) return prc;
    }
    if (T <= kDecodeMaxT) {
        DecodeArgs args{};
        fill_plan(args, ws, ys, count, a, y_dtype, residual, dbg, ends, splits, nseg);
        args.variant = kVarGemm;
        const int r = launch_decode(args, dbg != nullptr, st);
        // W8 shapes the row-wave kernel does not take run on the GEMM path
        if (!(args.w8 && r == 1)) return r;
    }
    GemmArgs args{};
    fill_plan(args, ws, ys, count, a, y_dtype, residual, dbg, ends, splits, nseg);
    return launch_gemm(args, dbg != nullptr, st);
}

// One split count for every token (the GEMV and fan-out GEMV plans).
int decode_uniform(const kxw4_weight_t *const *ws, void *const *ys, int count,
                   const kxw4_act_t *a, int y_dtype, const float *residual, int S, int variant,
                   hipStream_t st) {
    int ends[1] = {a->T};
    int splits[kMaxWeights][kMaxSegments];
    for (int i = 0; i < count; ++i) splits[i][0] = S;
    DecodeArgs args{};
    fill_plan(args, ws, ys, count, a, y_dtype, residual, nullptr, ends, splits, 1);
    args.variant = variant;
    const int r = launch_decode(args, false, st);
    return r == 1 ? KXW4_ESHAPE : r;
}

}  // namespace

extern "C" {

int kxw4_abi_version(void) { return KXW4_ABI_VERSION; }

int kxw4_set_option(const char *name, int value, int *previous) {
    if (!name) return KXW4_EARG;
    for (const OptionDesc &d : kOptions) {
        if (strcmp(d.name, name) != 0) continue;
        if (value < d.lo || value > d.hi) return KXW4_ESHAPE;
        Options &o = mutable_options();
        if (previous) *previous = o.*(d.field);
        o.*(d.field) = value;
        return KXW4_OK;
    }
    return KXW4_EARG;
}

const char *kxw4_error_string(int code) {
    switch (code) {
    case KXW4_OK: return "ok";
    case KXW4_EARG: return "missing operand or wrong tier";
    case KXW4_ESHAPE: return "bad shape, offsets or split plan";
    case KXW4_EPREP: return "activation not prepared";
    case KXW4_ESPLIT: return "split plan not closable in one work-group";
    case KXW4_ETIER: return "tier not built by this library";
    case KXW4_EHIP: return "HIP runtime error";
    default: return "unknown error";
    }
}

size_t kxw4_code_bytes(int M, int K) { return (size_t)M * (size_t)K / 2; }

size_t kxw4_scale_count(int M, int K, int group) {
    return valid_group(group) ? (size_t)M * (size_t)(K / group) : 0;
}

// kernels_dpas.cpp:170-173.
int kxw4_gemv_splits(int groups) {
    if (groups <= 4) return 16;
    return groups >= 4096 ? 1 : 8;
}

// kernels_dpas.cpp:1226-1250.
int kxw4_gemm_splits(int rgroups, int tgroups, int ktiles, int forced) {
    if (!valid_split(forced)) forced = 0;
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

int kxw4_pack_weight(const int8_t *codes, const uint16_t *scales, int M, int K, int group,
                     uint8_t *out_codes, uint16_t *out_scales, void *stream) {
    if (!codes || !scales || !out_codes || !out_scales) return KXW4_EARG;
    if (!valid_shape(M, K, group)) return KXW4_ESHAPE;
    return launch_pack(codes, scales, M, K, group, out_codes, out_scales, as_stream(stream));
}

int kxw4_unpack_weight(const kxw4_weight_t *w, int8_t *codes, uint16_t *scales, void *stream) {
    const int rc = check_weight(w);
    if (rc) return rc;
    if (!codes) return KXW4_EARG;
    if (w->scale_enc == KXW4_SCALE_W8)
        return launch_unpack_s8(w->codes, w->scales, w->M, w->K, codes, scales, as_stream(stream));
    return launch_unpack(w->codes, w->scales, w->M, w->K, w->group, codes, scales,
                         as_stream(stream));
}

int kxw4_pack_weight_s8(const int8_t *codes, const uint16_t *scales, int M, int K, uint8_t *out_codes,
                        uint16_t *out_scales, void *stream) {
    if (!codes || !scales || !out_codes || !out_scales) return KXW4_EARG;
    if (!valid_shape(M, K, 32)) return KXW4_ESHAPE;
    return launch_pack_s8(codes, scales, M, K, out_codes, out_scales, as_stream(stream));
}

// x_w8_repack_weight's checks (kernels_dpas.cpp:558-560): -1 missing operand,
// -2 shape.
int kxw4_repack_e2m3_s8(const uint8_t *payload, const float *block_scale_inv, int scale_cols, int M,
                        int K, uint8_t *out_codes, uint16_t *out_scales, void *stream) {
    if (!payload || !block_scale_inv || !out_codes || !out_scales || scale_cols <= 0) return KXW4_EARG;
    if (M <= 0 || K <= 0 || M % 16 || K % 128) return KXW4_ESHAPE;
    if (scale_cols != K / 32 && scale_cols != K / 128) return KXW4_ESHAPE;
    return launch_repack_e2m3_s8(payload, block_scale_inv, scale_cols, M, K, out_codes, out_scales,
                                 as_stream(stream));
}

int kxw4_import_ref_weight(const uint8_t *ref_codes, const uint16_t *ref_scales, int M, int K,
                           int group, uint8_t *out_codes, uint16_t *out_scales, void *stream) {
    if (!ref_codes || !ref_scales || !out_codes || !out_scales) return KXW4_EARG;
    if (!valid_shape(M, K, group) || group == 128) return KXW4_ESHAPE;
    return launch_import_ref(ref_codes, ref_scales, M, K, group, out_codes, out_scales,
                             as_stream(stream));
}

// x_w4_repack_weight_mode's checks (kernels_dpas.cpp:404-406): -1 missing
// operand, -2 shape, -3 odd K32 tile count for K64.
int kxw4_repack_e2m3(const uint8_t *payload, const float *block_scale_inv, int scale_cols, int M,
                     int K, int mode, uint8_t *out_codes, uint16_t *out_scales, void *stream) {
    if (!payload || !block_scale_inv || !out_codes || !out_scales || scale_cols <= 0)
        return KXW4_EARG;
    if (M <= 0 || K <= 0 || M % 16 || K % 128) return KXW4_ESHAPE;
    if (mode == 2 && ((K / 32) & 1)) return KXW4_EPREP;
    if (mode != 0 && mode != 1 && mode != 2) return KXW4_ESHAPE;
    if (scale_cols != K / 32 && scale_cols != K / 128) return KXW4_ESHAPE;
    return launch_repack_e2m3(payload, block_scale_inv, scale_cols, M, K, mode == 2 ? 64 : mode == 1 ? 16 : 32,
                              out_codes, out_scales, as_stream(stream));
}

int kxw4_quantize_act(const void *x, int x_dtype, int T, int K, int block, int8_t *q, float *scale,
                      int32_t *sum, void *stream) {
    if (!x || !q || !scale) return KXW4_EARG;
    if (T <= 0 || K <= 0 || K % 64 || (block != 0 && block != 32)) return KXW4_ESHAPE;
    if (x_dtype != KXW4_F32 && x_dtype != KXW4_BF16) return KXW4_ESHAPE;
    return launch_quantize(x, x_dtype, T, K, block, q, scale, sum, as_stream(stream));
}

int kxw4_rmsnorm(float *out, const float *in, const uint16_t *w, int T, int H, float eps,
                 void *stream) {
    if (!out || !in || !w) return KXW4_EARG;
    if (T <= 0 || H <= 0) return KXW4_ESHAPE;
    return launch_rmsnorm(out, in, w, T, H, eps, as_stream(stream));
}

int kxw4_quantize_act_s4(const void *x, int x_dtype, int T, int K, uint8_t *q4, float *scale,
                         int32_t *sum, void *stream) {
    if (!x || !q4 || !scale || !sum) return KXW4_EARG;
    if (T <= 0 || K <= 0 || K % 128 || (x_dtype != KXW4_F32 && x_dtype != KXW4_BF16)) return KXW4_ESHAPE;
    return launch_quantize_s4(x, x_dtype, T, K, q4, scale, sum, as_stream(stream));
}

int kxw4_silu_mul_quant(float *out, const float *gate, const float *up, int T, int K, int block,
                        int8_t *q, float *scale, int32_t *sum, void *stream) {
    if (!gate || !up || !q || !scale) return KXW4_EARG;
    if (T <= 0 || K <= 0 || K % 64 || (block != 0 && block != 32)) return KXW4_ESHAPE;
    return launch_silu_mul_quant(out, gate, up, T, K, block, q, scale, sum, as_stream(stream));
}

int kxw4_rmsnorm_quant(float *out, const float *in, const uint16_t *w, int T, int H, float eps,
                       int block, int8_t *q, float *scale, int32_t *sum, void *stream) {
    if (!in || !w || !q || !scale) return KXW4_EARG;
    if (T <= 0 || H <= 0 || H % 64 || (block != 0 && block != 32)) return KXW4_ESHAPE;
    return launch_rmsnorm_quant(out, in, w, T, H, eps, block, q, scale, sum, as_stream(stream));
}

int kxw4_gemv(const kxw4_weight_t *w, const kxw4_act_t *a, void *y, int y_dtype,
              const float *residual, int splits, void *stream) {
    int rc = check_weight(w);
    if (rc) return rc;
    if (!y) return KXW4_EARG;
    rc = check_act(a, w->K, w->scale_enc);
    if (rc) return rc;
    if (a->T > kDecodeMaxT || (y_dtype != KXW4_F32 && y_dtype != KXW4_BF16)) return KXW4_ESHAPE;
    if ((w->scale_enc == KXW4_SCALE_W8 || w->group == 16) && a->T > 16) return KXW4_ESHAPE;
    if (w->group == 16 && a->block != 32) return KXW4_EARG;   // K16: block-32 activations
    const int S = splits ? splits : kxw4_gemv_splits(w->M / 16);
    if (!valid_split(S)) return KXW4_ESHAPE;
    const kxw4_weight_t *ws[1] = {w};
    void *ys[1] = {y};
    return decode_uniform(ws, ys, 1, a, y_dtype, residual, S, kVarGemv, as_stream(stream));
}

// kernels_dpas.cpp:947-967: -1 bad set, -2 non-uniform tier/K or missing
// output, -3 unprepared activation, -4 split count beyond the fused reducer.
int kxw4_gemv_fanout(const kxw4_weight_t *const *ws, void *const *ys, int count,
                     const kxw4_act_t *a, int y_dtype, void *stream) {
    if (!ws || !ys || count <= 0 || count > kMaxWeights) return KXW4_EARG;
    int groups = 0;
    for (int i = 0; i < count; ++i) {
        const kxw4_weight_t *w = ws[i];
        if (!w || !w->codes || !w->scales || !ys[i] || w->K != ws[0]->K ||
            !valid_shape(w->M, w->K, w->group) || w->group != ws[0]->group ||
            w->scale_enc != ws[0]->scale_enc)
            return KXW4_ESHAPE;
        if (w->scale_enc == KXW4_SCALE_W8) return KXW4_ETIER;   // no W8 fan-out in the reference
        if (w->group == 16) return KXW4_ESHAPE;                 // nor K16 (kernels_dpas.cpp:956-959)
        groups += w->M / 16;
    }
    if (!a || !a->q || !a->scale || a->K != ws[0]->K) return KXW4_EPREP;
    const int rc = check_act(a, ws[0]->K, ws[0]->scale_enc);
    if (rc) return rc == KXW4_ESHAPE ? KXW4_EPREP : rc;
    if (a->T > kDecodeMaxT || (y_dtype != KXW4_F32 && y_dtype != KXW4_BF16)) return KXW4_ESHAPE;
    const int S = kxw4_gemv_splits(groups);
    if (S > 16) return KXW4_ESPLIT;
    return decode_uniform(ws, ys, count, a, y_dtype, nullptr, S, kVarFanout, as_stream(stream));
}

int kxw4_gemm(const kxw4_weight_t *w, const kxw4_act_t *a, void *y, int y_dtype,
              const float *residual, const int *offsets, int segments, int forced_splits,
              void *stream) {
    const kxw4_weight_t *ws[1] = {w};
    void *ys[1] = {y};
    if (!w) return KXW4_EARG;
    return gemm_common(ws, ys, 1, a, y_dtype, residual, offsets, segments, forced_splits, nullptr,
                       as_stream(stream));
}

int kxw4_gemm_fanout(const kxw4_weight_t *const *ws, void *const *ys, int count,
                     const kxw4_act_t *a, int y_dtype, const int *offsets, int segments,
                     int forced_splits, void *stream) {
    return gemm_common(ws, ys, count, a, y_dtype, nullptr, offsets, segments, forced_splits,
                       nullptr, as_stream(stream));
}

// x_gemm_w4a4's checks (kernels_dpas.cpp:1503-1504): -1 for a weight that is
// not the K64 tier with FP16|zp scales, -2 for missing operands or shapes.
int kxw4_gemm_w4a4(const kxw4_weight_t *w, const uint8_t *q4, const float *scale, const int32_t *sum,
                   int T, void *y, int y_dtype, const float *residual, void *stream) {
    if (!w || !w->codes || !w->scales || w->group != 64 || w->scale_enc != KXW4_SCALE_FP16_ZP4)
        return KXW4_EARG;
    if (!valid_shape(w->M, w->K, w->group)) return KXW4_ESHAPE;
    if (!q4 || !scale || !sum || !y || T <= 0) return KXW4_ESHAPE;
    if (y_dtype != KXW4_F32 && y_dtype != KXW4_BF16) return KXW4_ESHAPE;
    // 32-bit per-lane offsets inside the kernel
    if ((long long)T * 64 >= (1ll << 31) || (long long)w->M * w->K / 2 >= (1ll << 31) ||
        (long long)(w->K / 64) * T >= (1ll << 31))
        return KXW4_ESHAPE;
    W4a4Args args{};
    args.q4 = q4;
    args.as4 = scale;
    args.codes = w->codes;
    args.scales = w->scales;
    args.y = y;
    args.residual = residual;
    args.M = w->M;
    args.K = w->K;
    args.T = T;
    args.y_bf16 = y_dtype == KXW4_BF16 ? 1 : 0;
    return launch_w4a4(args, as_stream(stream));
}

int kxw4_partials(const kxw4_weight_t *w, const kxw4_act_t *a, int32_t *P, void *stream) {
    if (!w || !P) return KXW4_EARG;
    const kxw4_weight_t *ws[1] = {w};
    void *ys[1] = {nullptr};
    return gemm_common(ws, ys, 1, a, KXW4_F32, nullptr, nullptr, 0, 0, P, as_stream(stream));
}

}  // extern "C"
