// compat_check.cpp — the reference-signature shims (include/kxw4_compat.hpp)
// against the CPU oracle, bit for bit. Written the way a caller of the
// reference's projection interface (xpu/src/tq_common.hpp:385-461) is: a
// tq_qmma_weight_t holding a dense-E2M3 payload, x_w4_repack_weight_mode,
// prepared single-token activations, fan-out, chunk quantization and the
// packed GEMM. Prints one line per check and exits non-zero on a mismatch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/kxw4_compat.hpp"
#include "../../oracle/w4a8_oracle.h"

static int g_fail = 0, g_pass = 0;

#define HIPCHECK(x)                                                               \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(2);                                                         \
        }                                                                         \
    } while (0)

template <class T>
static T *dev_copy(const std::vector<T> &h) {
    T *d = nullptr;
    HIPCHECK(hipMalloc(&d, h.size() * sizeof(T) + 16));
    HIPCHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <class T>
static std::vector<T> host_copy(const T *d, size_t n) {
    std::vector<T> h(n);
    HIPCHECK(hipDeviceSynchronize());
    HIPCHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

static void check(bool ok, const char *what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
    if (ok) ++g_pass;
    else ++g_fail;
}

template <class T>
static bool same_bits(const std::vector<T> &a, const std::vector<T> &b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(T)) == 0;
}

struct Source {
    int M, K, mode;
    std::vector<uint8_t> payload;
    std::vector<float> bs;
    int scale_cols;
    std::vector<int8_t> codes;      // oracle repack
    std::vector<uint16_t> scales;
};

static Source make_source(std::mt19937 &rng, int M, int K, int mode) {
    Source s;
    s.M = M;
    s.K = K;
    s.mode = mode;
    const int Kt = K / 32;
    s.payload.resize((size_t)(M / 16) * Kt * 384);
    for (auto &b : s.payload) b = (uint8_t)(rng() & 0xFF);
    s.scale_cols = Kt / 4;
    s.bs.resize((size_t)((M + 127) / 128) * s.scale_cols);
    std::uniform_real_distribution<float> u(0.001f, 0.05f);
    for (auto &v : s.bs) v = u(rng);
    const int group = mode == 2 ? 64 : mode == 1 ? 16 : 32;
    s.codes.resize((size_t)M * K);
    s.scales.resize((size_t)M * (K / group));
    // contract = 1: the device fit contracts its multiply-adds as icpx would
    if (orc_repack_e2m3(s.payload.data(), s.bs.data(), s.scale_cols, M, K, mode, 1, s.codes.data(),
                        s.scales.data()) != 0) {
        std::printf("oracle repack failed\n");
        std::exit(2);
    }
    return s;
}

static tq_qmma_weight_t make_weight(const Source &s) {
    tq_qmma_weight_t w;
    std::memset(&w, 0, sizeof(w));
    w.M = s.M;
    w.K = s.K;
    w.Mt = s.M / 16;
    w.Kt = s.K / 32;
    w.d_A = dev_copy(s.payload);
    w.d_block_scale_inv = dev_copy(s.bs);
    w.block_scaled = 1;
    w.e2m3 = 1;
    w.scale_rows = (s.M + 127) / 128;
    w.scale_cols = s.scale_cols;
    return w;
}

static orc_weight_t oracle_weight(const Source &s) {
    orc_weight_t o;
    o.M = s.M;
    o.K = s.K;
    o.group = s.mode == 2 ? 64 : s.mode == 1 ? 16 : 32;
    o.scale_enc = ORC_SCALE_FP16_ZP4;
    o.codes = s.codes.data();
    o.scales = s.scales.data();
    return o;
}

// oracle projection of x[T][K] (fp32) through reference-mode quantization
static std::vector<float> oracle_project(const Source &s, const std::vector<float> &x, int T,
                                         int variant, const std::vector<int> &splits,
                                         const float *residual) {
    std::vector<int8_t> q((size_t)T * s.K);
    std::vector<float> sc((size_t)T * (s.K / 32));
    std::vector<int32_t> sm((size_t)T * (s.K / 32));
    orc_quantize_act(x.data(), T, s.K, 32, q.data(), sc.data(), sm.data());
    orc_act_t a{T, s.K, 32, q.data(), sc.data(), sm.data()};
    orc_weight_t w = oracle_weight(s);
    std::vector<float> y((size_t)T * s.M, 0.0f);
    // contract = 1: one fused multiply-add per chain step, as the kernels run it
    orc_project(&w, &a, variant, splits.data(), 1, residual, 0, y.data(), 0, s.M);
    return y;
}

int main() {
    std::mt19937 rng(20261201);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    orc_set_num_threads(8);

    // ---- repack: K32 (mode 0) and K64 (mode 2) -----------------------------
    Source s32 = make_source(rng, 1024, 2048, 0);
    Source s64 = make_source(rng, 512, 2048, 2);
    Source s64b = make_source(rng, 256, 2048, 2);
    tq_qmma_weight_t w32 = make_weight(s32), w64 = make_weight(s64), w64b = make_weight(s64b);
    check(x_w4_repack_weight(&w32) == 0 && w32.s4_ready && !w32.s4_k64 && !w32.d_A, "x_w4_repack_weight K32");
    check(x_w4_repack_weight_mode(&w64, 2) == 0 && w64.s4_k64, "x_w4_repack_weight_mode K64");
    check(x_w4_repack_weight_mode(&w64b, 2) == 0, "x_w4_repack_weight_mode K64 (second weight)");
    for (const auto *p : {&s32, &s64}) {
        const tq_qmma_weight_t &w = p == &s32 ? w32 : w64;
        kxw4_weight_t d{w.M, w.K, p->mode == 2 ? 64 : 32, KXW4_SCALE_FP16_ZP4, w.d_s4, w.d_s4_scale};
        int8_t *dc;
        uint16_t *ds;
        HIPCHECK(hipMalloc(&dc, (size_t)w.M * w.K));
        HIPCHECK(hipMalloc(&ds, p->scales.size() * 2));
        check(kxw4_unpack_weight(&d, dc, ds, nullptr) == 0, "unpack repacked weight");
        check(same_bits(host_copy(dc, (size_t)w.M * w.K), p->codes) &&
                  same_bits(host_copy(ds, p->scales.size()), p->scales),
              p->mode == 2 ? "repacked codes+scales == oracle (K64)" : "repacked codes+scales == oracle (K32)");
        HIPCHECK(hipFree(dc));
        HIPCHECK(hipFree(ds));
    }

    // ---- single-token GEMV, with and without residual ----------------------
    std::vector<float> x(2048), res(1024);
    for (auto &v : x) v = nd(rng);
    for (auto &v : res) v = nd(rng);
    float *dx = dev_copy(x), *dres = dev_copy(res), *dy;
    HIPCHECK(hipMalloc(&dy, 4096 * sizeof(float) * 64));
    const std::vector<int> sp32(1, orc_gemv_splits(1024 / 16));
    check(x_gemv_w4a8(&w32, dx, dy) == 0, "x_gemv_w4a8 returns 0");
    check(same_bits(host_copy(dy, 1024), oracle_project(s32, x, 1, ORC_VAR_GEMV, sp32, nullptr)),
          "x_gemv_w4a8 == oracle");
    check(x_gemv_w4a8_add(&w32, dx, dres, dy) == 0, "x_gemv_w4a8_add returns 0");
    check(same_bits(host_copy(dy, 1024), oracle_project(s32, x, 1, ORC_VAR_GEMV, sp32, res.data())),
          "x_gemv_w4a8_add == oracle");
    check(x_gemv_qmma_add(&w32, dx, dres, dy) == 0 &&
              same_bits(host_copy(dy, 1024), oracle_project(s32, x, 1, ORC_VAR_GEMV, sp32, res.data())),
          "x_gemv_qmma_add routes to W4A8");

    // ---- fused RMSNorm + quantization, then prepared GEMV -------------------
    std::vector<uint16_t> wn(2048);
    for (auto &v : wn) v = orc_f32_to_bf16(0.1f * nd(rng));
    uint16_t *dwn = dev_copy(wn);
    float *dnorm;
    HIPCHECK(hipMalloc(&dnorm, 2048 * sizeof(float)));
    x_rmsnorm_quant(dnorm, dx, dwn, 2048, 1e-6f);
    std::vector<float> xn(2048);
    orc_rmsnorm(x.data(), wn.data(), 2048, 1e-6f, xn.data());
    check(same_bits(host_copy(dnorm, 2048), xn), "x_rmsnorm_quant hidden == oracle");
    {
        float *dn2;
        HIPCHECK(hipMalloc(&dn2, 2048 * sizeof(float)));
        x_rmsnorm_chunk(dn2, dx, dwn, 2048, 1, 1e-6f);
        check(same_bits(host_copy(dn2, 2048), xn), "x_rmsnorm_chunk == oracle");
        HIPCHECK(hipFree(dn2));
    }
    const std::vector<int> sp64(1, orc_gemv_splits(512 / 16));
    check(x_gemv_w4a8_prepared(&w64, dy) == 0 &&
              same_bits(host_copy(dy, 512), oracle_project(s64, xn, 1, ORC_VAR_GEMV, sp64, nullptr)),
          "x_rmsnorm_quant + x_gemv_w4a8_prepared (K64) == oracle");
    check(x_gemv_qmma_prepared(&w64, dx, dy, dres) == 0 &&
              same_bits(host_copy(dy, 512), oracle_project(s64, xn, 1, ORC_VAR_GEMV, sp64, res.data())),
          "x_gemv_qmma_prepared with residual == oracle");

    // ---- SiLU*up + quantization, then fan-out over two K64 weights ----------
    std::vector<float> g(2048), u(2048), h(2048);
    for (auto &v : g) v = nd(rng);
    for (auto &v : u) v = nd(rng);
    orc_silu_mul(g.data(), u.data(), h.data(), 2048);
    float *dg = dev_copy(g), *du = dev_copy(u), *dh, *dy2;
    HIPCHECK(hipMalloc(&dh, 2048 * sizeof(float)));
    HIPCHECK(hipMalloc(&dy2, 512 * sizeof(float)));
    x_silu_mul_quant(dh, dg, du, 2048);
    // the hidden vector goes through expf, so it matches within 1e-5 rather
    // than bit for bit; the projection is then checked on the GPU's hidden
    const std::vector<float> hg = host_copy(dh, 2048);
    double worst = 0.0;
    for (int i = 0; i < 2048; ++i)
        worst = std::fmax(worst, std::fabs((double)hg[i] - h[i]) / (std::fabs((double)h[i]) + 1e-30));
    check(worst < 1e-5, "x_silu_mul_quant hidden within 1e-5 of oracle");
    h = hg;
    const tq_qmma_weight_t *ws[2] = {&w64, &w64b};
    float *ys[2] = {dy, dy2};
    const std::vector<int> spf(1, orc_gemv_splits((512 + 256) / 16));
    check(x_gemv_w4a8_fanout(ws, ys, 2) == 0, "x_gemv_w4a8_fanout returns 0");
    check(same_bits(host_copy(dy, 512), oracle_project(s64, h, 1, ORC_VAR_FANOUT, spf, nullptr)) &&
              same_bits(host_copy(dy2, 256), oracle_project(s64b, h, 1, ORC_VAR_FANOUT, spf, nullptr)),
          "fan-out outputs == oracle");

    // ---- chunk quantization + packed GEMM ----------------------------------
    const int T = 72;
    std::vector<float> xt((size_t)T * 2048);
    for (auto &v : xt) v = nd(rng);
    float *dxt = dev_copy(xt), *das, *dyt;
    int8_t *daq;
    int32_t *dasum;
    HIPCHECK(hipMalloc(&daq, (size_t)T * 2048));
    HIPCHECK(hipMalloc(&das, (size_t)T * 64 * sizeof(float)));
    HIPCHECK(hipMalloc(&dasum, (size_t)T * 64 * sizeof(int32_t)));
    HIPCHECK(hipMalloc(&dyt, (size_t)T * 1024 * sizeof(float)));
    x_quantize_act_chunk(dxt, 2048, T, daq, das, dasum);
    const int offsets[3] = {0, 8, T};
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, offsets, 2) == 0, "x_gemm_w4a8 (2 segments) returns 0");
    std::vector<int> spt(T);
    orc_segment_splits(offsets, 2, T, 1024, 2048, 0, spt.data());
    check(same_bits(host_copy(dyt, (size_t)T * 1024), oracle_project(s32, xt, T, ORC_VAR_GEMM, spt, nullptr)),
          "x_gemm_w4a8 packed == oracle (per-segment splits)");

    // ---- W4A4: s4 chunk quantization + W4A4 GEMM on the K64 weight ----------
    {
        const int T4 = 40, K = 2048, M = 512;
        uint8_t *daq4;
        float *das4, *dy4;
        int32_t *dsum4;
        HIPCHECK(hipMalloc(&daq4, (size_t)T4 * K / 2));
        HIPCHECK(hipMalloc(&das4, (size_t)T4 * (K / 64) * sizeof(float)));
        HIPCHECK(hipMalloc(&dsum4, (size_t)T4 * (K / 64) * sizeof(int32_t)));
        HIPCHECK(hipMalloc(&dy4, (size_t)T4 * M * sizeof(float)));
        x_quantize_act_chunk_s4(dxt, K, T4, daq4, das4, dsum4);
        std::vector<int8_t> q((size_t)T4 * K);
        std::vector<float> sc((size_t)T4 * (K / 64));
        std::vector<int32_t> sm((size_t)T4 * (K / 64));
        orc_quantize_act_s4(xt.data(), T4, K, q.data(), sc.data(), sm.data());
        // device layout: codes [K/128][T][64 B] tile order, scale/sum [K/64][T]
        const std::vector<uint8_t> hq = host_copy(daq4, (size_t)T4 * K / 2);
        const std::vector<float> hs = host_copy(das4, sc.size());
        const std::vector<int32_t> hsum = host_copy(dsum4, sm.size());
        bool codes_ok = true, ss_ok = true;
        for (int t = 0; t < T4; ++t)
            for (int k = 0; k < K; ++k) {
                const int kb = k / 128, kk = k % 128, i = kk / 32, g = (kk / 8) % 4, b = kk % 8;
                const uint8_t byte = hq[((size_t)kb * T4 + t) * 64 + 16 * g + 4 * i + (b & 3)];
                const int nib = b < 4 ? (byte & 0xF) : (byte >> 4);
                codes_ok &= (nib >= 8 ? nib - 16 : nib) == q[(size_t)t * K + k];
            }
        for (int t = 0; t < T4; ++t)
            for (int u = 0; u < K / 64; ++u) {
                ss_ok &= std::memcmp(&hs[(size_t)u * T4 + t], &sc[(size_t)t * (K / 64) + u], 4) == 0;
                ss_ok &= hsum[(size_t)u * T4 + t] == sm[(size_t)t * (K / 64) + u];
            }
        check(codes_ok, "x_quantize_act_chunk_s4 codes == oracle");
        check(ss_ok, "x_quantize_act_chunk_s4 scales and sums == oracle ([K/64][T])");
        check(x_gemm_w4a4(&w64, daq4, das4, dsum4, dy4, T4) == 0, "x_gemm_w4a4 returns 0");
        orc_act_t a{T4, K, 64, q.data(), sc.data(), sm.data()};
        orc_weight_t ow = oracle_weight(s64);
        std::vector<float> y((size_t)T4 * M, 0.0f);
        const std::vector<int> one(T4, 1);
        orc_project(&ow, &a, ORC_VAR_GEMM, one.data(), 1, nullptr, 0, y.data(), 0, M);
        check(same_bits(host_copy(dy4, (size_t)T4 * M), y), "x_gemm_w4a4 == oracle");
        check(x_gemm_w4a4(&w32, daq4, das4, dsum4, dy4, T4) == -1, "x_gemm_w4a4 on a K32 weight = -1");
        check(x_gemm_w4a4(&w64, daq4, das4, dsum4, dy4, 36) == -2, "x_gemm_w4a4 T % 8 != 0 = -2");
        check(x_gemm_w4a4(&w64, daq4, das4, nullptr, dy4, T4) == -2, "x_gemm_w4a4 without sums = -2");
        HIPCHECK(hipFree(daq4));
        HIPCHECK(hipFree(das4));
        HIPCHECK(hipFree(dsum4));
        HIPCHECK(hipFree(dy4));
    }

    // ---- K16 tier: x_w4_repack_weight_mode(w, 1) and the K16 GEMV ---------
    {
        Source s16 = make_source(rng, 256, 2048, 1);
        tq_qmma_weight_t w16 = make_weight(s16);
        check(x_w4_repack_weight_mode(&w16, 1) == 0 && w16.s4_k16 && !w16.s4_k64, "x_w4_repack_weight_mode K16");
        orc_weight_t o16{256, 2048, 16, ORC_SCALE_FP16_ZP4, s16.codes.data(), s16.scales.data()};
        std::vector<int8_t> q(2048);
        std::vector<float> sc(64);
        std::vector<int32_t> sm(64);
        orc_quantize_act(x.data(), 1, 2048, 32, q.data(), sc.data(), sm.data());
        orc_act_t a{1, 2048, 32, q.data(), sc.data(), sm.data()};
        const std::vector<int> sp(1, orc_gemv_splits(256 / 16));
        std::vector<float> y(256, 0.0f), yr(256, 0.0f);
        orc_project(&o16, &a, ORC_VAR_GEMV, sp.data(), 1, nullptr, 0, y.data(), 0, 256);
        orc_project(&o16, &a, ORC_VAR_GEMV, sp.data(), 1, res.data(), 0, yr.data(), 0, 256);
        check(x_gemv_w4a8(&w16, dx, dy) == 0 && same_bits(host_copy(dy, 256), y), "x_gemv_w4a8 K16 == oracle");
        check(x_gemv_w4a8_add(&w16, dx, dres, dy) == 0 && same_bits(host_copy(dy, 256), yr),
              "x_gemv_w4a8_add K16 == oracle");
        const tq_qmma_weight_t *k16s[2] = {&w16, &w16};
        float *k16y[2] = {dy, dy2};
        check(x_gemv_w4a8_fanout(k16s, k16y, 2) == -2, "K16 fan-out = -2");
        check(x_gemm_w4a8(&w16, daq, das, dasum, dyt, T) == -1, "K16 GEMM = -1");
    }

    // ---- W8A8 tier: x_w8_repack_weight, GEMV (+add, tier routing), GEMM ---
    {
        const int M8 = 512, K8 = 2048;
        Source s8 = make_source(rng, M8, K8, 0);
        tq_qmma_weight_t w8 = make_weight(s8);
        check(x_w8_repack_weight(&w8) == 0 && w8.s8_ready && !w8.d_A && w8.d_s8, "x_w8_repack_weight");
        std::vector<int8_t> c8((size_t)M8 * K8);
        std::vector<uint16_t> sc8((size_t)M8 * (K8 / 32));
        orc_repack_e2m3_s8(s8.payload.data(), s8.bs.data(), s8.scale_cols, M8, K8, 1, c8.data(), sc8.data());
        orc_weight_t o8{M8, K8, 32, ORC_SCALE_S8, c8.data(), sc8.data()};
        auto proj8 = [&](const std::vector<float> &xv, int T, int variant, const std::vector<int> &sp,
                         const float *resid) {
            std::vector<int8_t> q((size_t)T * K8);
            std::vector<float> sc((size_t)T * (K8 / 32));
            std::vector<int32_t> sm((size_t)T * (K8 / 32));
            orc_quantize_act(xv.data(), T, K8, 32, q.data(), sc.data(), sm.data());
            orc_act_t a{T, K8, 32, q.data(), sc.data(), sm.data()};
            std::vector<float> y((size_t)T * M8, 0.0f);
            orc_project(&o8, &a, variant, sp.data(), 1, resid, 0, y.data(), 0, M8);
            return y;
        };
        const std::vector<int> sp8(1, orc_gemv_splits(M8 / 16));
        check(x_gemv_w8a8(&w8, dx, dy) == 0 && same_bits(host_copy(dy, M8), proj8(x, 1, ORC_VAR_GEMV, sp8, nullptr)),
              "x_gemv_w8a8 == oracle");
        check(x_gemv_w8a8_add(&w8, dx, dres, dy) == 0 &&
                  same_bits(host_copy(dy, M8), proj8(x, 1, ORC_VAR_GEMV, sp8, res.data())),
              "x_gemv_w8a8_add == oracle");
        check(x_gemv_qmma_prepared(&w8, dx, dy, dres) == 0 &&
                  same_bits(host_copy(dy, M8), proj8(x, 1, ORC_VAR_GEMV, sp8, res.data())),
              "x_gemv_qmma_prepared routes to W8A8");
        const std::vector<int> one(T, 1);
        check(x_gemm_w8a8(&w8, daq, das, dyt, T) == 0 &&
                  same_bits(host_copy(dyt, (size_t)T * M8), proj8(xt, T, ORC_VAR_GEMM, one, nullptr)),
              "x_gemm_w8a8 (T = 72) == oracle");
        const std::vector<int> one8(8, 1);
        const std::vector<float> x8(xt.begin(), xt.begin() + (size_t)8 * K8);
        check(x_gemm_w8a8(&w8, daq, das, dyt, 8) == 0 &&
                  same_bits(host_copy(dyt, (size_t)8 * M8), proj8(x8, 8, ORC_VAR_GEMM, one8, nullptr)),
              "x_gemm_w8a8 (T = 8, spec wave) == oracle");
        check(x_gemm_w8a8(&w8, daq, das, dyt, 36) == -2, "x_gemm_w8a8 T % 8 != 0 = -2");
        check(x_gemm_w8a8(&w32, daq, das, dyt, 8) == -1, "x_gemm_w8a8 without s8 = -1");
        check(x_gemv_w8a8(&w32, dx, dy) == -1, "x_gemv_w8a8 without s8 = -1");
    }

    // ---- argument checks keep the reference's codes ------------------------
    tq_qmma_weight_t bad;
    std::memset(&bad, 0, sizeof(bad));
    check(x_gemv_w4a8(nullptr, dx, dy) == -1, "x_gemv_w4a8(null) = -1");
    check(x_w4_repack_weight(&bad) == -1, "repack without payload = -1");
    bad = make_weight(s64b);
    bad.M = 100;
    check(x_w4_repack_weight(&bad) == -2, "repack M % 16 != 0 = -2");
    check(x_gemv_qmma_prepared(&bad, dx, dy) == KXW4_ETIER, "no W4 tier = KXW4_ETIER");
    check(x_gemv_w4a8_fanout(ws, ys, 5) == -1, "fan-out count 5 = -1");
    const int bad_off[3] = {0, 80, T};
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, bad_off, 2) == -2, "GEMM offsets past T = -2");
    // x_gemm_w4a8's -2 cases (kernels_dpas.cpp:1338, 1349-1356, 1364)
    check(x_gemm_w4a8(&w32, nullptr, das, dasum, dyt, T, nullptr, 0) == -2, "x_gemm_w4a8 null aq = -2");
    check(x_gemm_w4a8(&w32, daq, nullptr, dasum, dyt, T, nullptr, 0) == -2, "x_gemm_w4a8 null as = -2");
    check(x_gemm_w4a8(&w32, daq, das, nullptr, dyt, T, nullptr, 0) == -2, "x_gemm_w4a8 null asum = -2");
    check(x_gemm_w4a8(&w32, daq, das, dasum, nullptr, T, nullptr, 0) == -2, "x_gemm_w4a8 null y = -2");
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, 0, nullptr, 0) == -2, "x_gemm_w4a8 T = 0 = -2");
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, 36, nullptr, 0) == -2, "x_gemm_w4a8 T % 8 != 0 = -2");
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, nullptr, 1) == -2, "x_gemm_w4a8 segments without offsets = -2");
    const int off_ragged[3] = {0, 12, T};
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, off_ragged, 2) == -2, "x_gemm_w4a8 offset % 8 != 0 = -2");
    const int off_first[3] = {8, 16, T};
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, off_first, 2) == -2, "x_gemm_w4a8 offsets[0] != 0 = -2");
    const int off_empty[3] = {0, 0, T};
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, off_empty, 2) == -2, "x_gemm_w4a8 empty segment = -2");
    check(x_gemm_w4a8(&w32, daq, das, dasum, dyt, T, offsets, 9) == -2, "x_gemm_w4a8 9 segments = -2");
    check(x_gemm_w4a8(nullptr, daq, das, dasum, dyt, T, nullptr, 0) == -1, "x_gemm_w4a8 null weight = -1");

    std::printf("compat: %d passed, %d failed\n", g_pass, g_fail);
    return g_fail ? 1 : 0;
}
