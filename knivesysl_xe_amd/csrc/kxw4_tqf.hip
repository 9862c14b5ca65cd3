// kxw4_tqf.hip — TQF1 ingest (host code): the reference's model container
// (xpu/src/tqf_loader.cpp:393-626) walked tensor by tensor without reading
// payloads, and its block-scaled dense-E2M3 QMMA tensors (186-255) repacked
// straight into this library's W4 / W8 layouts.
//
// File layout, as tqf_loader.cpp reads it: "TQF1", uint32 header_bytes,
// uint32 u[16] (flags, family, non-quant dtype, H, I, L, V, nh, nkv, hd, the
// five linear-attention dimensions, max positions), float fl[3], uint32
// tail[8] (tail[4] = tied embeddings, tail[7] = has MTP), uint8 layer_types[L];
// then embed (BF16 [V][H]), norm (BF16 [H]), lm_head (QMMA [V][H], absent when
// tied), per layer input_ln and post_ln (BF16 [H]), mlp_gate / mlp_up
// (QMMA [I][H]), mlp_down (QMMA [H][I]), then for a full-attention layer
// q_norm / k_norm (BF16 [hd]) and q / k / v / o projections, for a
// linear-attention layer A_log (F32), dt_bias (BF16), norm (F32), conv1d
// (BF16) and the in_a / in_b / in_qkv / in_z / out projections; then the MTP
// section (15 BF16 tensors) when flags carry HAS_MTP. A QMMA tensor is
// uint32 scale_rows, uint32 scale_cols, FP32 block scales [rows][cols] and
// the fragment payload [M/16][K/32][384 B].
#include "../../include/kxw4.h"
#include "kxw4_internal.hpp"

#include <climits>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

namespace {

constexpr uint32_t kFlagFp8Qmma = 1u << 0;
constexpr uint32_t kFlagBlockScaled = 1u << 5;
constexpr uint32_t kFlagRowMajor = 1u << 6;
constexpr uint32_t kFlagWordMajor = 1u << 7;
constexpr uint32_t kFlagE2M3 = 1u << 8;
constexpr uint32_t kFlagSparse24 = 1u << 9;
constexpr uint32_t kFlagHasMtp = 1u << 10;
constexpr uint32_t kDtypeBf16 = 2;
constexpr int kMaxLayers = 64;
constexpr int kLayerLinear = 1, kLayerFull = 2;
constexpr size_t kE2M3TileBytes = 384;

struct Walker {
    FILE *f = nullptr;
    uint64_t pos = 0, size = 0;
    std::vector<kxw4_tqf_tensor_t> out;
    bool ok = true;

    void add(const std::string &name, int kind, int M, int K, uint64_t bytes, int sr = 0, int sc = 0) {
        kxw4_tqf_tensor_t t;
        std::memset(&t, 0, sizeof(t));
        std::snprintf(t.name, sizeof(t.name), "%s", name.c_str());
        t.kind = kind;
        t.M = M;
        t.K = K;
        t.scale_rows = sr;
        t.scale_cols = sc;
        t.offset = pos;
        t.bytes = bytes;
        out.push_back(t);
    }
    // a plain tensor of `count` elements of `esize` bytes
    void vec(const std::string &name, int kind, uint64_t count, uint64_t esize) {
        if (!ok) return;
        const uint64_t bytes = count * esize;
        if (count && bytes / count != esize) { ok = false; return; }
        if (pos + bytes > size) { ok = false; return; }
        add(name, kind, (int)(count <= INT_MAX ? count : 0), 1, bytes);
        pos += bytes;
    }
    // a QMMA record (tqf_loader.cpp:186-255)
    void qmma(const std::string &name, int M, int K) {
        if (!ok) return;
        if (M <= 0 || K <= 0 || M % 16 || K % 32) { ok = false; return; }
        uint32_t sr = 0, sc = 0;
        if (pos + 8 > size || std::fseek(f, (long)pos, SEEK_SET) != 0 || std::fread(&sr, 4, 1, f) != 1 ||
            std::fread(&sc, 4, 1, f) != 1) {
            ok = false;
            return;
        }
        if (sr != (uint32_t)((M + 127) / 128) || (sc != (uint32_t)((K + 127) / 128) && sc != (uint32_t)((K + 31) / 32))) {
            ok = false;
            return;
        }
        const uint64_t bytes = 8 + (uint64_t)sr * sc * 4 + (uint64_t)(M / 16) * (K / 32) * kE2M3TileBytes;
        if (pos + bytes > size) { ok = false; return; }
        add(name, KXW4_TQF_QMMA, M, K, bytes, (int)sr, (int)sc);
        pos += bytes;
    }
};

}  // namespace

struct kxw4_tqf {
    std::string path;
    uint32_t u[16];
    float fl[3];
    uint32_t tail[8];
    std::vector<kxw4_tqf_tensor_t> tensors;
};

extern "C" {

int kxw4_tqf_open(const char *path, kxw4_tqf_t **out) {
    if (!path || !out) return KXW4_EARG;
    *out = nullptr;
    FILE *f = std::fopen(path, "rb");
    if (!f) return KXW4_EARG;
    auto fail = [&](int rc) {
        std::fclose(f);
        return rc;
    };
    char magic[4];
    uint32_t header_bytes = 0, u[16], tail[8];
    float fl[3];
    if (std::fread(magic, 1, 4, f) != 4 || std::memcmp(magic, "TQF1", 4) != 0) return fail(KXW4_EARG);
    if (std::fread(&header_bytes, 4, 1, f) != 1 || std::fread(u, 4, 16, f) != 16 || std::fread(fl, 4, 3, f) != 3 ||
        std::fread(tail, 4, 8, f) != 8)
        return fail(KXW4_EARG);
    // validate_header_fields (tqf_loader.cpp:276-315)
    for (int i = 3; i < 16; ++i)
        if (u[i] > (uint32_t)INT_MAX) return fail(KXW4_ESHAPE);
    const int H = (int)u[3], I = (int)u[4], L = (int)u[5], V = (int)u[6], nh = (int)u[7], nkv = (int)u[8],
              hd = (int)u[9];
    const int lkh = (int)u[10], lkd = (int)u[11], lvh = (int)u[12], lvd = (int)u[13], lconv = (int)u[14];
    if (H <= 0 || I <= 0 || L <= 0 || L > kMaxLayers || V <= 0 || nh <= 0 || nkv <= 0 || hd <= 0)
        return fail(KXW4_ESHAPE);
    const uint32_t flags = u[0];
    if (u[2] != kDtypeBf16) return fail(KXW4_ETIER);
    const uint32_t need = kFlagFp8Qmma | kFlagBlockScaled | kFlagE2M3;
    if ((flags & need) != need || (flags & (kFlagRowMajor | kFlagWordMajor | kFlagSparse24))) return fail(KXW4_ETIER);
    if (header_bytes != 4u + 4u + 16u * 4u + 3u * 4u + 8u * 4u + (uint32_t)L) return fail(KXW4_ESHAPE);
    uint8_t types[kMaxLayers];
    if (std::fread(types, 1, (size_t)L, f) != (size_t)L) return fail(KXW4_EARG);
    bool linear = false;
    for (int i = 0; i < L; ++i) {
        if (types[i] == kLayerLinear) linear = true;
        else if (types[i] != kLayerFull) return fail(KXW4_ESHAPE);
    }
    if (linear && (lkh <= 0 || lkd <= 0 || lvh <= 0 || lvd <= 0 || lconv <= 0)) return fail(KXW4_ESHAPE);
    const long long lkey = (long long)lkh * lkd, lval = (long long)lvh * lvd, conv = 2 * lkey + lval;
    const long long attn = (long long)nh * hd, qrows = 2 * attn, kvrows = (long long)nkv * hd;
    if (conv > INT_MAX || qrows > INT_MAX || kvrows > INT_MAX) return fail(KXW4_ESHAPE);

    Walker w;
    w.f = f;
    if (std::fseek(f, 0, SEEK_END) != 0) return fail(KXW4_EARG);
    const long end = std::ftell(f);
    if (end < 0) return fail(KXW4_EARG);
    w.size = (uint64_t)end;
    w.pos = 4 + 4 + 64 + 12 + 32 + (uint64_t)L;
    w.vec("embed", KXW4_TQF_BF16, (uint64_t)V * H, 2);
    w.vec("norm", KXW4_TQF_BF16, (uint64_t)H, 2);
    if (!tail[4]) w.qmma("lm_head", V, H);
    for (int i = 0; i < L && w.ok; ++i) {
        const std::string p = "layer" + std::to_string(i) + ".";
        w.vec(p + "input_ln", KXW4_TQF_BF16, H, 2);
        w.vec(p + "post_ln", KXW4_TQF_BF16, H, 2);
        w.qmma(p + "mlp_gate", I, H);
        w.qmma(p + "mlp_up", I, H);
        w.qmma(p + "mlp_down", H, I);
        if (types[i] == kLayerFull) {
            w.vec(p + "q_norm", KXW4_TQF_BF16, hd, 2);
            w.vec(p + "k_norm", KXW4_TQF_BF16, hd, 2);
            w.qmma(p + "q_proj", (int)qrows, H);
            w.qmma(p + "k_proj", (int)kvrows, H);
            w.qmma(p + "v_proj", (int)kvrows, H);
            w.qmma(p + "o_proj", H, (int)attn);
        } else {
            w.vec(p + "linear_A_log", KXW4_TQF_F32, lvh, 4);
            w.vec(p + "linear_dt_bias", KXW4_TQF_BF16, lvh, 2);
            w.vec(p + "linear_norm", KXW4_TQF_F32, lvd, 4);
            w.vec(p + "linear_conv1d", KXW4_TQF_BF16, (uint64_t)conv * lconv, 2);
            w.qmma(p + "linear_in_a", lvh, H);
            w.qmma(p + "linear_in_b", lvh, H);
            w.qmma(p + "linear_in_qkv", (int)conv, H);
            w.qmma(p + "linear_in_z", (int)lval, H);
            w.qmma(p + "linear_out", H, (int)lval);
        }
    }
    if (flags & kFlagHasMtp) {
        // skip_mtp_section (tqf_loader.cpp:318-389): 15 BF16 tensors
        const uint64_t h = H, in = I, q = qrows, kv = kvrows, at = attn;
        const struct {
            const char *name;
            uint64_t count;
        } mtp[] = {{"mtp.pre_fc_norm_emb", h}, {"mtp.pre_fc_norm_hidden", h}, {"mtp.fc", h * 2 * h},
                   {"mtp.input_ln", h},        {"mtp.post_ln", h},           {"mtp.q_norm", (uint64_t)hd},
                   {"mtp.k_norm", (uint64_t)hd}, {"mtp.q_proj", q * h},       {"mtp.k_proj", kv * h},
                   {"mtp.v_proj", kv * h},     {"mtp.o_proj", h * at},       {"mtp.mlp_gate", in * h},
                   {"mtp.mlp_up", in * h},     {"mtp.mlp_down", h * in},     {"mtp.norm", h}};
        for (const auto &t : mtp) w.vec(t.name, KXW4_TQF_BF16, t.count, 2);
    }
    // the payload must end exactly at the end of the file (tqf_loader.cpp:603-614)
    if (!w.ok || w.pos != w.size) return fail(KXW4_ESHAPE);
    std::fclose(f);
    kxw4_tqf *t = new (std::nothrow) kxw4_tqf;
    if (!t) return KXW4_EHIP;
    t->path = path;
    std::memcpy(t->u, u, sizeof(u));
    std::memcpy(t->fl, fl, sizeof(fl));
    std::memcpy(t->tail, tail, sizeof(tail));
    t->tensors = std::move(w.out);
    *out = t;
    return KXW4_OK;
}

void kxw4_tqf_close(kxw4_tqf_t *t) { delete t; }

int kxw4_tqf_count(const kxw4_tqf_t *t) { return t ? (int)t->tensors.size() : KXW4_EARG; }

int kxw4_tqf_header(const kxw4_tqf_t *t, uint32_t *u16, float *f3, uint32_t *tail8) {
    if (!t) return KXW4_EARG;
    if (u16) std::memcpy(u16, t->u, sizeof(t->u));
    if (f3) std::memcpy(f3, t->fl, sizeof(t->fl));
    if (tail8) std::memcpy(tail8, t->tail, sizeof(t->tail));
    return KXW4_OK;
}

int kxw4_tqf_tensor(const kxw4_tqf_t *t, int index, kxw4_tqf_tensor_t *out) {
    if (!t || !out || index < 0 || index >= (int)t->tensors.size()) return KXW4_EARG;
    *out = t->tensors[(size_t)index];
    return KXW4_OK;
}

int kxw4_tqf_find(const kxw4_tqf_t *t, const char *name) {
    if (!t || !name) return KXW4_EARG;
    for (size_t i = 0; i < t->tensors.size(); ++i)
        if (std::strcmp(t->tensors[i].name, name) == 0) return (int)i;
    return KXW4_EARG;
}

int kxw4_tqf_load_qmma(const kxw4_tqf_t *t, int index, int mode, uint8_t *out_codes, uint16_t *out_scales,
                       void *stream) {
    if (!t || !out_codes || !out_scales || index < 0 || index >= (int)t->tensors.size()) return KXW4_EARG;
    const kxw4_tqf_tensor_t &d = t->tensors[(size_t)index];
    if (d.kind != KXW4_TQF_QMMA) return KXW4_EARG;
    if (d.M % 16 || d.K % 128) return KXW4_ESHAPE;
    if (mode != 0 && mode != 1 && mode != 2 && mode != 8) return KXW4_ESHAPE;
    const size_t sbytes = (size_t)d.scale_rows * d.scale_cols * 4;
    const size_t pbytes = (size_t)(d.M / 16) * (d.K / 32) * kE2M3TileBytes;
    // staging: pinned host buffer, device copies of the record, then the
    // repack kernel on `stream`
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t *host = nullptr, *dev = nullptr;
    if (hipHostMalloc((void **)&host, sbytes + pbytes) != hipSuccess) return KXW4_EHIP;
    int rc = KXW4_OK;
    FILE *f = std::fopen(t->path.c_str(), "rb");
    if (!f || std::fseek(f, (long)(d.offset + 8), SEEK_SET) != 0 || std::fread(host, 1, sbytes + pbytes, f) != sbytes + pbytes)
        rc = KXW4_EARG;
    if (f) std::fclose(f);
    if (rc == KXW4_OK && hipMalloc((void **)&dev, sbytes + pbytes) != hipSuccess) rc = KXW4_EHIP;
    if (rc == KXW4_OK && hipMemcpyAsync(dev, host, sbytes + pbytes, hipMemcpyHostToDevice, st) != hipSuccess)
        rc = KXW4_EHIP;
    if (rc == KXW4_OK) {
        const float *bs = reinterpret_cast<const float *>(dev);
        const uint8_t *payload = dev + sbytes;
        rc = mode == 8 ? kxw4_repack_e2m3_s8(payload, bs, d.scale_cols, d.M, d.K, out_codes, out_scales, stream)
                       : kxw4_repack_e2m3(payload, bs, d.scale_cols, d.M, d.K, mode, out_codes, out_scales, stream);
    }
    if (dev && hipStreamSynchronize(st) != hipSuccess && rc == KXW4_OK) rc = KXW4_EHIP;
    if (dev) (void)hipFree(dev);
    (void)hipHostFree(host);
    return rc;
}

}  // extern "C"
