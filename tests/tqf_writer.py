"""Writes synthetic TQF1 model containers in the layout the reference's
loader reads (xpu/src/tqf_loader.cpp:393-626; QMMA records 186-255): test
fixtures for the ingest path, seeded and small."""
import struct

import numpy as np

FLAG_FP8_QMMA, FLAG_BLOCK_SCALED, FLAG_E2M3, FLAG_HAS_MTP = 1 << 0, 1 << 5, 1 << 8, 1 << 10
FULL, LINEAR = 2, 1


def spec(H=128, I=256, V=64, nh=2, nkv=1, hd=64, lvh=16, lvd=64, lkh=1, lkd=64, lconv=4,
         types=(FULL, LINEAR), tied=False, mtp=True, k32_scales=False):
    return dict(H=H, I=I, V=V, nh=nh, nkv=nkv, hd=hd, lvh=lvh, lvd=lvd, lkh=lkh, lkd=lkd,
                lconv=lconv, types=tuple(types), tied=tied, mtp=mtp, k32_scales=k32_scales)


def tensor_list(s):
    """(name, kind, M, K) in file order; kind 'bf16' / 'f32' (M = count) or 'qmma'."""
    H, I, V, hd = s["H"], s["I"], s["V"], s["hd"]
    attn, q, kv = s["nh"] * hd, 2 * s["nh"] * hd, s["nkv"] * hd
    lval, conv = s["lvh"] * s["lvd"], 2 * s["lkh"] * s["lkd"] + s["lvh"] * s["lvd"]
    out = [("embed", "bf16", V * H, 1), ("norm", "bf16", H, 1)]
    if not s["tied"]:
        out.append(("lm_head", "qmma", V, H))
    for i, t in enumerate(s["types"]):
        p = f"layer{i}."
        out += [(p + "input_ln", "bf16", H, 1), (p + "post_ln", "bf16", H, 1),
                (p + "mlp_gate", "qmma", I, H), (p + "mlp_up", "qmma", I, H), (p + "mlp_down", "qmma", H, I)]
        if t == FULL:
            out += [(p + "q_norm", "bf16", hd, 1), (p + "k_norm", "bf16", hd, 1),
                    (p + "q_proj", "qmma", q, H), (p + "k_proj", "qmma", kv, H),
                    (p + "v_proj", "qmma", kv, H), (p + "o_proj", "qmma", H, attn)]
        else:
            out += [(p + "linear_A_log", "f32", s["lvh"], 1), (p + "linear_dt_bias", "bf16", s["lvh"], 1),
                    (p + "linear_norm", "f32", s["lvd"], 1), (p + "linear_conv1d", "bf16", conv * s["lconv"], 1),
                    (p + "linear_in_a", "qmma", s["lvh"], H), (p + "linear_in_b", "qmma", s["lvh"], H),
                    (p + "linear_in_qkv", "qmma", conv, H), (p + "linear_in_z", "qmma", lval, H),
                    (p + "linear_out", "qmma", H, lval)]
    if s["mtp"]:
        out += [("mtp.pre_fc_norm_emb", "bf16", H, 1), ("mtp.pre_fc_norm_hidden", "bf16", H, 1),
                ("mtp.fc", "bf16", H * 2 * H, 1), ("mtp.input_ln", "bf16", H, 1), ("mtp.post_ln", "bf16", H, 1),
                ("mtp.q_norm", "bf16", hd, 1), ("mtp.k_norm", "bf16", hd, 1), ("mtp.q_proj", "bf16", q * H, 1),
                ("mtp.k_proj", "bf16", kv * H, 1), ("mtp.v_proj", "bf16", kv * H, 1),
                ("mtp.o_proj", "bf16", H * attn, 1), ("mtp.mlp_gate", "bf16", I * H, 1),
                ("mtp.mlp_up", "bf16", I * H, 1), ("mtp.mlp_down", "bf16", H * I, 1), ("mtp.norm", "bf16", H, 1)]
    return out


def write(path, s, seed=0, flags=None, header_bytes=None, extra=b""):
    """Returns {name: (scales f32 [rows][cols], payload uint8)} of the QMMA
    records written."""
    rng = np.random.default_rng(seed)
    L = len(s["types"])
    if flags is None:
        flags = FLAG_FP8_QMMA | FLAG_BLOCK_SCALED | FLAG_E2M3 | (FLAG_HAS_MTP if s["mtp"] else 0)
    u = [flags, 7, 2, s["H"], s["I"], L, s["V"], s["nh"], s["nkv"], s["hd"],
         s["lkh"], s["lkd"], s["lvh"], s["lvd"], s["lconv"], 4096]
    tail = [0, 0, 0, 0, int(s["tied"]), 1, 0, int(s["mtp"])]
    hb = 4 + 4 + 64 + 12 + 32 + L if header_bytes is None else header_bytes
    qmma = {}
    with open(path, "wb") as f:
        f.write(b"TQF1")
        f.write(struct.pack("<I", hb))
        f.write(struct.pack("<16I", *u))
        f.write(struct.pack("<3f", 1e-6, 1e7, 0.25))
        f.write(struct.pack("<8I", *tail))
        f.write(bytes(s["types"]))
        for name, kind, M, K in tensor_list(s):
            if kind == "bf16":
                f.write(rng.integers(0, 1 << 16, M, dtype=np.uint16).tobytes())
            elif kind == "f32":
                f.write(rng.standard_normal(M).astype(np.float32).tobytes())
            else:
                rows = (M + 127) // 128
                cols = (K + 31) // 32 if s["k32_scales"] else (K + 127) // 128
                sc = rng.uniform(0.001, 0.05, (rows, cols)).astype(np.float32)
                payload = rng.integers(0, 256, (M // 16) * (K // 32) * 384, dtype=np.uint8)
                f.write(struct.pack("<II", rows, cols))
                f.write(sc.tobytes())
                f.write(payload.tobytes())
                qmma[name] = (sc, payload)
        f.write(extra)
    return qmma
