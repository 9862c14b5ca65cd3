"""TQF1 ingest (kxw4_tqf_*, tqf_loader.cpp:393-626): the tensor walk and the
reference's header checks on synthetic containers, on the CPU; the repack of
QMMA records into the W4 / W8 layouts against the oracle, on the GPU."""
import ctypes as C
import os

import numpy as np
import pytest

from knivesysl_xe_amd import _lib
from tests import tqf_writer as W


def open_rc(path):
    h = C.c_void_p()
    rc = _lib.lib().kxw4_tqf_open(str(path).encode(), C.byref(h))
    if rc == 0:
        _lib.lib().kxw4_tqf_close(h)
    return rc


def table(path):
    L = _lib.lib()
    h = C.c_void_p()
    assert L.kxw4_tqf_open(str(path).encode(), C.byref(h)) == 0
    out = []
    for i in range(L.kxw4_tqf_count(h)):
        d = _lib.TqfTensor()
        assert L.kxw4_tqf_tensor(h, i, C.byref(d)) == 0
        out.append((d.name.decode(), d.kind, d.M, d.K, d.scale_rows, d.scale_cols, d.offset, d.bytes))
    assert L.kxw4_tqf_find(h, b"layer1.linear_out") >= 0 and L.kxw4_tqf_find(h, b"nope") == -1
    L.kxw4_tqf_close(h)
    return out


@pytest.mark.parametrize("tied,mtp,k32", [(False, True, False), (True, False, True)])
def test_walk_matches_the_written_sequence(tmp_path, tied, mtp, k32):
    s = W.spec(tied=tied, mtp=mtp, k32_scales=k32)
    path = tmp_path / "m.tqf"
    W.write(path, s)
    got = table(path)
    want = W.tensor_list(s)
    assert [g[0] for g in got] == [w[0] for w in want]
    kinds = {"bf16": 0, "f32": 1, "qmma": 2}
    pos = 4 + 4 + 64 + 12 + 32 + len(s["types"])
    for g, (name, kind, M, K) in zip(got, want):
        assert g[1] == kinds[kind] and g[6] == pos, name
        if kind == "qmma":
            rows, cols = (M + 127) // 128, ((K + 31) // 32 if k32 else (K + 127) // 128)
            assert (g[2], g[3], g[4], g[5]) == (M, K, rows, cols)
            assert g[7] == 8 + rows * cols * 4 + (M // 16) * (K // 32) * 384
        else:
            assert g[2] == M and g[7] == M * (2 if kind == "bf16" else 4)
        pos += g[7]
    assert pos == os.path.getsize(path)


def test_header_checks_keep_the_reference_rules(tmp_path):
    s = W.spec()
    p = tmp_path / "m.tqf"
    W.write(p, s)
    assert open_rc(p) == 0
    data = p.read_bytes()
    (tmp_path / "magic.tqf").write_bytes(b"TQF2" + data[4:])
    assert open_rc(tmp_path / "magic.tqf") == _lib.EARG
    (tmp_path / "short.tqf").write_bytes(data[:-1])
    assert open_rc(tmp_path / "short.tqf") == _lib.ESHAPE        # payload must end at EOF
    W.write(tmp_path / "long.tqf", s, extra=b"\0")
    assert open_rc(tmp_path / "long.tqf") == _lib.ESHAPE
    W.write(tmp_path / "hb.tqf", s, header_bytes=123)
    assert open_rc(tmp_path / "hb.tqf") == _lib.ESHAPE
    W.write(tmp_path / "flags.tqf", s, flags=W.FLAG_FP8_QMMA | W.FLAG_BLOCK_SCALED)
    assert open_rc(tmp_path / "flags.tqf") == _lib.ETIER         # dense E2M3 payloads only
    W.write(tmp_path / "rm.tqf", s, flags=W.FLAG_FP8_QMMA | W.FLAG_BLOCK_SCALED | W.FLAG_E2M3 | (1 << 6))
    assert open_rc(tmp_path / "rm.tqf") == _lib.ETIER
    assert open_rc(tmp_path / "missing.tqf") == _lib.EARG


@pytest.mark.gpu
@pytest.mark.parametrize("name,mode", [("layer0.mlp_gate", 0), ("layer0.mlp_down", 1), ("lm_head", 2),
                                       ("layer1.linear_in_qkv", 8), ("layer0.q_proj", 0)])
def test_load_qmma_matches_oracle_repack(tmp_path, name, mode):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from knivesysl_xe_amd import ops
    from oracle import oracle as O
    s = W.spec(V=128)
    path = tmp_path / "m.tqf"
    recs = W.write(path, s, seed=3)
    sc, payload = recs[name]
    with ops.TqfFile(path) as f:
        t = [d for d in f.tensors() if d["name"] == name][0]
        M, K = t["M"], t["K"]
        if mode == 8:
            w = f.load_w8(name)
            want_c, want_s = O.repack_e2m3_s8(payload, sc.reshape(-1), t["scale_cols"], M, K)
        else:
            w = f.load_w4(name, mode)
            want_c, want_s = O.repack_e2m3(payload, sc.reshape(-1), t["scale_cols"], M, K, mode)
    c, s2 = w.unpack()
    assert np.array_equal(c.cpu().numpy(), want_c)
    assert np.array_equal(s2.cpu().numpy().view(np.uint16), want_s)
