"""The reference-signature C++ shims (include/kxw4_compat.hpp).

CPU: libkxw4.so exports every x_* function the header declares, with the
reference's parameter types (xpu/src/tq_common.hpp:385-461).
GPU: tests/compat/compat_check (built by __graft_entry__.build()) drives the
shims the way the reference's callers do and compares every output with the
CPU oracle bit for bit.
"""
import os
import re
import shutil
import subprocess

import pytest

from knivesysl_xe_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "compat", "_build", "compat_check")


def declared_shims():
    text = open(os.path.join(ROOT, "include", "kxw4_compat.hpp")).read()
    text = re.sub(r"//.*", "", text)
    return sorted(set(re.findall(r"\b(x_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.skipif(shutil.which("nm") is None, reason="nm not available")
def test_library_exports_reference_signatures():
    _lib.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", _lib.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = {m.group(1): m.group(2) for m in
                re.finditer(r" T (x_[a-z0-9_]+)\((.*)\)$", out, flags=re.M)}
    names = declared_shims()
    assert len(names) >= 14
    for n in names:
        assert n in exported, n
    # spot-check parameter types against the reference's declarations
    assert exported["x_gemm_w4a8"] == ("tq_qmma_weight_t const*, signed char const*, float const*, "
                                       "int const*, float*, int, int const*, int")
    assert exported["x_gemv_w4a8_fanout"] == "tq_qmma_weight_t const* const*, float* const*, int"
    assert exported["x_rmsnorm_quant"] == "float*, float const*, unsigned short const*, int, float"
    assert exported["x_gemm_w4a4"] == ("tq_qmma_weight_t const*, unsigned char const*, float const*, "
                                       "int const*, float*, int")
    assert exported["x_quantize_act_chunk_s4"] == "float const*, int, int, unsigned char*, float*, int*"
    assert exported["x_gemm_w8a8"] == "tq_qmma_weight_t const*, signed char const*, float const*, float*, int"
    assert exported["x_rmsnorm_chunk"] == "float*, float const*, unsigned short const*, int, int, float"
    assert "kxw4_compat_set_stream" in out


@pytest.mark.gpu
def test_reference_signature_shims_match_oracle():
    assert os.path.exists(EXE), "tests/compat/_build/compat_check missing: run __graft_entry__.build()"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout
