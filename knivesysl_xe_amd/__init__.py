"""knivesysl_xe_amd — MI355X-native W4A8 projection path of knivesysl-xe.

libkxw4.so holds the gfx950 HIP kernels behind the C ABI in include/kxw4.h;
`ops` is the torch-tensor front end, `workloads` the BASELINE configurations
with their seeded synthetic inputs.
"""
from . import _lib  # noqa: F401
from ._lib import BF16, F32, SCALE_FP16, SCALE_FP16_ZP4, KxError  # noqa: F401

__all__ = ["ops", "workloads", "build"]
