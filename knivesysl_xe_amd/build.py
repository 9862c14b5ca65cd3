"""Compile libkxw4.so for gfx950 (hipcc through knivesysl_xe_amd/csrc/Makefile)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(force: bool = True, jobs: int = 8) -> str:
    """Build the library in-tree; `force` recompiles every source."""
    cmd = ["make", "-C", CSRC, f"-j{jobs}"]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)
    return os.path.join(HERE, "libkxw4.so")


if __name__ == "__main__":
    print(build())
