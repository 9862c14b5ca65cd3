"""The BASELINE.json configurations and their seeded synthetic inputs.

Names: BASELINE's M is the token count (the reference's T) and N the output
rows (the reference's M). Draw order per config, numpy PCG64 seeded with
`seed`: for each weight in order, int4 codes uniform in [-8, 7] ([N][K] int8),
then FP16 scales |N(0,1)| * 0.02 ([N][K/G]); then the activation: N(0,1)
float32 -> BF16 (round to nearest even), or for the "silu" activation g then u
(both N(0,1) float32) and x = bf16(silu(g) * u) computed in float32.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np


@dataclass(frozen=True)
class Config:
    name: str
    K: int
    rows: List[int]            # output rows of each weight (gate, up, ...)
    group: int
    tokens: int                # BASELINE "M"
    act: str = "normal"        # "normal" | "silu"
    out_bf16: bool = False
    kind: str = "gemm"         # "gemv" (x_gemv_w4a8 arithmetic) | "gemm"
    segments: Optional[List[int]] = None   # packed prompt lengths (sum = tokens)
    bound: str = "hbm"         # roofline that bounds the kernel
    note: str = ""

    @property
    def offsets(self):
        if not self.segments:
            return None
        return [0] + list(np.cumsum(self.segments).tolist())

    def algorithmic_bytes(self) -> int:
        """codes + FP16 scales + activation input + output. Decode (GEMV) rows
        count the BF16 activation, prefill (GEMM) rows the int8 activation."""
        N = sum(self.rows)
        codes = N * self.K // 2
        scales = N * (self.K // self.group) * 2
        act = self.tokens * self.K * (2 if self.bound == "hbm" else 1)
        out = self.tokens * N * (2 if self.out_bf16 else 4)
        return codes + scales + act + out

    def ops(self) -> int:
        return 2 * self.tokens * sum(self.rows) * self.K


CONFIGS = {
    "cfg0": Config("cfg0", 4096, [4096], 128, 1, kind="gemv",
                   note="single W4A8 GEMV, M=1, K=N=4096, G=128, FP32 out"),
    "cfg1": Config("cfg1", 5120, [17408, 17408], 128, 8, out_bf16=True,
                   note="decode MLP gate+up, M=8, K=5120, N=2x17408, G=128, BF16 out"),
    "cfg2_m1": Config("cfg2_m1", 17408, [5120], 64, 1, act="silu", kind="gemv",
                      note="K64 down projection GEMV, M=1, K=17408, N=5120"),
    "cfg2_m512": Config("cfg2_m512", 17408, [5120], 64, 512, act="silu", bound="mfma",
                        note="K64 down projection GEMM, M=512"),
    "cfg3": Config("cfg3", 5120, [5120], 128, 2048, bound="mfma",
                   note="prefill GEMM M=2048, K=N=5120, G=128"),
    "cfg4": Config("cfg4", 5120, [17408, 17408], 128, 3965, bound="mfma",
                   segments=[17, 64, 300, 512, 1024, 2048],
                   note="packed prefill, 6 segments, K=5120, N=2x17408"),
}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Reference RNE conversion (kernels_core.cpp:21-24)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclass
class Inputs:
    codes: List[np.ndarray] = field(default_factory=list)    # int8 [N][K]
    scales: List[np.ndarray] = field(default_factory=list)   # uint16 FP16 bits [N][K/G]
    x_bf16: Optional[np.ndarray] = None                      # uint16 [T][K]


def generate(cfg: Config, seed: int = 0, tokens: Optional[int] = None) -> Inputs:
    rng = np.random.default_rng(seed)
    out = Inputs()
    for N in cfg.rows:
        out.codes.append(rng.integers(-8, 8, size=(N, cfg.K), dtype=np.int8))
        s = np.abs(rng.standard_normal((N, cfg.K // cfg.group), dtype=np.float32)) * np.float32(0.02)
        out.scales.append(s.astype(np.float16).view(np.uint16))
    T = cfg.tokens if tokens is None else tokens
    if cfg.act == "silu":
        g = rng.standard_normal((T, cfg.K), dtype=np.float32)
        u = rng.standard_normal((T, cfg.K), dtype=np.float32)
        x = (g / (np.float32(1) + np.exp(-g))) * u
    else:
        x = rng.standard_normal((T, cfg.K), dtype=np.float32)
    out.x_bf16 = f32_to_bf16_bits(x.astype(np.float32))
    return out
