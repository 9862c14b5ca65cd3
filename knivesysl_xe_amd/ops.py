"""Torch-tensor front end of the W4A8 projection library.

The functions mirror the reference's projection interface (xpu/src/
tq_common.hpp:385-461) one for one, with explicit activation buffers instead
of the reference's library-global scratch:

    reference                         here
    x_w4_repack_weight_mode           W4Weight.repack_e2m3
    x_w8_repack_weight                W4Weight.repack_e2m3_s8 (W8A8 tier)
    (load-time integer codes)         W4Weight.from_codes
    reference DPAS layout import      W4Weight.from_reference_layout
    x_quantize_act_s8 / _chunk        quantize_act
    x_silu_mul_quant                  silu_mul_quant
    x_rmsnorm_quant (+ chunk)         rmsnorm_quant
    x_rmsnorm_chunk                   rmsnorm
    x_gemv_w4a8[_add|_prepared]       gemv
    x_gemv_w4a8_fanout                gemv_fanout
    x_gemm_w4a8                       gemm
    (one launch for gate+up)          gemm_fanout
    qwn_load's read_qmma + repack     TqfFile.load_w4 / load_w8 (TQF1 ingest)
    x_quantize_act_chunk_s4           quantize_act_s4
    x_gemm_w4a4                       gemm_w4a4

Torch provides device memory and the current stream only; every kernel is
the HIP code in libkxw4.so, reached through ctypes. Tensors must live on a
GPU; nothing here falls back to the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import BF16, F32, SCALE_FP16, SCALE_FP16_ZP4, SCALE_W8, check, lib


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return C.c_void_p(t.data_ptr())


def _need(t, name: str, dtypes, shape, device) -> torch.Tensor:
    """Validate a caller-supplied buffer before its pointer reaches a kernel:
    a tensor on `device` (the weight's GPU), contiguous, of one of `dtypes` and exactly
    `shape`. The kernels trust these sizes, so a mismatch raises here."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.device != torch.device(device):
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if isinstance(dtypes, torch.dtype):
        dtypes = (dtypes,)
    if t.dtype not in dtypes:
        raise ValueError(f"{name} must be {' or '.join(str(d) for d in dtypes)}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t


_BITS16 = (torch.int16, torch.uint16) if hasattr(torch, "uint16") else (torch.int16,)


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise ValueError(f"unsupported dtype {dt}")


@dataclass
class W4Weight:
    """One packed projection: the W4 fields of tq_qmma_weight_t
    (tq_common.hpp:62-72) in the gfx950 tile layout."""
    M: int
    K: int
    group: int
    scale_enc: int
    codes: torch.Tensor      # uint8 [M*K/2]
    scales: torch.Tensor     # int16 bits [M/16 * K/group * 16]

    def c(self) -> _lib.Weight:
        return _lib.Weight(self.M, self.K, self.group, self.scale_enc,
                           self.codes.data_ptr(), self.scales.data_ptr())

    @classmethod
    def empty(cls, M: int, K: int, group: int, scale_enc: int, device="cuda") -> "W4Weight":
        nbytes = M * K if scale_enc == SCALE_W8 else M * K // 2
        codes = torch.empty(nbytes, dtype=torch.uint8, device=device)
        scales = torch.empty(M * (K // group), dtype=torch.int16, device=device)
        return cls(M, K, group, scale_enc, codes, scales)

    @classmethod
    def from_codes(cls, codes: torch.Tensor, scales: torch.Tensor, group: int,
                   scale_enc: int = SCALE_FP16) -> "W4Weight":
        """codes: int8 [M][K] in [-8, 7]; scales: int16 (FP16 bits) [M][K/group]."""
        M, K = codes.shape
        w = cls.empty(M, K, group, scale_enc, codes.device)
        check("kxw4_pack_weight", lib().kxw4_pack_weight(
            _ptr(codes), _ptr(scales), M, K, group, _ptr(w.codes), _ptr(w.scales), _stream()))
        return w

    @classmethod
    def from_codes_s8(cls, codes: torch.Tensor, scales: torch.Tensor) -> "W4Weight":
        """W8A8 tier: codes int8 [M][K]; scales int16 (FP16 bits) [M][K/32]."""
        M, K = codes.shape
        w = cls.empty(M, K, 32, SCALE_W8, codes.device)
        check("kxw4_pack_weight_s8", lib().kxw4_pack_weight_s8(
            _ptr(codes), _ptr(scales), M, K, _ptr(w.codes), _ptr(w.scales), _stream()))
        return w

    @classmethod
    def repack_e2m3_s8(cls, payload: torch.Tensor, block_scale_inv: torch.Tensor, scale_cols: int,
                       M: int, K: int) -> "W4Weight":
        """x_w8_repack_weight: dense-E2M3 payload -> the W8A8 tier."""
        w = cls.empty(M, K, 32, SCALE_W8, payload.device)
        check("kxw4_repack_e2m3_s8", lib().kxw4_repack_e2m3_s8(
            _ptr(payload), _ptr(block_scale_inv), scale_cols, M, K, _ptr(w.codes), _ptr(w.scales),
            _stream()))
        return w

    @classmethod
    def from_reference_layout(cls, ref_codes: torch.Tensor, ref_scales: torch.Tensor, M: int,
                              K: int, group: int) -> "W4Weight":
        """The reference's d_s4 / d_s4_scale buffers (kernels_dpas.cpp:294-342)."""
        w = cls.empty(M, K, group, SCALE_FP16_ZP4, ref_codes.device)
        check("kxw4_import_ref_weight", lib().kxw4_import_ref_weight(
            _ptr(ref_codes), _ptr(ref_scales), M, K, group, _ptr(w.codes), _ptr(w.scales),
            _stream()))
        return w

    @classmethod
    def repack_e2m3(cls, payload: torch.Tensor, block_scale_inv: torch.Tensor, scale_cols: int,
                    M: int, K: int, mode: int) -> "W4Weight":
        """x_w4_repack_weight_mode: mode 0 = K32, 1 = K16 (the K16 tier), 2 = K64."""
        group = {0: 32, 1: 16, 2: 64}.get(mode, 32)
        w = cls.empty(M, K, group, SCALE_FP16_ZP4, payload.device)
        check("kxw4_repack_e2m3", lib().kxw4_repack_e2m3(
            _ptr(payload), _ptr(block_scale_inv), scale_cols, M, K, mode, _ptr(w.codes),
            _ptr(w.scales), _stream()))
        return w

    def unpack(self):
        codes = torch.empty(self.M, self.K, dtype=torch.int8, device=self.codes.device)
        scales = torch.empty(self.M, self.K // self.group, dtype=torch.int16,
                             device=self.codes.device)
        wc = self.c()
        check("kxw4_unpack_weight", lib().kxw4_unpack_weight(
            C.byref(wc), _ptr(codes), _ptr(scales), _stream()))
        return codes, scales


@dataclass
class QuantAct:
    """Quantized activations: q [T][K] int8 in MFMA slot order, scale
    [T][K/32] or [T], exact code sums [T][K/32]."""
    T: int
    K: int
    block: int
    q: torch.Tensor
    scale: torch.Tensor
    sum: torch.Tensor

    def c(self) -> _lib.Act:
        return _lib.Act(self.T, self.K, self.block, self.q.data_ptr(), self.scale.data_ptr(),
                        self.sum.data_ptr())

    @classmethod
    def empty(cls, T: int, K: int, block: int, device="cuda") -> "QuantAct":
        q = torch.empty(T, K, dtype=torch.int8, device=device)
        scale = torch.empty((T, K // 32) if block == 32 else (T,), dtype=torch.float32,
                            device=device)
        s = torch.empty(T, K // 32, dtype=torch.int32, device=device)
        return cls(T, K, block, q, scale, s)


def slot_permutation(K: int) -> torch.Tensor:
    """perm[k] = storage position of element k (MFMA slot order per 64-chunk)."""
    k = torch.arange(K)
    return (k & ~63) + 16 * ((k >> 3) & 3) + 8 * ((k >> 5) & 1) + (k & 7)


def act_from_codes(q: torch.Tensor, scale: torch.Tensor, sums: torch.Tensor,
                   block: int) -> QuantAct:
    """Wrap already-quantized natural-order codes (e.g. test fixtures)."""
    T, K = q.shape
    perm = slot_permutation(K).to(q.device)
    qs = torch.empty_like(q)
    qs[:, perm] = q
    return QuantAct(T, K, block, qs.contiguous(), scale.contiguous(), sums.contiguous())


def act_codes_natural(a: QuantAct) -> torch.Tensor:
    perm = slot_permutation(a.K).to(a.q.device)
    return a.q[:, perm]


def quantize_act(x: torch.Tensor, block: int = 0, out: Optional[QuantAct] = None) -> QuantAct:
    """Quantize [T][K] f32/bf16 activations; `out` (same T, K, block) is
    reused when given, so the call allocates nothing."""
    T, K = x.shape
    if out is not None and (out.T, out.K, out.block) != (T, K, block):
        raise ValueError("out does not match the activation shape / block")
    a = out if out is not None else QuantAct.empty(T, K, block, x.device)
    check("kxw4_quantize_act", lib().kxw4_quantize_act(
        _ptr(x), _dtype_code(x.dtype), T, K, block, _ptr(a.q), _ptr(a.scale), _ptr(a.sum),
        _stream()))
    return a


@dataclass
class QuantActS4:
    """s4 activations of the W4A4 GEMM: codes q4 [K/128][T][64] uint8 in the
    packed-weight nibble order, scale [K/64][T] f32 and exact code sums
    [K/64][T] i32 (the reference's as4/asum4 layout)."""
    T: int
    K: int
    q4: torch.Tensor
    scale: torch.Tensor
    sum: torch.Tensor

    @classmethod
    def empty(cls, T: int, K: int, device="cuda") -> "QuantActS4":
        q4 = torch.empty(K // 128, T, 64, dtype=torch.uint8, device=device)
        scale = torch.empty(K // 64, T, dtype=torch.float32, device=device)
        s = torch.empty(K // 64, T, dtype=torch.int32, device=device)
        return cls(T, K, q4, scale, s)


def quantize_act_s4(x: torch.Tensor, out: Optional[QuantActS4] = None) -> QuantActS4:
    """Quantize [T][K] f32/bf16 activations to s4 (per (token, K64) absmax/7);
    `out` (same T, K) is reused when given."""
    T, K = x.shape
    if out is not None and (out.T, out.K) != (T, K):
        raise ValueError("out does not match the activation shape")
    a = out if out is not None else QuantActS4.empty(T, K, x.device)
    check("kxw4_quantize_act_s4", lib().kxw4_quantize_act_s4(
        _ptr(x), _dtype_code(x.dtype), T, K, _ptr(a.q4), _ptr(a.scale), _ptr(a.sum), _stream()))
    return a


def s4_codes_natural(a: QuantActS4) -> torch.Tensor:
    """[T][K] int8 codes in K order (inverse of the tile nibble order)."""
    b = a.q4.view(a.K // 128, a.T, 4, 4, 4)                  # [kb][t][g][i][byte]
    lo = (b & 0xF).to(torch.int8)
    hi = (b >> 4).to(torch.int8)
    nib = torch.cat([lo, hi], dim=-1)                        # [kb][t][g][i][b]
    nib = torch.where(nib >= 8, nib - 16, nib)
    return nib.permute(1, 0, 3, 2, 4).reshape(a.T, a.K).contiguous()   # k = 128kb + 32i + 8g + b


def silu_mul_quant(gate: torch.Tensor, up: torch.Tensor, block: int = 32, keep_hidden=True):
    """SiLU(gate) * up of [T][K] f32 rows, quantized (x_silu_mul_quant)."""
    T, K = gate.shape
    _need(gate, "gate", torch.float32, (T, K), gate.device)
    _need(up, "up", torch.float32, (T, K), gate.device)
    a = QuantAct.empty(T, K, block, gate.device)
    hidden = torch.empty(T, K, dtype=torch.float32, device=gate.device) if keep_hidden else None
    check("kxw4_silu_mul_quant", lib().kxw4_silu_mul_quant(
        _ptr(hidden), _ptr(gate), _ptr(up), T, K, block, _ptr(a.q), _ptr(a.scale),
        _ptr(a.sum), _stream()))
    return hidden, a


def rmsnorm_quant(x: torch.Tensor, w_bf16_bits: torch.Tensor, eps: float, block: int = 32,
                  keep_normed=True):
    """(1+w) RMSNorm of [T][H] f32 rows fused with the quantizer
    (x_rmsnorm_quant); w is [H] BF16 bits (int16 or bfloat16)."""
    T, H = x.shape
    _need(x, "x", torch.float32, (T, H), x.device)
    _need(w_bf16_bits, "w", _BITS16 + (torch.bfloat16,), (H,), x.device)
    a = QuantAct.empty(T, H, block, x.device)
    out = torch.empty(T, H, dtype=torch.float32, device=x.device) if keep_normed else None
    check("kxw4_rmsnorm_quant", lib().kxw4_rmsnorm_quant(
        _ptr(out), _ptr(x), _ptr(w_bf16_bits), T, H, eps, block, _ptr(a.q), _ptr(a.scale),
        _ptr(a.sum), _stream()))
    return out, a


def rmsnorm(x: torch.Tensor, w_bf16_bits: torch.Tensor, eps: float, out=None) -> torch.Tensor:
    """Batched (1+w) RMSNorm of [T][H] f32 rows (x_rmsnorm_chunk)."""
    T, H = x.shape
    _need(x, "x", torch.float32, (T, H), x.device)
    _need(w_bf16_bits, "w", _BITS16 + (torch.bfloat16,), (H,), x.device)
    if out is not None:
        _need(out, "out", torch.float32, (T, H), x.device)
    y = out if out is not None else torch.empty(T, H, dtype=torch.float32, device=x.device)
    check("kxw4_rmsnorm", lib().kxw4_rmsnorm(_ptr(y), _ptr(x), _ptr(w_bf16_bits), T, H, eps,
                                             _stream()))
    return y


def _out(T: int, M: int, dtype, device, out=None, name="out"):
    """The [T][M] output buffer: `out` after validation, else a new tensor."""
    _dtype_code(dtype)
    if out is not None:
        return _need(out, name, dtype, (T, M), device)
    return torch.empty(T, M, dtype=dtype, device=device)


def _residual(residual, T: int, M: int, device):
    if residual is not None:
        _need(residual, "residual", torch.float32, (T, M), device)
    return residual


def _check_weight(w: "W4Weight", device):
    if not torch.device(device).type == "cuda":
        raise ValueError("weights must be on the GPU")
    nbytes = w.M * w.K if w.scale_enc == SCALE_W8 else w.M * w.K // 2
    _need(w.codes, "weight codes", torch.uint8, (nbytes,), device)
    _need(w.scales, "weight scales", _BITS16, (w.M * (w.K // w.group),), device)


def _check_act(a: QuantAct, device):
    _need(a.q, "activation codes", torch.int8, (a.T, a.K), device)
    _need(a.scale, "activation scales", torch.float32,
          (a.T, a.K // 32) if a.block == 32 else (a.T,), device)
    _need(a.sum, "activation sums", torch.int32, (a.T, a.K // 32), device)


def gemv(w: W4Weight, a: QuantAct, dtype=torch.float32, residual=None, splits: int = 0,
         out=None) -> torch.Tensor:
    dev = w.codes.device
    _check_weight(w, dev)
    _check_act(a, dev)
    y = _out(a.T, w.M, dtype, dev, out)
    _residual(residual, a.T, w.M, dev)
    wc, ac = w.c(), a.c()
    check("kxw4_gemv", lib().kxw4_gemv(C.byref(wc), C.byref(ac), _ptr(y), _dtype_code(dtype),
                                       _ptr(residual), splits, _stream()))
    return y


def _weight_array(ws: Sequence[W4Weight]):
    cs = [w.c() for w in ws]
    arr = (C.POINTER(_lib.Weight) * len(ws))(*[C.pointer(c) for c in cs])
    return cs, arr


def _outs(ws: Sequence[W4Weight], T: int, dtype, device, outs):
    if outs is not None and len(outs) != len(ws):
        raise ValueError(f"outs has {len(outs)} tensors for {len(ws)} weights")
    return [_out(T, w.M, dtype, device, None if outs is None else outs[i], f"outs[{i}]")
            for i, w in enumerate(ws)]


def gemv_fanout(ws: Sequence[W4Weight], a: QuantAct, dtype=torch.float32, outs=None):
    dev = ws[0].codes.device
    for w in ws:
        _check_weight(w, dev)
    _check_act(a, dev)
    ys = _outs(ws, a.T, dtype, dev, outs)
    keep, warr = _weight_array(ws)
    yarr = (C.c_void_p * len(ws))(*[y.data_ptr() for y in ys])
    ac = a.c()
    check("kxw4_gemv_fanout", lib().kxw4_gemv_fanout(warr, yarr, len(ws), C.byref(ac),
                                                     _dtype_code(dtype), _stream()))
    return ys


def _offsets(offsets):
    if offsets is None:
        return None, 0
    arr = (C.c_int * len(offsets))(*[int(o) for o in offsets])
    return arr, len(offsets) - 1


def gemm(w: W4Weight, a: QuantAct, dtype=torch.float32, residual=None, offsets=None,
         forced_splits: int = 0, out=None) -> torch.Tensor:
    dev = w.codes.device
    _check_weight(w, dev)
    _check_act(a, dev)
    y = _out(a.T, w.M, dtype, dev, out)
    _residual(residual, a.T, w.M, dev)
    off, nseg = _offsets(offsets)
    wc, ac = w.c(), a.c()
    check("kxw4_gemm", lib().kxw4_gemm(C.byref(wc), C.byref(ac), _ptr(y), _dtype_code(dtype),
                                       _ptr(residual), off, nseg, forced_splits, _stream()))
    return y


def gemm_fanout(ws: Sequence[W4Weight], a: QuantAct, dtype=torch.float32, offsets=None,
                forced_splits: int = 0, outs=None):
    dev = ws[0].codes.device
    for w in ws:
        _check_weight(w, dev)
    _check_act(a, dev)
    ys = _outs(ws, a.T, dtype, dev, outs)
    keep, warr = _weight_array(ws)
    yarr = (C.c_void_p * len(ws))(*[y.data_ptr() for y in ys])
    off, nseg = _offsets(offsets)
    ac = a.c()
    check("kxw4_gemm_fanout", lib().kxw4_gemm_fanout(warr, yarr, len(ws), C.byref(ac),
                                                     _dtype_code(dtype), off, nseg,
                                                     forced_splits, _stream()))
    return ys


class PreparedGemv:
    """gemv with its checks and argument marshalling done once: each call is
    one kxw4_gemv on the current stream, for loops that launch the same
    projection on the same buffers (serving steps, benchmarks). The tensors
    must stay alive and keep their shapes; their contents may change."""

    def __init__(self, w: W4Weight, a: QuantAct, dtype=torch.float32, residual=None,
                 splits: int = 0, out=None):
        dev = w.codes.device
        _check_weight(w, dev)
        _check_act(a, dev)
        self.y = _out(a.T, w.M, dtype, dev, out)
        _residual(residual, a.T, w.M, dev)
        self._keep = (w, a, residual)
        self._wc, self._ac = w.c(), a.c()
        self._args = (C.byref(self._wc), C.byref(self._ac), _ptr(self.y), _dtype_code(dtype),
                      _ptr(residual), splits)

    def __call__(self) -> torch.Tensor:
        check("kxw4_gemv", lib().kxw4_gemv(*self._args, _stream()))
        return self.y


class PreparedGemmFanout:
    """gemm_fanout with its checks and argument marshalling done once: each
    call is one kxw4_gemm_fanout on the current stream (see PreparedGemv)."""

    def __init__(self, ws: Sequence[W4Weight], a: QuantAct, dtype=torch.float32, offsets=None,
                 forced_splits: int = 0, outs=None):
        dev = ws[0].codes.device
        for w in ws:
            _check_weight(w, dev)
        _check_act(a, dev)
        self.ys = _outs(ws, a.T, dtype, dev, outs)
        self._keep = (list(ws), a)
        self._wcs, self._warr = _weight_array(ws)
        self._yarr = (C.c_void_p * len(ws))(*[y.data_ptr() for y in self.ys])
        self._off, nseg = _offsets(offsets)
        self._ac = a.c()
        self._args = (self._warr, self._yarr, len(ws), C.byref(self._ac), _dtype_code(dtype),
                      self._off, nseg, forced_splits)

    def __call__(self):
        check("kxw4_gemm_fanout", lib().kxw4_gemm_fanout(*self._args, _stream()))
        return self.ys


def gemm_w4a4(w: W4Weight, a: QuantActS4, dtype=torch.float32, residual=None,
              out=None) -> torch.Tensor:
    """W4A4 GEMM of s4 activations against a K64 weight with FP16|zp scales."""
    dev = w.codes.device
    _check_weight(w, dev)
    _need(a.q4, "s4 codes", torch.uint8, (a.K // 128, a.T, 64), dev)
    _need(a.scale, "s4 scales", torch.float32, (a.K // 64, a.T), dev)
    _need(a.sum, "s4 sums", torch.int32, (a.K // 64, a.T), dev)
    if a.K != w.K:
        raise ValueError(f"activation K {a.K} != weight K {w.K}")
    y = _out(a.T, w.M, dtype, dev, out)
    _residual(residual, a.T, w.M, dev)
    wc = w.c()
    check("kxw4_gemm_w4a4", lib().kxw4_gemm_w4a4(
        C.byref(wc), _ptr(a.q4), _ptr(a.scale), _ptr(a.sum), a.T, _ptr(y), _dtype_code(dtype),
        _ptr(residual), _stream()))
    return y


class TqfFile:
    """A TQF1 model container opened for ingest (tqf_loader.cpp:393-626): the
    tensor table is read at open, payloads only by load_w4 / load_w8."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check("kxw4_tqf_open", lib().kxw4_tqf_open(str(path).encode(), C.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().kxw4_tqf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def header(self):
        u = (C.c_uint32 * 16)()
        f = (C.c_float * 3)()
        t = (C.c_uint32 * 8)()
        check("kxw4_tqf_header", lib().kxw4_tqf_header(self._h, u, f, t))
        return list(u), list(f), list(t)

    def tensors(self):
        out = []
        for i in range(lib().kxw4_tqf_count(self._h)):
            d = _lib.TqfTensor()
            check("kxw4_tqf_tensor", lib().kxw4_tqf_tensor(self._h, i, C.byref(d)))
            out.append({"name": d.name.decode(), "kind": d.kind, "M": d.M, "K": d.K,
                        "scale_rows": d.scale_rows, "scale_cols": d.scale_cols,
                        "offset": d.offset, "bytes": d.bytes})
        return out

    def find(self, name: str) -> int:
        i = lib().kxw4_tqf_find(self._h, name.encode())
        if i < 0:
            raise KeyError(name)
        return i

    def _load(self, name: str, mode: int, group: int, scale_enc: int) -> W4Weight:
        i = self.find(name)
        d = _lib.TqfTensor()
        check("kxw4_tqf_tensor", lib().kxw4_tqf_tensor(self._h, i, C.byref(d)))
        w = W4Weight.empty(d.M, d.K, group, scale_enc)
        check("kxw4_tqf_load_qmma", lib().kxw4_tqf_load_qmma(
            self._h, i, mode, _ptr(w.codes), _ptr(w.scales), _stream()))
        return w

    def load_w4(self, name: str, mode: int = 0) -> W4Weight:
        """x_w4_repack_weight_mode of one QMMA tensor: 0 = K32, 1 = K16, 2 = K64."""
        return self._load(name, mode, {0: 32, 1: 16, 2: 64}[mode], SCALE_FP16_ZP4)

    def load_w8(self, name: str) -> W4Weight:
        """x_w8_repack_weight of one QMMA tensor (the W8A8 tier)."""
        return self._load(name, 8, 32, SCALE_W8)


def partials(w: W4Weight, a: QuantAct) -> torch.Tensor:
    unit = 32 if a.block == 32 else w.group
    P = torch.empty(a.T, w.M, w.K // unit, dtype=torch.int32, device=a.q.device)
    wc, ac = w.c(), a.c()
    check("kxw4_partials", lib().kxw4_partials(C.byref(wc), C.byref(ac), _ptr(P), _stream()))
    return P


class option:
    """Set one kernel-selection option (kxw4_set_option) for a `with` block
    and restore its previous value afterwards, e.g.
    `with ops.option("decode_kernel", 1): ...` for the K-parallel kernel."""

    def __init__(self, name: str, value: int):
        self.name, self.value, self.prev = name, int(value), None

    def __enter__(self):
        prev = C.c_int()
        check("kxw4_set_option", lib().kxw4_set_option(self.name.encode(), self.value, C.byref(prev)))
        self.prev = prev.value
        return self

    def __exit__(self, *exc):
        check("kxw4_set_option", lib().kxw4_set_option(self.name.encode(), self.prev, None))


def gemv_splits(groups: int) -> int:
    return lib().kxw4_gemv_splits(groups)


def gemm_splits(rgroups: int, tgroups: int, ktiles: int, forced: int = 0) -> int:
    return lib().kxw4_gemm_splits(rgroups, tgroups, ktiles, forced)


PROBE_SINK_WORDS = 1 << 16


def probe_mfma_i8(shape: int, iters: int, sink: torch.Tensor) -> tuple:
    """Enqueue the int8 MFMA rate probe (shape 0 = 32x32x32, 1 = 16x16x64) on
    the current stream; returns (sink words written, operation count). Each
    word is iters * K when its wave's accumulators all hold exactly that."""
    ops_count = C.c_double()
    n = lib().kxw4_probe_mfma_i8(shape, iters, _ptr(sink), sink.numel(), C.byref(ops_count), _stream())
    if n < 0:
        raise _lib.KxError("kxw4_probe_mfma_i8", n)
    return n, ops_count.value


def probe_hold(flag: torch.Tensor, max_us: int, status: torch.Tensor) -> None:
    """Enqueue the stream hold on the current stream: it waits until the host
    sets flag[0] (a pinned CPU int32 tensor) to nonzero or max_us pass, then
    writes 1 (released) or 2 (timed out) to status[0] (a device int32
    tensor)."""
    if (flag.device.type != "cpu" or not flag.is_pinned() or flag.dtype != torch.int32
            or status.device.type != "cuda" or status.dtype != torch.int32):
        raise _lib.KxError("kxw4_probe_hold", _lib.EARG)
    check("kxw4_probe_hold", lib().kxw4_probe_hold(C.c_void_p(flag.data_ptr()), int(max_us), _ptr(status),
                                                   _stream()))


def probe_issue(mode: int, waves_per_simd: int, iters: int, sink: torch.Tensor) -> tuple:
    """Enqueue the issue-mix probe (mode 0 MFMA only, 1 FP32 chain only, 2 both
    in one wave, 3 both in separate waves) on the current stream; `sink` is
    float32. Returns (sink words written, blocks per SIMD)."""
    if sink.dtype != torch.float32:
        raise _lib.KxError("kxw4_probe_issue", _lib.EARG)
    blocks = C.c_double()
    n = lib().kxw4_probe_issue(mode, waves_per_simd, iters, _ptr(sink), sink.numel(), C.byref(blocks), _stream())
    if n < 0:
        raise _lib.KxError("kxw4_probe_issue", n)
    return n, blocks.value


def probe_read_shapes() -> int:
    return lib().kxw4_probe_read_shapes()


def probe_read(buf: torch.Tensor, sink: torch.Tensor, shape: int = 0) -> int:
    """Enqueue the pure-read probe over all of `buf` on the current stream in
    launch shape `shape`; returns the number of checksum words written."""
    n = lib().kxw4_probe_read(_ptr(buf), buf.numel() * buf.element_size(), shape, _ptr(sink), sink.numel(),
                              _stream())
    if n < 0:
        raise _lib.KxError("kxw4_probe_read", n)
    return n
