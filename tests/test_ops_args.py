"""The torch front end validates every caller buffer before its pointer
reaches a kernel (the kernels trust the sizes they are given). These checks
run before any HIP call, so they are covered here on the CPU."""
import pytest
import torch

from knivesysl_xe_amd import ops


def test_need_rejects_dtype_shape_layout_and_device():
    t = torch.zeros(8, 16, dtype=torch.float32)
    assert ops._need(t, "t", torch.float32, (8, 16), "cpu") is t
    with pytest.raises(ValueError, match="must be torch.float32"):
        ops._need(t.bfloat16(), "t", torch.float32, (8, 16), "cpu")
    with pytest.raises(ValueError, match="shape"):
        ops._need(t, "t", torch.float32, (8, 17), "cpu")
    with pytest.raises(ValueError, match="shape"):
        ops._need(t.view(128), "t", torch.float32, (8, 16), "cpu")
    with pytest.raises(ValueError, match="contiguous"):
        ops._need(t.t(), "t", torch.float32, (16, 8), "cpu")
    with pytest.raises(ValueError, match="must be on cuda"):
        ops._need(t, "t", torch.float32, (8, 16), "cuda:0")
    with pytest.raises(ValueError, match="torch.Tensor"):
        ops._need(None, "t", torch.float32, (8, 16), "cpu")


def test_out_and_residual_are_checked_against_the_projection():
    out = torch.zeros(8, 64, dtype=torch.bfloat16)
    # a bf16 buffer for an f32 projection, a short one, the right one
    with pytest.raises(ValueError, match="out must be torch.float32"):
        ops._out(8, 64, torch.float32, "cpu", out)
    with pytest.raises(ValueError, match="shape"):
        ops._out(8, 128, torch.bfloat16, "cpu", out)
    assert ops._out(8, 64, torch.bfloat16, "cpu", out) is out
    with pytest.raises(ValueError, match="unsupported dtype"):
        ops._out(8, 64, torch.float16, "cpu", None)
    with pytest.raises(ValueError, match="residual must be torch.float32"):
        ops._residual(out, 8, 64, "cpu")
    with pytest.raises(ValueError, match="shape"):
        ops._residual(torch.zeros(8, 32), 8, 64, "cpu")


def test_outs_count_must_match_weights():
    w = ops.W4Weight(64, 128, 128, 0, torch.zeros(64 * 64, dtype=torch.uint8),
                     torch.zeros(64, dtype=torch.int16))
    with pytest.raises(ValueError, match="outs has 1 tensors for 2 weights"):
        ops._outs([w, w], 8, torch.float32, "cpu", [torch.zeros(8, 64)])
    with pytest.raises(ValueError, match=r"outs\[1\]"):
        ops._outs([w, w], 8, torch.float32, "cpu", [torch.zeros(8, 64), torch.zeros(8, 32)])


def test_weight_and_activation_buffers_are_checked():
    w = ops.W4Weight(64, 128, 128, 0, torch.zeros(64 * 64, dtype=torch.uint8),
                     torch.zeros(64, dtype=torch.int16))
    with pytest.raises(ValueError, match="weights must be on the GPU"):
        ops._check_weight(w, "cpu")
    short = ops.W4Weight(64, 128, 128, 0, torch.zeros(64 * 32, dtype=torch.uint8),
                         torch.zeros(64, dtype=torch.int16))
    with pytest.raises(ValueError, match="weights must be on the GPU"):
        ops.gemv(short, None)
    a = ops.QuantAct.empty(8, 128, 0, "cpu")
    ops._check_act(a, "cpu")
    bad = ops.QuantAct(8, 128, 32, a.q, a.scale, a.sum)      # per-token scales, block 32
    with pytest.raises(ValueError, match="activation scales"):
        ops._check_act(bad, "cpu")


def test_float_producers_take_float32_rows():
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    w = torch.zeros(128, dtype=torch.int16)
    with pytest.raises(ValueError, match="x must be torch.float32"):
        ops.rmsnorm(x, w, 1e-6)
    with pytest.raises(ValueError, match="x must be torch.float32"):
        ops.rmsnorm_quant(x, w, 1e-6)
    with pytest.raises(ValueError, match="w must have shape"):
        ops.rmsnorm(x.float(), torch.zeros(64, dtype=torch.int16), 1e-6)
    with pytest.raises(ValueError, match="gate must be torch.float32"):
        ops.silu_mul_quant(x, x)
    with pytest.raises(ValueError, match="up must have shape"):
        ops.silu_mul_quant(x.float(), torch.zeros(2, 64))
