"""The machine probes (kxw4_probe_mfma_i8, kxw4_probe_read; counterpart of
xpu/probe/dpas_probe.cpp): the all-ones MFMA chains must end at exactly
iters * K in every wave (the reference's `d == iters * K` check), and the read
probe must cover the buffer and reject bad arguments.
"""
import pytest

torch = pytest.importorskip("torch")

from knivesysl_xe_amd import ops  # noqa: E402
from knivesysl_xe_amd._lib import KxError  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.mark.parametrize("shape,k", [(0, 32), (1, 64)])
@pytest.mark.parametrize("iters", [1, 37, 1000])
def test_mfma_probe_counts(shape, k, iters):
    sink = torch.full((ops.PROBE_SINK_WORDS,), 7, dtype=torch.int32, device="cuda")
    n, count = ops.probe_mfma_i8(shape, iters, sink)
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert n == cus * 8                              # 2 work-groups of 4 waves per CU
    assert torch.all(sink[:n] == iters * k)
    assert torch.all(sink[n:] == 7)                  # nothing written past the waves
    assert count == n * 4 * iters * (2 * 32 * 32 * 32 if shape == 0 else 2 * 16 * 16 * 64)


@pytest.mark.parametrize("shape", range(8))
def test_read_probe(shape):
    assert ops.probe_read_shapes() == 8
    sink = torch.full((ops.PROBE_SINK_WORDS,), 7, dtype=torch.int32, device="cuda")
    buf = torch.zeros((3 << 20) + 48, dtype=torch.uint8, device="cuda")
    n = ops.probe_read(buf, sink, shape)
    torch.cuda.synchronize()
    assert n > 0 and torch.all(sink[:n] == 0)       # a zero buffer folds to zero
    assert torch.all(sink[n:] == 7)
    for pos in (0, 12345, buf.numel() - 1):         # one byte set: exactly one wave sees it
        buf.zero_()
        buf[pos] = 0x5A
        n = ops.probe_read(buf, sink, shape)
        torch.cuda.synchronize()
        nz = sink[:n][sink[:n] != 0]
        # the fold XORs dwords, so the byte keeps its place in its dword
        assert nz.numel() == 1 and nz.item() == 0x5A << (8 * (pos % 4))
    with pytest.raises(KxError):
        ops.probe_read(buf[1:17], sink)              # misaligned
    with pytest.raises(KxError):
        ops.probe_read(buf, sink, 8)                 # no such launch shape
    with pytest.raises(KxError):
        ops.probe_mfma_i8(2, 10, sink)               # no such shape
    with pytest.raises(KxError):
        ops.probe_mfma_i8(0, 10, sink[:16])          # sink too small
