"""The machine probes (kxw4_probe_mfma_i8, kxw4_probe_read, kxw4_probe_issue; counterpart of
xpu/probe/dpas_probe.cpp): the all-ones MFMA chains must end at exactly
iters * K in every wave (the reference's `d == iters * K` check), the read
probe must cover the buffer, the issue probe must write one deterministic word
per wave, and all of them must reject bad arguments. The timing harness's
stream hold (kxw4_probe_hold) must end on the host's flag, or on its own
bound when the flag stays clear.
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


@pytest.mark.parametrize("mode,wps", [(0, 1), (1, 3), (2, 2), (3, 4)])
def test_issue_probe(mode, wps):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.full((ops.PROBE_SINK_WORDS,), 7.0, dtype=torch.float32, device="cuda")
    n, blocks = ops.probe_issue(mode, wps, 25, sink)
    first = sink[:n].clone()
    torch.cuda.synchronize()
    assert n == cus * 4 * wps                        # one word per wave
    assert blocks == 4 * 25 * (wps // 2 if mode == 3 else wps)
    assert torch.all(sink[n:] == 7.0)
    assert torch.isfinite(first).all()
    wave = torch.arange(n, device="cuda") % (4 * wps)
    if mode == 1:
        assert torch.all(first == 0.0)               # the chain alone folds zeros
    elif mode == 3:                                  # waves 4-7 of each eight run the chain alone
        chain = (wave >> 2) & 1 == 1
        assert torch.all(first[chain] == 0.0) and torch.all(first[~chain] != 0.0)
    else:
        assert torch.all(first != 0.0)
        assert torch.all(first == first[0])          # every wave runs the same work
    # and the same words run after run
    ops.probe_issue(mode, wps, 25, sink)
    torch.cuda.synchronize()
    assert torch.equal(sink[:n], first)


def test_issue_probe_arguments():
    sink = torch.zeros(ops.PROBE_SINK_WORDS, dtype=torch.float32, device="cuda")
    for mode, wps, iters in ((4, 1, 1), (-1, 1, 1), (0, 0, 1), (0, 5, 1), (3, 3, 1), (0, 1, 0)):
        with pytest.raises(KxError):
            ops.probe_issue(mode, wps, iters, sink)
    with pytest.raises(KxError):
        ops.probe_issue(0, 1, 1, sink[:16])          # sink too small
    with pytest.raises(KxError):
        ops.probe_issue(0, 1, 1, sink.view(torch.int32))  # float32 sink only


def test_hold_released_by_the_host_flag():
    # the hold keeps the stream until the host sets the pinned flag: work
    # queued behind it waits, then runs; status 1 = released by the flag
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.zeros(1, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ops.probe_hold(flag, 200000, status)
    out.add_(1.0)                                   # queued behind the hold
    e = torch.cuda.Event()
    e.record()
    assert not e.query()                            # still held: the flag is not set
    flag.fill_(1)
    torch.cuda.synchronize()
    assert int(status.item()) == 1 and float(out.item()) == 1.0


def test_hold_times_out_when_the_flag_stays_clear():
    # the host never sets the flag: the hold's own bound ends it (status 2)
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    ops.probe_hold(flag, 3000, status)
    e1.record()
    torch.cuda.synchronize()
    assert int(status.item()) == 2
    assert 2.5 <= e0.elapsed_time(e1) <= 50.0       # ms: about the 3 ms bound


def test_hold_arguments():
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    pinned = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    for flag, max_us in ((torch.zeros(1, dtype=torch.int32), 1000),        # not pinned
                         (pinned, 0), (pinned, 2000000),
                         (torch.zeros(1, dtype=torch.int32, device="cuda"), 1000)):
        with pytest.raises(KxError):
            ops.probe_hold(flag, max_us, status)
