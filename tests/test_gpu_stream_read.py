"""The read-floor kernel (lcml_fp8_stream_read) reads every 16-byte unit of
its buffer: a single marker word, placed at share boundaries, at the ends
and inside, makes the thread that loads it fold to the marker and write the
sink, for several grid sizes (shares that divide the buffer and shares
that do not)."""
import pytest
import torch

from luisaml_amd import capi

pytestmark = pytest.mark.gpu

MARK = 0x9E3779B9


@pytest.mark.parametrize("workgroups", [1, 7, 172, 512, 768, 2048])
def test_stream_read_reads_every_unit(dev, workgroups):
    n_words = 4 * 100003  # 16-byte units not divisible by the grid
    buf = torch.zeros(n_words, dtype=torch.int32, device=dev)
    units = n_words // 4
    per = (units + workgroups - 1) // workgroups
    for unit in sorted({min(u, units - 1) for u in (0, units - 1, per - 1, per, 3 * per + 5, units // 2)}):
        buf.zero_()
        buf[4 * unit + 2] = MARK - (1 << 32)  # the marker's bits as an int32
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        capi.stream_read(buf, sink, workgroups)
        torch.cuda.synchronize()
        assert int(sink.item()) & 0xFFFFFFFF == MARK, (workgroups, unit)
    buf.zero_()
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    capi.stream_read(buf, sink, workgroups)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
