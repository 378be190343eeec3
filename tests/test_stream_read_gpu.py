"""The streaming-read probe behind bench.py --stream-sweep (measurement only,
no counterpart in the reference): every 16-byte word of the buffer is read.
One word holds the probe's sink pattern and every other word is zero, so the
lane that loads that word (and only it) writes the sink: a word the probe
skipped would leave the sink untouched."""
import pytest
import torch

from conftest import print_case
from drama_moe import _lib

pytestmark = pytest.mark.gpu
PATTERN = (0x2468ACE1, 0x13579BDF, 0x7F00FF01)


@pytest.mark.parametrize("words", [1, 7, 2048 * 4 + 3, (16 << 20) // 16 + 3, (96 << 20) // 16 + 5])
def test_stream_read_reaches_every_word(cuda, words):
    print_case("stream read", words)
    lib = _lib.library()
    buf = torch.zeros(words, 4, dtype=torch.int32, device=cuda)
    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    stream = _lib.stream_handle(cuda)
    for position in sorted({0, words // 2, words - 1}):
        buf[position] = torch.tensor([*PATTERN, position + 1], dtype=torch.int64).to(torch.int32)
        sink.zero_()
        _lib.check(lib.dmoe_stream_read(_lib.ptr(buf), words * 16, _lib.ptr(sink), stream))
        torch.cuda.synchronize()
        assert int(sink.item()) == position + 1, position
        buf[position] = 0
    _lib.check(lib.dmoe_stream_read(_lib.ptr(buf), words * 16, _lib.ptr(sink.zero_()), stream))
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
