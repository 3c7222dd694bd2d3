"""The bench's device-ceiling probes (lfm3_measure_stream_read,
lfm3_measure_mfma_f16) compute what they claim: the read's per-block XORs
fold to the XOR of every word of the buffer, and the all-ones MFMA loop
leaves each wave exactly 1024 x iterations."""
import numpy as np
import pytest

import lfm3amd as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,blocks", [(64 << 20, 1024), (16, 1), (4096 + 16, 7),
                                           ((3 << 20) + 48, 256)])
def test_stream_read_folds_every_word(nbytes, blocks):
    words = L.uniform_u32(L.SEED, f"cal.read.{nbytes}", nbytes // 4, 0, 0xffffffff)
    buf = L.DeviceBuffer.of(words)
    sink = L.DeviceBuffer(blocks * 4)
    L.check(L.lib().lfm3_measure_stream_read(buf.addr, nbytes, sink.addr, blocks, None))
    L.synchronize()
    got = np.bitwise_xor.reduce(sink.download(np.uint32, blocks))
    assert int(got) == int(np.bitwise_xor.reduce(words))


@pytest.mark.parametrize("iterations,blocks", [(1, 1), (300, 17), (16384, 4)])
def test_mfma_loop_counts_exactly(iterations, blocks):
    sink = L.DeviceBuffer(blocks * 4 * 4)
    L.check(L.lib().lfm3_measure_mfma_f16(iterations, blocks, sink.addr, None))
    L.synchronize()
    got = sink.download(np.float32, blocks * 4)
    assert np.all(got == np.float32(1024 * iterations))
    assert L.lib().lfm3_measure_mfma_f16_flops(iterations, blocks) == \
        blocks * 4 * 8 * iterations * 16 * 16 * 32 * 2
