"""The streaming-read probe the benchmark measures HBM ceilings with
(libsmx_probe.so, a library of its own beside the decode path's) reads
every byte it is given: each wave's sink word equals the XOR of the 32-bit
words it read (wave w of workgroup b: 16-byte words b*256*L + i*256 + 64*w +
lane, i < L; the last workgroup's clamped loads re-read the final 16 bytes,
computed here the same way)."""
import numpy as np
import pytest

from _util import pkg

pytestmark = pytest.mark.gpu


def _host_xor(words: np.ndarray, loads: int, nwords: int) -> np.ndarray:
    n16 = words.size // 4
    q = words.reshape(n16, 4)
    nwg = nwords // 4
    b, w, i, lane = np.meshgrid(np.arange(nwg), np.arange(4), np.arange(loads), np.arange(64),
                                indexing="ij")
    idx = np.minimum(b * 256 * loads + i * 256 + 64 * w + lane, n16 - 1)  # the kernel's clamp
    vals = q[idx]  # [nwg, 4, loads, 64, 4]
    return np.bitwise_xor.reduce(vals.reshape(nwg, 4, -1), axis=2).reshape(-1)


@pytest.mark.parametrize("nbytes", [16, 4096, (1 << 20) + 48, 14_008_320])
@pytest.mark.parametrize("loads", [1, 2, 4, 8, 16])
def test_read_probe_xor(nbytes, loads):
    import torch
    ops = pkg("native.probe")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(nbytes + loads)
    words = rng.integers(0, 2 ** 32, nbytes // 4, dtype=np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(dev)
    nwords = ops.read_probe_sink_size(nbytes, loads)
    assert nwords == 4 * -(-nbytes // (4096 * loads))
    sink = torch.zeros(nwords, dtype=torch.int32, device=dev)
    ops.read_probe(src, nbytes, sink, loads)
    got = sink.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, _host_xor(words, loads, nwords))
