"""The HBM streaming-read probe (bench.py's measured read ceiling) reads every 16-byte piece of its
buffer exactly once, for every loads-in-flight count and load kind the ceiling sweep uses: the XOR
of all sink words equals the XOR of all 32-bit words of the buffer."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("u,nt", [(4, 0), (8, 0), (16, 0), (4, 1), (8, 1), (16, 1)])
@pytest.mark.parametrize("nbytes,blocks", [(1 << 20, 8), ((1 << 20) + 48, 3), (4096, 64), (16, 1)])
def test_read_probe_reads_every_piece_once(gpu, nbytes, blocks, u, nt):
    import torch
    import ds41_gfx950 as G
    rng = np.random.default_rng(nbytes + blocks)
    host = rng.integers(0, 256, nbytes, dtype=np.uint8)
    buf = torch.from_numpy(host).to(gpu)
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=gpu)
    if (u, nt) == (4, 0):
        G.hbm_read_probe(buf, sink, blocks)
    else:
        G.hbm_read_probe_ex(buf, sink, blocks, u, nt)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.view(np.uint32))
    assert got == want
