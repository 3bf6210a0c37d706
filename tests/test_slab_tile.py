"""Tiling of canonical expert slabs (ds41_expert_slab_tile_host), on the CPU: the 16-byte piece of row n,
K32 group g of each [N][K/2] weight tensor moves to (n / 16) * (K / 32) * 256 + g * 256 + (n % 16) * 16,
the scales and the padding between tensors stay where they are. Checked against a numpy statement of
that permutation, and as a bijection (every byte of the tiled tensor comes from the row-major one)."""
import numpy as np
import pytest

import ds41_gfx950 as G


def numpy_tile(slab, H, I):
    off, size = G.slab_layout(H, I)
    out = slab.copy()
    for idx, N, K in ((0, I, H), (2, I, H), (4, H, I)):
        ng = K // 32
        w = slab[off[idx]:off[idx] + N * K // 2].reshape(N // 16, 16, ng, 16)  # [row group][row][group][16 B]
        out[off[idx]:off[idx] + N * K // 2] = w.transpose(0, 2, 1, 3).reshape(-1)
    return out


@pytest.mark.parametrize("H,I", [(512, 256), (1024, 512), (4096, 2880)])
def test_host_tiling_matches_numpy(H, I):
    off, size = G.slab_layout(H, I)
    rng = np.random.default_rng(H + I)
    count = 2
    src = rng.integers(0, 256, count * size, dtype=np.uint8)
    dst = np.zeros_like(src)
    G.slab_tile_host(src, dst, H, I, count)
    for c in range(count):
        s = src[c * size:(c + 1) * size]
        assert np.array_equal(dst[c * size:(c + 1) * size], numpy_tile(s, H, I))
    assert np.array_equal(np.sort(dst), np.sort(src))  # a permutation of the bytes
    assert G.lib().ds41_expert_slab_tile_host(src.ctypes.data, src.ctypes.data, H, I, 1) == 1  # in place: refused
