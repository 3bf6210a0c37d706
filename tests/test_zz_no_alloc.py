"""The allocation-free verify layer (ds41_moe_verify_layer_noalloc) against ds41_moe_verify_layer,
through the C ABI.

The no-alloc entry runs the same kernels on a fixed device array instead of the caller's workspace,
so the bar is identical output bits (and identical routing) for the same inputs. Two calls in a row
share the array; the second uses a smaller shape, so anything the first call left behind that the
second one read would show up as a difference. A shape whose workspace exceeds the array is
rejected with hipErrorInvalidValue before any launch."""
import numpy as np
import pytest

from test_gpu_moe import dev, host, make_layer, rand_x, say

pytestmark = pytest.mark.gpu

# (T, H, I, E, K, shared): configs[1]'s layer, then a smaller one on the same array.
CALLS = [(4, 4096, 2880, 384, 6, True), (2, 1024, 512, 32, 4, False)]


def _layer(gpu, T, H, I, E, K, shared, seed):
    import torch
    import ds41_gfx950 as G
    P, experts = make_layer(gpu, seed, H, I, E, T)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(seed + 1)
    x = dev(rand_x(rng, T, H), gpu)
    wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
    bias = dev(np.zeros(E, np.float32), gpu)
    return P, table, x, wg, bias


def test_noalloc_layer_matches_workspace_layer(gpu):
    import torch
    import ds41_gfx950 as G
    assert G.moe_layer_noalloc_max_bytes() == 1536 * 1024
    keep = []
    for n, (T, H, I, E, K, shared) in enumerate(CALLS):
        say(f"no-alloc layer call {n}: T={T} H={H} I={I} E={E} K={K} shared={shared}")
        assert G.layer_workspace_bytes(T, H, I, E, K) <= G.moe_layer_noalloc_max_bytes()
        P, table, x, wg, bias = _layer(gpu, T, H, I, E, K, shared, 70 + n)
        keep.append((P, table))
        si = E if shared else -1
        outs = []
        for noalloc in (False, True):
            y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
            ids = torch.full((T, K), -1, dtype=torch.int32, device=gpu)
            wts = torch.full((T, K), float("nan"), dtype=torch.float32, device=gpu)
            if noalloc:
                ws = torch.empty(0, dtype=torch.uint8, device=gpu)  # ignored by the entry point
                a = G.make_layer_args(x, wg, bias, table, 0, si, T, H, I, E, K, y, ws, ids_out=ids,
                                      weights_out=wts)
                a.workspace, a.workspace_bytes = 0, 0
                G.check(G.moe_layer_noalloc_rc(a), "ds41_moe_verify_layer_noalloc")
            else:
                ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
                a = G.make_layer_args(x, wg, bias, table, 0, si, T, H, I, E, K, y, ws, ids_out=ids,
                                      weights_out=wts)
                G.moe_layer(a)
            torch.cuda.synchronize()
            assert G.take_status() == 0
            outs.append((host(y), host(ids), host(wts)))
        (y0, i0, w0), (y1, i1, w1) = outs
        say(f"  differing bf16 outputs {int(np.sum(y0 != y1))} of {y0.size}")
        assert np.array_equal(i0, i1) and np.array_equal(w0.view(np.uint32), w1.view(np.uint32))
        assert np.array_equal(y0, y1)
        assert not np.any((y1 & 0x7fff) > 0x7f80), "NaN in the no-alloc output"


def test_noalloc_layer_rejects_oversized_workspace(gpu):
    import torch
    import ds41_gfx950 as G
    T, H, I, E, K = 8, 8192, 6144, 64, 8  # a shape the layer accepts, with a 1.7 MB workspace
    need = G.layer_workspace_bytes(T, H, I, E, K)
    say(f"no-alloc layer rejects T={T} H={H} I={I} K={K}: workspace {need} B > "
        f"{G.moe_layer_noalloc_max_bytes()} B")
    assert need > G.moe_layer_noalloc_max_bytes()
    z = torch.zeros(16, dtype=torch.uint8, device=gpu)
    a = G.make_layer_args(z, z, z, z, 0, -1, T, H, I, E, K, z, z)
    assert G.moe_layer_noalloc_rc(a) == 1  # hipErrorInvalidValue, before any launch
