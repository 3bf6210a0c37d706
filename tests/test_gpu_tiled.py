"""Tiled expert weights (weight_layout 1, ds41_expert_slab_tile) through the verify layer and the verify
stack, through the C ABI.

Tiling only reorders where the GEMV loads each 16-byte weight piece from; every lane gets the same bytes
for the same MFMA, so the bar is bit-identical outputs, ids and weights against the row-major layout,
on the fused and the separate down + reduce paths, with an FP8 shared expert, and through a stack with a
host tier and an HBM cache. The device tiling must equal the host tiling byte for byte."""
import ctypes

import numpy as np
import pytest

from test_gpu_moe import dev, host, rand_x, say

pytestmark = pytest.mark.gpu


def make_slabs(gpu, seed, n, H, I):
    import torch
    import ds41_gfx950 as G
    off, size = G.slab_layout(H, I)
    g = torch.Generator(device=gpu).manual_seed(seed)
    s = torch.randint(0, 256, (n, size), dtype=torch.uint8, device=gpu, generator=g)
    for i, (a, b) in ((1, (I, H // 32)), (3, (I, H // 32)), (5, (H, I // 32))):
        s[:, off[i]:off[i] + a * b].random_(119, 124, generator=g)
    t = torch.empty_like(s)
    G.slab_tile(s, t, H, I, n)
    return s, t, off, size


def table_of(slabs, off):
    import torch
    import ds41_gfx950 as G
    entries = [G.slab_entry(slabs[e].data_ptr(), off, e) for e in range(slabs.shape[0])]
    return torch.frombuffer(bytearray(b"".join(bytes(e) for e in entries)), dtype=torch.uint8).to(slabs.device)


def test_device_tiling_equals_host_tiling(gpu):
    import ds41_gfx950 as G
    H, I = 4096, 2880
    s, t, off, size = make_slabs(gpu, 1, 3, H, I)
    want = np.zeros(3 * size, np.uint8)
    G.slab_tile_host(s.cpu().numpy().reshape(-1), want, H, I, 3)
    assert np.array_equal(t.cpu().numpy().reshape(-1), want)


# (T, H, I, E, K, shared, fp8 shared): configs[1], T=8 with a 72-row tile (separate down + reduce), small
# shapes, an FP8 shared expert
CASES = [(4, 4096, 2880, 384, 6, True, False), (8, 1024, 4096, 64, 8, True, False), (1, 512, 512, 32, 4, True, False),
         (5, 2048, 1536, 96, 3, False, False), (4, 4096, 2880, 64, 6, False, True)]


@pytest.mark.parametrize("T,H,I,E,K,shared,fp8", CASES)
def test_tiled_layer_bitexact(gpu, T, H, I, E, K, shared, fp8):
    import torch
    import ds41_gfx950 as G
    say(f"tiled layer T={T} H={H} I={I} E={E} K={K} shared={shared} fp8={fp8}")
    s, t, off, size = make_slabs(gpu, 10 + T, E + 1, H, I)
    tables = {0: table_of(s, off), 1: table_of(t, off)}
    rng = np.random.default_rng(20 + T)
    f8 = None
    if fp8:
        from test_gpu_dense_fp8 import fp8_shared
        f8_dev = {k: dev(v, gpu) for k, v in fp8_shared(rng, H, I).items()}
        f8 = G.fp8_expert(f8_dev)
    for rep in range(2):
        x = dev(rand_x(rng, T, H), gpu)
        wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
        bias = dev(np.zeros(E, np.float32), gpu)
        for mask in (0, 32):
            out = {}
            for layout in (0, 1):
                ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
                y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
                ids = torch.full((T, K), -1, dtype=torch.int32, device=gpu)
                a = G.make_layer_args(x, wg, bias, tables[layout], 0, E if shared and not fp8 else -1, T, H, I, E, K, y,
                                      ws, ids_out=ids)
                a.weight_layout = layout
                a.stage_mask = mask
                if f8 is not None:
                    a.shared_fp8 = ctypes.addressof(f8)
                G.moe_layer(a)
                torch.cuda.synchronize()
                assert G.take_status() == 0
                out[layout] = (host(y), host(ids))
            assert np.array_equal(out[0][1], out[1][1])
            diff = int(np.sum(out[0][0] != out[1][0]))
            say(f"  rep {rep} mask {mask}: differing outputs {diff} of {out[0][0].size}")
            assert diff == 0 and not np.any(out[1][0] == 0x7fc0)


def test_tiled_stack_with_host_tier_and_cache_bitexact(gpu):
    """A 3-layer stack at configs[4]'s layer shape (16 host-tier experts per layer) in both layouts: the tiled
    stack's host slabs are tiled too. Router routing and Zipf-like given ids; then both stacks get an HBM cache
    and prefetches."""
    import torch
    import ds41_gfx950 as G
    L, T, H, I, E, K = 3, 4, 4096, 2880, 96, 6
    say(f"tiled stack L={L} T={T} H={H} I={I} E={E}")
    stacks, keep = {}, []
    host_sets = [list(range(l, E, 6)) for l in range(L)]
    layers = {0: [], 1: []}
    for l in range(L):
        s, t, off, size = make_slabs(gpu, 40 + l, E + 1, H, I)
        hs = host_sets[l]
        hidx = np.full(E, -1, np.int32)
        hidx[hs] = np.arange(len(hs), dtype=np.int32)
        hidx_dev = torch.from_numpy(hidx).to(gpu)
        wg = torch.from_numpy((np.random.default_rng(l).standard_normal((E, H)) * 0.02).astype(np.float32)).to(gpu)
        bias = torch.zeros(E, dtype=torch.float32, device=gpu)
        for layout, sl in ((0, s), (1, t)):
            entries = [G.DeviceExpert() if e in hs else G.slab_entry(sl[e].data_ptr(), off, e) for e in range(E + 1)]
            table = torch.frombuffer(bytearray(b"".join(bytes(e) for e in entries)), dtype=torch.uint8).to(gpu)
            pinned = torch.empty((len(hs), size), dtype=torch.uint8, pin_memory=True)
            pinned.copy_(sl[hs].cpu())
            layers[layout].append(dict(router_w=wg, router_bias=bias, table=table, expert_base=0, shared_index=E,
                                       host_index=hidx_dev, host_slabs=pinned))
            keep.append((sl, table, pinned))
    for layout in (0, 1):
        stacks[layout] = G.VerifyStack(layers[layout], T, H, I, E, K, slab_bytes=size, weight_layout=layout)
    rng = np.random.default_rng(7)

    def run(st, x, route=None):
        y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
        lo = torch.empty((L, T, H), dtype=torch.bfloat16, device=gpu)
        ids = torch.empty((L, T, K), dtype=torch.int32, device=gpu)
        st.step(x, y, route_ids=route, layer_out=lo, ids_out=ids)
        torch.cuda.synchronize()
        return host(y), host(lo), host(ids)

    for phase in ("plain", "cache"):
        if phase == "cache":
            for layout in (0, 1):
                stacks[layout].cache(24)
        for step in range(4):
            x = dev(rand_x(rng, T, H), gpu)
            route = None
            if step % 2:
                rid = np.stack([[rng.choice(E, K, replace=False) for _ in range(T)] for _ in range(L)]).astype(np.int32)
                route = torch.from_numpy(rid).to(gpu)
                if phase == "cache":
                    for layout in (0, 1):
                        stacks[layout].prefetch_routes(rid)
            a, b = run(stacks[0], x, route), run(stacks[1], x, route)
            for u, v in zip(a, b):
                assert np.array_equal(u, v)
            assert G.take_status() == 0
    for st in stacks.values():
        st.close()
