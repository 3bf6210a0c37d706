"""The decode layer's fused down projection + ordered reduction against the two separate kernels
(stage_mask bit 5), through the C ABI.

Bar: identical output bits. In the fused kernel one wave runs each job's whole down GEMV with the
same chunk sequence and MFMA chain as the separate down kernel (the job's weight scales staged in
LDS, all I/32 pieces of them), and the workgroup then adds each token's bf16 rows in the reduce
kernel's order (ascending expert id, shared row last), so no rounding step differs. Cases cover I
above 4096 (more than 128 scale pieces per 16-row block) and an FP8 shared expert, whose row the
fused kernel reads from the FP8 down kernel's output. Parity of the layer against the oracle
(rel-L2 <= 1e-3) is covered by test_gpu_moe.py and test_gpu_dense_fp8.py."""
import numpy as np
import pytest

from test_gpu_moe import dev, host, make_layer, rand_x, say

pytestmark = pytest.mark.gpu

# (T, H, I, E, K, shared): config 1 with and without the shared expert, T = 6 at the same shape
# (a 142 KB LDS tile), fewer jobs than waves (T = 1), and T = 8, K = 8, I = 4096, whose 72-row
# tile does not fit (both runs take the separate kernels).
CASES = [(4, 4096, 2880, 384, 6, True), (4, 4096, 2880, 64, 6, False), (6, 4096, 2880, 128, 6, True),
         (8, 1024, 4096, 64, 8, True),
         (1, 512, 512, 32, 4, True), (5, 2048, 1536, 96, 3, True), (7, 768, 1024, 48, 5, False),
         (2, 1024, 6144, 32, 2, True), (1, 1024, 8192, 32, 1, True), (3, 512, 5120, 16, 2, False)]


@pytest.mark.parametrize("T,H,I,E,K,shared", CASES)
def test_fused_down_reduce_matches_separate_kernels(gpu, T, H, I, E, K, shared):
    import torch
    import ds41_gfx950 as G
    say(f"fused down+reduce T={T} H={H} I={I} E={E} K={K} shared={shared}")
    P, experts = make_layer(gpu, 31 + T, H, I, E, T)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(32 + I)
    for rep in range(2):  # two inputs through the same workspace
        x_np = rand_x(rng, T, H)
        wg_np = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        x, wg = dev(x_np, gpu), dev(wg_np, gpu)
        bias = dev(np.zeros(E, np.float32), gpu)
        ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
        out = {}
        for mask in (0, 32):
            y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
            a = G.make_layer_args(x, wg, bias, table, 0, E if shared else -1, T, H, I, E, K, y, ws)
            a.stage_mask = mask
            G.moe_layer(a)
            torch.cuda.synchronize()
            assert G.take_status() == 0
            out[mask] = host(y)
        fused, sep = out[0], out[32]
        assert not np.any(fused == 0x7fc0), "unwritten output"
        diff = int(np.sum(fused != sep))
        say(f"  rep {rep}: differing bf16 outputs {diff} of {fused.size}")
        assert np.array_equal(fused, sep)


def test_fused_down_reduce_fp8_shared_matches_separate_kernels(gpu):
    """configs[1]'s layer with the checkpoint's FP8 shared expert: fused and separate kernels give
    the same bits (the fused kernel takes the shared row from the FP8 down kernel's output)."""
    import ctypes
    import torch
    import ds41_gfx950 as G
    from test_gpu_dense_fp8 import fp8_shared
    T, H, I, E, K = 4, 4096, 2880, 64, 6
    say(f"fused down+reduce with FP8 shared expert T={T} H={H} I={I} E={E} K={K}")
    P, experts = make_layer(gpu, 41, H, I, E, T)
    table, _ = G.device_table(experts[:E], gpu)
    rng = np.random.default_rng(42)
    f8_dev = {k: dev(v, gpu) for k, v in fp8_shared(rng, H, I).items()}
    f8 = G.fp8_expert(f8_dev)
    x = dev(rand_x(rng, T, H), gpu)
    wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
    bias = dev(np.zeros(E, np.float32), gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    out = {}
    for mask in (0, 32):
        y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
        a = G.make_layer_args(x, wg, bias, table, 0, -1, T, H, I, E, K, y, ws)
        a.shared_fp8 = ctypes.addressof(f8)
        a.stage_mask = mask
        G.moe_layer(a)
        torch.cuda.synchronize()
        assert G.take_status() == 0
        out[mask] = host(y)
    say(f"  differing bf16 outputs {int(np.sum(out[0] != out[32]))} of {out[0].size}")
    assert not np.any(out[0] == 0x7fc0), "unwritten output"
    assert np.array_equal(out[0], out[32])
