"""GPU parity of the FP8 W8A8 shared-expert path (components/dense/src/dense.cu:37-91,
ops.cu:103-106, batch.inc:330-335) against the oracle, through the C ABI.

Bars: MXFP8 quantisation and the shared-expert activation bit-exact; projections, the shared
expert and the MoE layer with an FP8 shared expert within rel-L2 1e-3 of the oracle's exact
per-block result (the bar for MoE outputs)."""
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a, gpu):
    import torch
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(gpu).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def host(t):
    import torch
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.sum((a - b) ** 2) / max(np.sum(b ** 2), 1e-300)))


def fp8_weights(rng, n, k, kind="normal"):
    """E4M3 codes + 32x32 block E8M0 scales. "normal": N(0,1) values quantised per block the way an
    FP8 checkpoint is (amax -> 448); "bytes": uniform codes (all exponents, no NaN)."""
    if kind == "bytes":
        w = rng.integers(0, 256, (n, k), dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] = 0x3C
        ws = rng.integers(118, 126, (n // 32, k // 32), dtype=np.uint8)
        return w, ws
    import torch  # generated on the GPU; any valid codes do, the oracle reads the same bytes
    g = torch.Generator(device="cuda:0").manual_seed(int(rng.integers(1 << 31)))
    v = torch.randn((n, k), generator=g, device="cuda:0", dtype=torch.float32)
    blocks = v.abs().reshape(n // 32, 32, k // 32, 32).amax(dim=(1, 3))
    e = torch.ceil(torch.log2(blocks.clamp_min(1e-30) / 448.0))
    ws = (e + 127 - 6).to(torch.uint8)  # extra 2^-6 overall: weights of size ~0.01
    scale = torch.exp2(e).repeat_interleave(32, 0).repeat_interleave(32, 1)
    w = (v / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    w = torch.where((w & 0x7F) == 0x7F, torch.full_like(w, 0x7E), w)
    return w.cpu().numpy(), ws.cpu().numpy()


def rand_x(rng, m, k):
    return O.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))


def test_dense_quant_bitexact(gpu):
    import ds41_gfx950 as G
    rng = np.random.default_rng(1)
    x = rand_x(rng, 5, 4096)
    a, s = G.dense_quant(dev(x, gpu))
    q, qs = O.quantize_mxfp8(x)
    assert np.array_equal(host(a), q) and np.array_equal(host(s), qs)


def test_shared_act_bitexact(gpu):
    import ds41_gfx950 as G
    rng = np.random.default_rng(2)
    g = O.bf16_bits((rng.standard_normal((4, 2880)) * 6).astype(np.float32))
    u = O.bf16_bits((rng.standard_normal((4, 2880)) * 6).astype(np.float32))
    z, a, s = G.dense_shared_act(dev(g, gpu), dev(u, gpu))
    want = O.swiglu(g, u, None, 10.0)
    q, qs = O.quantize_mxfp8(want)
    assert np.array_equal(host(z), want)
    assert np.array_equal(host(a), q) and np.array_equal(host(s), qs)


@pytest.mark.parametrize("m,n,k,kind", [(1, 64, 256, "bytes"), (4, 2880, 4096, "normal"), (8, 4096, 2880, "normal"),
                                        (3, 96, 160, "bytes"), (5, 32, 32, "bytes"), (2, 512, 15360, "normal"),
                                        (7, 128, 480, "normal")])
def test_dense_fp8_vs_oracle(gpu, m, n, k, kind):
    import ds41_gfx950 as G
    say(f"dense fp8 M={m} N={n} K={k} {kind}")
    rng = np.random.default_rng(m * 7 + n + k)
    w, ws = fp8_weights(rng, n, k, kind)
    x = rand_x(rng, m, k)
    xq, xs = O.quantize_mxfp8(x)
    y = G.dense_fp8(dev(xq, gpu), dev(xs, gpu), dev(w, gpu), dev(ws, gpu), n)
    import torch
    torch.cuda.synchronize()
    acc, ref = O.dense_fp8(w, ws, xq, xs, m, n, k)
    err = rel_l2(O.bf16_to_f32(host(y)), O.bf16_to_f32(ref))
    say(f"  rel-L2 {err:.3e}, bf16 exact {np.mean(host(y) == ref):.4f}")
    assert err <= 1e-3


def fp8_shared(rng, H, I):
    g, gs = fp8_weights(rng, I, H)
    u, us = fp8_weights(rng, I, H)
    d, ds = fp8_weights(rng, H, I)
    return dict(gate=g, gate_scale=gs, up=u, up_scale=us, down=d, down_scale=ds)


def test_moe_layer_with_fp8_shared_expert(gpu):
    """The decode layer with its shared expert in FP8 (args.shared_fp8): routed experts MXFP4 as
    before; the output equals the ordered reduce of the oracle's routed rows and its FP8 shared
    expert row."""
    import torch
    import ds41_gfx950 as G
    from test_gpu_moe import make_layer
    H, I, E, K, T = 4096, 2880, 64, 6, 4
    say(f"moe layer with FP8 shared expert T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 21, H, I, E, T)
    table, _ = G.device_table(experts[:E], gpu)
    rng = np.random.default_rng(22)
    sh_np = fp8_shared(rng, H, I)
    sh_dev = {k: dev(v, gpu) for k, v in sh_np.items()}
    f8 = G.fp8_expert(sh_dev)
    x_np = rand_x(rng, T, H)
    wg_np = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias_np = np.zeros(E, np.float32)
    x, wg, bias = dev(x_np, gpu), dev(wg_np, gpu), dev(bias_np, gpu)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    ids = torch.empty((T, K), dtype=torch.int32, device=gpu)
    wts = torch.empty((T, K), dtype=torch.float32, device=gpu)
    import ctypes
    args = G.make_layer_args(x, wg, bias, table, 0, -1, T, H, I, E, K, y, ws, ids_out=ids, weights_out=wts)
    args.shared_fp8 = ctypes.addressof(f8)
    G.moe_layer(args)
    torch.cuda.synchronize()
    assert G.take_status() == 0
    gids, gw, gy = host(ids), host(wts), host(y)
    xq, xs = O.quantize_mxfp8(x_np)
    routed = np.zeros((T, K, H), np.uint16)
    for e in sorted(set(gids.ravel().tolist())):
        ex = {k: host(v) for k, v in experts[e].items()}
        slots = [(t, j) for t in range(T) for j in range(K) if gids[t, j] == e]
        rows = np.array([t for t, _ in slots])
        out = O.expert_ffn(ex, xq[rows], xs[rows], np.array([gw[t, j] for t, j in slots], np.float32), H, I)
        for r, (t, j) in enumerate(slots):
            routed[t, j] = out[r]
    shared = O.shared_fp8_ffn(sh_np, xq, xs, H, I)
    ref = O.reduce_experts(routed, gids, shared)
    err = rel_l2(O.bf16_to_f32(gy), O.bf16_to_f32(ref))
    say(f"  y rel-L2 {err:.3e}, bf16 exact {np.mean(gy == ref):.4f}")
    assert err <= 1e-3
    # rejected arguments: an FP8 shared expert together with a table shared index
    args.shared_index = 0
    assert G.lib().ds41_moe_verify_layer(ctypes.byref(args), None) != 0
