"""GPU parity of the gfx950 MoE kernels against the oracle, through the C ABI.

Bars: MXFP4 dequant and MXFP8 quant bit-exact; router
top-k indices, route weights and the ordered reduction bit-exact given
identical inputs; projections and the MoE layer within rel-L2 1e-3 of the
oracle's fp32-accumulate result."""
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


def rand_mx(rng, n, k):
    return (rng.integers(0, 256, (n, k // 2), dtype=np.uint8),
            rng.integers(119, 124, (n, k // 32), dtype=np.uint8))


def rand_x(rng, m, k):
    return O.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))


def test_dequant_bitexact(gpu):
    import ds41_gfx950 as G
    say("dequant: exhaustive codes x scales")
    n, k = 256, 64
    w = np.zeros((n, k // 2), np.uint8)
    for c in range(16):
        w[:, c] = c | (((c + 7) % 16) << 4)
        w[:, 16 + c] = ((c * 3) % 16) | (c << 4)
    s = np.repeat(np.arange(256, dtype=np.uint8).reshape(n, 1), 2, axis=1)
    got = host(G.dequant_mxfp4(dev(w, gpu), dev(s, gpu), n, k))
    ref = O.dequant_mxfp4(w, s, n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))  # bit patterns, NaN included
    rng = np.random.default_rng(0)
    w, s = rand_mx(rng, 300, 4096)
    got = host(G.dequant_mxfp4(dev(w, gpu), dev(s, gpu), 300, 4096))
    assert np.array_equal(got.view(np.uint32), O.dequant_mxfp4(w, s, 300, 4096).view(np.uint32))


def test_quantize_mxfp8_bitexact(gpu):
    import ds41_gfx950 as G
    say("quantize_mxfp8")
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((16, 4096)) * rng.choice([1e-7, 1e-3, 1, 50, 1e5], (16, 1))).astype(np.float32)
    x[0, :64] = 0
    x[1, :32] = 448 * 8
    x[2, 3] = -0.0
    bits = O.bf16_bits(x)
    q, s = G.quantize_mxfp8(dev(bits, gpu))
    qr, sr = O.quantize_mxfp8(bits)
    assert np.array_equal(host(s), sr)
    assert np.array_equal(host(q), qr)
    # every finite bf16 magnitude once
    allv = (np.arange(0, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    allv = allv[: len(allv) // 32 * 32].reshape(-1, 32) * np.where(np.arange(32) % 2, 1, -1).astype(np.float32)
    bits = O.bf16_bits(allv.astype(np.float32))
    q, s = G.quantize_mxfp8(dev(bits, gpu))
    qr, sr = O.quantize_mxfp8(bits)
    assert np.array_equal(host(s), sr) and np.array_equal(host(q), qr)


def test_e4m3_hardware_converter_exact(gpu):
    """The quantisers convert with the device's E4M3 instruction; it must round exactly as the
    integer formulation of OCP E4M3 (nearest even, saturating) on every fp32 in [-448, 448],
    every value the clamped quantisers hand it (ds41_e4m3_converter_check, ~2.3e9 inputs, both
    byte positions of the packed form)."""
    import ctypes
    import torch
    import ds41_gfx950 as G
    say("e4m3 converter, every fp32 in [-448, 448]")
    bad = torch.zeros(1, dtype=torch.int64, device=gpu)
    assert G.lib().ds41_e4m3_converter_check(ctypes.c_void_p(bad.data_ptr()), None) == 0
    torch.cuda.synchronize()
    assert int(bad.item()) == 0


@pytest.mark.parametrize("m,n,k", [(1, 512, 1024), (1, 1024, 512), (4, 2880, 4096), (4, 4096, 2880),
                                   (8, 100, 96), (3, 17, 32), (5, 64, 160), (11, 48, 256)])
def test_raw_projection_vs_oracle(gpu, m, n, k):
    import ds41_gfx950 as G
    say(f"raw projection m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 7 + n + k)
    w, ws = rand_mx(rng, n, k)
    xq, xs = O.quantize_mxfp8(rand_x(rng, m, k))
    got = host(G.mxfp4_raw(dev(w, gpu), dev(ws, gpu), dev(xq, gpu), dev(xs, gpu), m, n, k))
    acc, ref = O.mxfp4_gemm(w, ws, xq, xs, m, n, k)
    err = rel_l2(O.bf16_to_f32(got), O.bf16_to_f32(ref))
    say(f"  rel-L2 vs oracle (bf16 boundary) {err:.3e}, bf16 exact {np.mean(got == ref):.4f}")
    assert err <= 1e-3
    assert np.mean(got == ref) > 0.97  # differences are last-place bf16 rounding flips


def test_grouped_jobs_all_projections_and_alignment(gpu):
    import torch
    import ds41_gfx950 as G
    say("grouped jobs")
    rng = np.random.default_rng(3)
    H, I, E = 512, 256, 5
    experts_np, experts_dev = [], []
    keep = []
    for e in range(E):
        g, gs = rand_mx(rng, I, H)
        u, us = rand_mx(rng, I, H)
        d, ds = rand_mx(rng, H, I)
        experts_np.append(dict(gate=g, gate_scale=gs, up=u, up_scale=us, down=d, down_scale=ds))
        ed = {}
        for name, arr in experts_np[-1].items():
            t = dev(arr, gpu)
            if e == 2 and name in ("gate", "down"):  # 8-byte aligned weight plane
                buf = torch.empty(arr.size + 8, dtype=torch.uint8, device=gpu)
                buf[8:].copy_(t.view(-1))
                keep.append(buf)
                t = buf[8:]
            keep.append(t)
            ed[name] = t
        experts_dev.append(ed)
    table, _ = G.device_table(experts_dev, gpu)
    tokens = [1, 3, 8, 2, 5]
    for proj, (n, k) in ((0, (I, H)), (1, (I, H)), (2, (H, I))):
        xs_np, outs, jobs = [], [], []
        for e in range(E):
            xq, xsc = O.quantize_mxfp8(rand_x(rng, tokens[e], k))
            xd, xsd = dev(xq, gpu), dev(xsc, gpu)
            out = torch.empty((tokens[e], n), dtype=torch.bfloat16, device=gpu)
            keep += [xd, xsd]
            xs_np.append((xq, xsc))
            outs.append(out)
            jobs.append((e, tokens[e], xd, xsd, out))
        jd = G.device_jobs(jobs, gpu)
        G.grouped(table, jd, E, proj, n, k, entry="ds41_xk_grouped_v1")
        torch.cuda.synchronize()
        key = ("gate", "up", "down")[proj]
        for e in range(E):
            acc, ref = O.mxfp4_gemm(experts_np[e][key], experts_np[e][key + "_scale"], xs_np[e][0], xs_np[e][1],
                                    tokens[e], n, k)
            got = host(outs[e])
            assert rel_l2(O.bf16_to_f32(got), O.bf16_to_f32(ref)) <= 1e-3, (proj, e)
    assert G.take_status() == 0
    assert G.lib().ds41_xk_projection_abi_version() == 1


def test_swiglu_vs_oracle(gpu):
    import ds41_gfx950 as G
    say("swiglu")
    rng = np.random.default_rng(4)
    g = O.bf16_bits((rng.standard_normal((24, 2880)) * 6).astype(np.float32))
    u = O.bf16_bits((rng.standard_normal((24, 2880)) * 6).astype(np.float32))
    w = rng.random(24).astype(np.float32)
    got = host(G.swiglu(dev(g, gpu), dev(u, gpu), dev(w, gpu), 10.0))
    ref = O.swiglu(g, u, w, 10.0)
    d = np.abs(O.bf16_to_f32(got) - O.bf16_to_f32(ref))
    say(f"  exact {np.mean(d == 0):.5f}")
    assert np.mean(d == 0) > 0.999  # expf may differ in the last fp32 place
    assert np.all(d <= np.abs(O.bf16_to_f32(ref)) * 2 ** -7 + 1e-30)


def test_reduce_bitexact(gpu):
    import ds41_gfx950 as G
    say("reduce_experts")
    rng = np.random.default_rng(5)
    rows, k, h = 4, 6, 4096
    routed = O.bf16_bits((rng.standard_normal((rows, k, h)) * 10.0 ** rng.integers(-2, 3, (rows, k, 1))).astype(np.float32))
    shared = O.bf16_bits(rng.standard_normal((rows, h)).astype(np.float32))
    ids = np.stack([rng.permutation(384)[:6] for _ in range(rows)]).astype(np.int32)
    got = host(G.reduce_experts(dev(routed, gpu), dev(ids, gpu), dev(shared, gpu)))
    assert np.array_equal(got, O.reduce_experts(routed, ids, shared))


def test_router_pieces_bitexact(gpu):
    import ds41_gfx950 as G
    say("router topk / weights / scores / logits")
    rng = np.random.default_rng(6)
    b = rng.standard_normal((8, 384)).astype(np.float32)
    b[:, rng.integers(0, 384, 50)] = b[0, 7]
    b[3] = np.round(b[3], 1)
    ids = host(G.router_topk(dev(b, gpu), 6))
    assert np.array_equal(ids, O.topk(b, 6))
    u = (rng.random((8, 384)) * 3).astype(np.float32)
    w = host(G.router_weights(dev(u, gpu), dev(ids, gpu), 1.5))
    assert np.array_equal(w, O.route_weights(u, ids, 1.5))
    z = (rng.standard_normal((8, 384)) * 8).astype(np.float32)
    z[0, :5] = [20.0, 20.5, -40, 0, 19.999]
    bias = (rng.standard_normal(384) * 0.1).astype(np.float32)
    gu, gb = G.router_scores(dev(z, gpu), dev(bias, gpu))
    ou, ob = O.router_scores(z, bias)
    ulp = np.abs(host(gu).view(np.int32) - ou.view(np.int32))
    say(f"  scores max ulp {ulp.max()}, exact {np.mean(ulp == 0):.4f}")
    assert ulp.max() <= 2
    x = rand_x(rng, 4, 4096)
    wg = (rng.standard_normal((384, 4096)) * 0.02).astype(np.float32)
    lg = host(G.router_logits(dev(x, gpu), dev(wg, gpu)))
    ref = O.router_logits(x, wg)
    assert np.max(np.abs(lg - ref)) <= 1e-5 * np.max(np.abs(ref))


def make_layer(gpu, rng_seed, H, I, E, T):
    """Random MXFP4 experts generated on the device (E routed + 1 shared at index E)."""
    import torch
    g = torch.Generator(device=gpu).manual_seed(rng_seed)

    def rnd(shape, lo, hi):
        return torch.randint(lo, hi, shape, dtype=torch.uint8, device=gpu, generator=g)

    P = dict(gate=rnd((E + 1, I, H // 2), 0, 256), gate_scale=rnd((E + 1, I, H // 32), 119, 124),
             up=rnd((E + 1, I, H // 2), 0, 256), up_scale=rnd((E + 1, I, H // 32), 119, 124),
             down=rnd((E + 1, H, I // 2), 0, 256), down_scale=rnd((E + 1, H, I // 32), 119, 124))
    experts = [{k: v[e] for k, v in P.items()} for e in range(E + 1)]
    return P, experts


def test_moe_layer_vs_oracle(gpu):
    import torch
    import ds41_gfx950 as G
    H, I, E, K, T = 4096, 2880, 384, 6, 4
    say(f"moe layer T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 11, H, I, E, T)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(12)
    x_np = rand_x(rng, T, H)
    wg_np = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias_np = np.zeros(E, np.float32)
    x, wg, bias = dev(x_np, gpu), dev(wg_np, gpu), dev(bias_np, gpu)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    ids = torch.empty((T, K), dtype=torch.int32, device=gpu)
    wts = torch.empty((T, K), dtype=torch.float32, device=gpu)
    logits = torch.empty((T, E), dtype=torch.float32, device=gpu)
    args = G.make_layer_args(x, wg, bias, table, 0, E, T, H, I, E, K, y, ws, ids_out=ids, weights_out=wts,
                             logits_out=logits)
    G.moe_layer(args)
    torch.cuda.synchronize()
    assert G.take_status() == 0
    lg, gids, gw, gy = host(logits), host(ids), host(wts), host(y)
    ref_logits = O.router_logits(x_np, wg_np)
    assert np.max(np.abs(lg - ref_logits)) <= 1e-5 * np.max(np.abs(ref_logits))
    u, b = O.router_scores(lg, bias_np)
    oids = O.topk(b, K)
    assert np.array_equal(gids, oids)
    # the route weights, bit for bit, from the device's own scores (the workspace holds the logits
    # [T][E] and then the scores [T][E], each 256-byte aligned): the fixed summation order leaves no
    # freedom; the scores themselves are within 2 ulp of the oracle's (test_router_pieces_bitexact)
    off_u = (T * E * 4 + 255) & ~255
    u_dev = ws[off_u:off_u + T * E * 4].cpu().numpy().view(np.float32).reshape(T, E)
    assert np.allclose(u_dev, u, rtol=4e-7, atol=0)
    assert np.array_equal(gw.view(np.uint32), O.route_weights(u_dev, gids, 1.5).view(np.uint32))
    plan = G.layer_plan(ws, T, H, I, E, K)
    assert plan == sorted(set(gids.ravel().tolist()))
    routed = sorted(set(gids.ravel().tolist()))
    experts_np = [None] * E
    for e in routed:
        experts_np[e] = {k: host(v) for k, v in experts[e].items()}
    shared_np = {k: host(v) for k, v in experts[E].items()}
    ref_y = O.moe_layer_routed(x_np, gids, gw, experts_np, shared_np, H, I)
    a, b = O.bf16_to_f32(gy), O.bf16_to_f32(ref_y)
    err = rel_l2(a, b)
    tok = [rel_l2(a[t], b[t]) for t in range(T)]
    say(f"  unique experts {len(routed)}, y rel-L2 {err:.3e}, per token max {max(tok):.3e}, "
        f"bf16 exact {np.mean(gy == ref_y):.4f}")
    assert err <= 1e-3
    assert max(tok) <= 1e-2  # every token, not only the whole tensor


def test_moe_layer_topk_ties_lower_id_first(gpu):
    """Eight experts with bit-identical router rows (identical scores) lead every token: the planner's
    top-6 must be the six lowest of them in ascending id (ties -> lower id, batch.inc:228-237)."""
    import torch
    import ds41_gfx950 as G
    H, I, E, K, T = 512, 256, 64, 6, 4
    P, experts = make_layer(gpu, 13, H, I, E, T)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(14)
    row = rand_x(rng, 1, H)
    x_np = np.repeat(row, T, axis=0)
    wg_np = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    tied = [2, 5, 9, 30, 31, 47, 50, 63]
    lead = (0.05 * np.sign(O.bf16_to_f32(row[0]))).astype(np.float32)
    wg_np[tied] = lead
    bias_np = np.zeros(E, np.float32)
    x, wg, bias = dev(x_np, gpu), dev(wg_np, gpu), dev(bias_np, gpu)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    ids = torch.empty((T, K), dtype=torch.int32, device=gpu)
    logits = torch.empty((T, E), dtype=torch.float32, device=gpu)
    G.moe_layer(G.make_layer_args(x, wg, bias, table, 0, E, T, H, I, E, K, y, ws, ids_out=ids, logits_out=logits))
    torch.cuda.synchronize()
    lg = host(logits)
    assert np.all(lg[:, tied] == lg[:, tied[:1]])  # identical rows give identical scores
    u, b = O.router_scores(lg, bias_np)
    assert np.array_equal(host(ids), O.topk(b, K))
    assert np.array_equal(host(ids), np.tile(np.array(tied[:K], np.int32), (T, 1)))


def test_layer_args_abi_pair_checked(gpu):
    """ds41_moe_layer_args from another build: a struct_bytes or abi_version this build does not
    know is rejected (hipErrorInvalidValue) and launches nothing, on both verify-layer entries; the
    same struct with this build's pair runs."""
    import ctypes
    import torch
    import ds41_gfx950 as G
    T, H, I, E, K = 2, 512, 256, 16, 4
    say(f"layer args abi pair T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 81, H, I, E, T)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(82)
    x = dev(rand_x(rng, T, H), gpu)
    wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
    bias = dev(np.zeros(E, np.float32), gpu)
    y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    a = G.make_layer_args(x, wg, bias, table, 0, E, T, H, I, E, K, y, ws)
    for version, size in ((G.ABI_VERSION + 1, ctypes.sizeof(G.MoeLayerArgs)),
                          (G.ABI_VERSION, ctypes.sizeof(G.MoeLayerArgs) - 8), (0, 0)):
        a.abi_version, a.struct_bytes = version, size
        assert G.lib().ds41_moe_verify_layer(ctypes.byref(a), G._stream()) == 1
        assert G.moe_layer_noalloc_rc(a) == 1
    torch.cuda.synchronize()
    assert np.all(np.isnan(O.bf16_to_f32(host(y))))  # nothing ran
    a.abi_version, a.struct_bytes = G.ABI_VERSION, ctypes.sizeof(G.MoeLayerArgs)
    G.moe_layer(a)
    torch.cuda.synchronize()
    assert G.take_status() == 0
    assert not np.any(np.isnan(O.bf16_to_f32(host(y))))
