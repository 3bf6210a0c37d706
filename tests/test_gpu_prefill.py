"""Chunked verify / prefill on the scaled MFMA (T >= 256 rows), through the C ABI:
the component GEMM (ds41_mxfp4_prefill_raw, ds41_grouped_mxfp4_prefill) and the
prefill MoE layer (ds41_moe_prefill_layer: device route plan, fused gate/up +
SwiGLU + MXFP8, down, ordered reduce) against the oracle.

Bar: MoE outputs within rel-L2 1e-3 of the oracle's fp32
accumulation; routing is the caller's, so the plan itself must be exact (every
token's rows summed in ascending expert id, shared expert last)."""
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


@pytest.mark.parametrize("m,n,k", [(256, 2880, 4096), (200, 4096, 2880), (1, 64, 32), (17, 100, 96),
                                   (64, 128, 256), (65, 64, 160), (130, 72, 544)])
def test_prefill_raw_vs_oracle(gpu, m, n, k):
    import ds41_gfx950 as G
    say(f"prefill raw m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 13 + n + k)
    w, ws = rand_mx(rng, n, k)
    xq, xs = O.quantize_mxfp8(rand_x(rng, m, k))
    got = host(G.prefill_raw(dev(w, gpu), dev(ws, gpu), dev(xq, gpu), dev(xs, gpu), m, n, k))
    acc, ref = O.mxfp4_gemm(w, ws, xq, xs, m, n, k)
    err = rel_l2(O.bf16_to_f32(got), O.bf16_to_f32(ref))
    say(f"  rel-L2 {err:.3e}, bf16 exact {np.mean(got == ref):.4f}")
    assert err <= 1e-3
    assert np.mean(got == ref) > 0.97


def test_prefill_raw_rejects_like_reference(gpu):
    import ctypes
    import ds41_gfx950 as G
    L = G.lib()
    assert L.ds41_mxfp4_prefill_raw(None, None, None, None, None, 257, 64, 256, None) == 1  # m > 256
    assert L.ds41_mxfp4_prefill_raw(None, None, None, None, None, 4, 64, 48, None) == 1     # k % 32
    assert L.ds41_grouped_mxfp4_prefill(None, None, 1, 0, 64, 256, 300, None) == 1        # max_tokens > 256
    del ctypes


def test_grouped_prefill_jobs(gpu):
    import torch
    import ds41_gfx950 as G
    say("grouped prefill jobs")
    rng = np.random.default_rng(31)
    H, I, E = 512, 256, 4
    experts_np, experts_dev, keep = [], [], []
    for e in range(E):
        g, gs = rand_mx(rng, I, H)
        u, us = rand_mx(rng, I, H)
        d, ds = rand_mx(rng, H, I)
        experts_np.append(dict(gate=g, gate_scale=gs, up=u, up_scale=us, down=d, down_scale=ds))
        ed = {k: dev(v, gpu) for k, v in experts_np[-1].items()}
        keep.append(ed)
        experts_dev.append(ed)
    table, _ = G.device_table(experts_dev, gpu)
    tokens = [256, 1, 97, 64]
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
        G.grouped_prefill(table, jd, E, proj, n, k, 256)
        torch.cuda.synchronize()
        key = ("gate", "up", "down")[proj]
        for e in range(E):
            acc, ref = O.mxfp4_gemm(experts_np[e][key], experts_np[e][key + "_scale"], xs_np[e][0], xs_np[e][1],
                                    tokens[e], n, k)
            assert rel_l2(O.bf16_to_f32(host(outs[e])), O.bf16_to_f32(ref)) <= 1e-3, (proj, e)
    assert G.take_status() == 0


def make_experts(gpu, seed, H, I, E):
    """E routed + 1 shared expert (index E) generated on the device."""
    import torch
    g = torch.Generator(device=gpu).manual_seed(seed)

    def rnd(shape, lo, hi):
        return torch.randint(lo, hi, shape, dtype=torch.uint8, device=gpu, generator=g)

    P = dict(gate=rnd((E + 1, I, H // 2), 0, 256), gate_scale=rnd((E + 1, I, H // 32), 119, 124),
             up=rnd((E + 1, I, H // 2), 0, 256), up_scale=rnd((E + 1, I, H // 32), 119, 124),
             down=rnd((E + 1, H, I // 2), 0, 256), down_scale=rnd((E + 1, H, I // 32), 119, 124))
    return P, [{k: v[e] for k, v in P.items()} for e in range(E + 1)]


def zipf_ids(rng, T, E, K, s=1.1, perm=None):
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    ids = np.stack([rng.choice(E, size=K, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    return ids if perm is None else perm[ids].astype(np.int32)


def run_prefill(gpu, experts, x_np, ids, w, H, I, E, K, shared=True):
    import torch
    import ds41_gfx950 as G
    T = x_np.shape[0]
    table, _ = G.device_table(experts, gpu)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.prefill_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    a = G.make_prefill_args(dev(x_np, gpu), dev(ids, gpu), dev(w, gpu), table, 0, E if shared else -1, T, H, I, E,
                            K, y, ws)
    G.moe_prefill(a)
    torch.cuda.synchronize()
    plan = G.prefill_plan_counts(ws, T, H, I, E, K)
    assert plan[0] == G.prefill_tiles(ws, T, H, I, E, K)
    return host(y), plan


def want_plan(counts, T):
    """The plan's split: 64-row tiles for experts with more than 8 rows and for the shared expert's T
    rows; GEMV jobs for the experts with 1..4 and with 5..8 rows."""
    big = counts[counts > 8]
    return (int(np.sum((big + 63) // 64)) + (T + 63) // 64, int(np.sum((counts >= 1) & (counts <= 4))),
            int(np.sum((counts >= 5) & (counts <= 8))))


def check_tokens(experts, x_np, ids, w, got, H, I, E, tokens):
    used = sorted(set(ids[tokens].ravel().tolist()))
    experts_np = [None] * E
    for e in used:
        experts_np[e] = {k: host(v) for k, v in experts[e].items()}
    shared_np = {k: host(v) for k, v in experts[E].items()}
    ref = O.moe_layer_routed(x_np[tokens], ids[tokens], w[tokens], experts_np, shared_np, H, I, threads=8)
    return rel_l2(O.bf16_to_f32(got[tokens]), O.bf16_to_f32(ref)), np.mean(got[tokens] == ref)


@pytest.mark.parametrize("T,E,skew", [(300, 32, "uniform"), (256, 32, "zipf"), (77, 64, "zipf"), (1, 8, "uniform"),
                                      (40, 32, "uniform"), (300, 1024, "zipf")])
def test_prefill_layer_vs_oracle(gpu, T, E, skew):
    """(300, 1024) takes the plan's key-sort path (5 groups x 1024 experts of token bitmaps exceed
    its LDS); the others its counting path."""
    import ds41_gfx950 as G
    H, I, K = 512, 256, 6
    say(f"prefill layer T={T} H={H} I={I} E={E} routing={skew}")
    P, experts = make_experts(gpu, 40 + T, H, I, E)
    rng = np.random.default_rng(41 + T)
    x_np = rand_x(rng, T, H)
    ids = (np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32) if skew == "uniform"
           else zipf_ids(rng, T, E, K))
    w = (rng.random((T, K)) + 0.1).astype(np.float32)
    w = (w / w.sum(axis=1, keepdims=True) * 1.5).astype(np.float32)
    G.take_status()
    got, tiles = run_prefill(gpu, experts, x_np, ids, w, H, I, E, K)
    counts = np.bincount(ids.ravel(), minlength=E)
    err, exact = check_tokens(experts, x_np, ids, w, got, H, I, E, np.arange(T))
    say(f"  rows per expert max {counts.max()}, plan (tiles, gemv<=4, gemv5-8) {tiles}, rel-L2 {err:.3e}, "
        f"bf16 exact {exact:.4f}")
    assert tiles == want_plan(counts, T)
    assert err <= 1e-3
    assert G.take_status() == 0


def test_prefill_layer_invalid_routes_nan(gpu):
    import ds41_gfx950 as G
    H, I, E, K, T = 512, 256, 16, 6, 40
    P, experts = make_experts(gpu, 50, H, I, E)
    rng = np.random.default_rng(51)
    x_np = rand_x(rng, T, H)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[7, 4] = ids[7, 1]
    w = np.full((T, K), 0.25, np.float32)
    G.take_status()
    got, tiles = run_prefill(gpu, experts, x_np, ids, w, H, I, E, K)
    assert tiles == (0, 0, 0) and np.all(np.isnan(O.bf16_to_f32(got)))
    assert G.take_status() & 4


def test_prefill_layer_config3_shape(gpu):
    """configs[3] shapes (T=512, H=4096, I=2880, 384 experts, Zipf(1.1) routing, so the hottest expert
    spans several 64-row tiles): all 512 tokens against the oracle."""
    import os
    import ds41_gfx950 as G
    H, I, E, K, T = 4096, 2880, 384, 6, 512
    say(f"prefill layer configs[3] T={T} H={H} I={I} E={E}")
    P, experts = make_experts(gpu, 60, H, I, E)
    rng = np.random.default_rng(61)
    x_np = rand_x(rng, T, H)
    ids = zipf_ids(rng, T, E, K, perm=rng.permutation(E))
    w = (rng.random((T, K)) + 0.1).astype(np.float32)
    w = (w / w.sum(axis=1, keepdims=True) * 1.5).astype(np.float32)
    G.take_status()
    got, tiles = run_prefill(gpu, experts, x_np, ids, w, H, I, E, K)
    counts = np.bincount(ids.ravel(), minlength=E)
    experts_np = [None] * E
    for e in np.nonzero(counts)[0]:
        experts_np[e] = {k: host(v) for k, v in experts[e].items()}
    shared_np = {k: host(v) for k, v in experts[E].items()}
    ref = O.moe_layer_routed(x_np, ids, w, experts_np, shared_np, H, I, threads=min(16, os.cpu_count() or 1))
    g, r = O.bf16_to_f32(got).astype(np.float64), O.bf16_to_f32(ref).astype(np.float64)
    err = rel_l2(g, r)
    per_token = np.sqrt(((g - r) ** 2).sum(1) / (r ** 2).sum(1))
    say(f"  unique experts {np.count_nonzero(counts)}, max rows {counts.max()}, tiles {tiles}, rel-L2 {err:.3e}, "
        f"bf16 exact {np.mean(got == ref):.4f}, per-token rel-L2 median {np.median(per_token):.2e} max "
        f"{per_token.max():.2e}")
    assert tiles == want_plan(counts, T)
    assert err <= 1e-3
    assert per_token.max() <= 1e-2  # every token, not only the whole tensor
    assert G.take_status() == 0


def test_prefill_matches_decode_layer_bitexact(gpu):
    """Given the decode layer's own routing, the prefill layer runs the same MFMA sequence per row (K
    order, fresh accumulators, same epilogue arithmetic), so its output must equal the decode layer's
    bit for bit at the configs[1] shapes."""
    import torch
    import ds41_gfx950 as G
    H, I, E, K, T = 4096, 2880, 384, 6, 4
    P, experts = make_experts(gpu, 70, H, I, E)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(71)
    x_np = rand_x(rng, T, H)
    wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
    bias = dev(np.zeros(E, np.float32), gpu)
    x = dev(x_np, gpu)
    y_dec = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    ids = torch.empty((T, K), dtype=torch.int32, device=gpu)
    wts = torch.empty((T, K), dtype=torch.float32, device=gpu)
    G.moe_layer(G.make_layer_args(x, wg, bias, table, 0, E, T, H, I, E, K, y_dec, ws, ids_out=ids, weights_out=wts))
    torch.cuda.synchronize()
    got, tiles = run_prefill(gpu, experts, x_np, host(ids), host(wts), H, I, E, K)
    dec = host(y_dec)
    say(f"  prefill vs decode: bit-identical {np.mean(got == dec):.5f}, tiles {tiles}")
    assert np.array_equal(got, dec)


@pytest.mark.parametrize("H,I,E,T", [(4096, 2880, 64, 256), (576, 352, 16, 96)])
def test_prefill_tiles_match_gemv_bitexact(gpu, H, I, E, T):
    """Each token's output depends only on its own routes, and a tile row runs the decode GEMV's MFMA
    sequence (chunks in ascending k, the magnitude halves into separate accumulators), so the layer
    over all T tokens (experts with > 8 rows in 64-row tiles) must equal, bit for bit, the layer run
    4 tokens at a time (every routed expert a GEMV job). H=576, I=352 cover partial K chunks and
    slices, byte-wise scale loads and half-empty channel blocks."""
    import ds41_gfx950 as G
    K = 6
    say(f"prefill tiles vs GEMV T={T} H={H} I={I} E={E}")
    P, experts = make_experts(gpu, 80 + H, H, I, E)
    rng = np.random.default_rng(81 + H)
    x_np = rand_x(rng, T, H)
    ids = zipf_ids(rng, T, E, K, perm=rng.permutation(E))
    w = (rng.random((T, K)) + 0.1).astype(np.float32)
    w = (w / w.sum(axis=1, keepdims=True) * 1.5).astype(np.float32)
    G.take_status()
    full, plan = run_prefill(gpu, experts, x_np, ids, w, H, I, E, K)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert plan == want_plan(counts, T) and plan[0] > (T + 63) // 64, plan
    parts = []
    for t0 in range(0, T, 4):
        got, p4 = run_prefill(gpu, experts, x_np[t0:t0 + 4], ids[t0:t0 + 4], w[t0:t0 + 4], H, I, E, K)
        assert p4[0] == 1  # only the shared expert's tile
        parts.append(got)
    chunked = np.concatenate(parts)
    same = np.mean(full == chunked)
    say(f"  plan {plan}, max rows {counts.max()}, bit-identical {same:.5f}")
    assert np.array_equal(full, chunked)
    assert G.take_status() == 0
