"""GPU parity of the MTP drafter's routed-expert service (ds41_target_experts, the
ds41_target_experts_fn of engine/include/ds41/target_shared.h:28-39 as routed_spark,
engine/src/forward.cu:1000-1097, serves it) and of the drafter's router top-3
(ds41_spark_topk3_gpu, spark forward.cu:28-40), through the C ABI.

Bars: top-3 ids bit-exact against the oracle (every input, NaN and signed zero included);
the whole [rows][3][H] output within rel-L2 1e-3 of the oracle's expert FFN on the same
MXFP8 rows and route weights (the MoE-layer bar), and every single slot within 5e-3: the
GPU's gate/up sums run in another order than the oracle's, so a BF16 gate/up value can
round the other way and move one MXFP8 activation code by one step (1/8 relative), which
alone costs one slot about 0.125 / sqrt(I) = 2.6e-3; a layer output sums 7 slots and
averages such steps out. Rejected routes and bad arguments fail as documented."""
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

H, I, NE = 5120, 2304, 128
DISTINCT = 12  # physical experts behind the 3 x 128 table entries


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


def phys(stage, e):
    return (7 * e + 5 * stage) % DISTINCT


_cache = {}


def drafter_table(gpu):
    """3 stages x 128 table entries (base 16) over DISTINCT random MXFP4 experts."""
    if "t" in _cache:
        return _cache["t"]
    import torch
    import ds41_gfx950 as G
    g = torch.Generator(device=gpu).manual_seed(77)

    def rnd(shape, lo, hi):
        return torch.randint(lo, hi, shape, dtype=torch.uint8, device=gpu, generator=g)

    P = dict(gate=rnd((DISTINCT, I, H // 2), 0, 256), gate_scale=rnd((DISTINCT, I, H // 32), 119, 124),
             up=rnd((DISTINCT, I, H // 2), 0, 256), up_scale=rnd((DISTINCT, I, H // 32), 119, 124),
             down=rnd((DISTINCT, H, I // 2), 0, 256), down_scale=rnd((DISTINCT, H, I // 32), 119, 124))
    ex = [{k: v[d] for k, v in P.items()} for d in range(DISTINCT)]
    entries = [None] * 16 + [ex[phys(s, e)] for s in range(3) for e in range(NE)]
    table, _ = G.device_table(entries, gpu)
    ex_np = [{k: host(v) for k, v in e.items()} for e in ex]
    _cache["t"] = (table, ex_np, P)
    return _cache["t"]


def run_case(gpu, svc, stage, x_np, ids_np, w_np):
    import torch
    rows = x_np.shape[0]
    out = torch.full((rows, 3, H), float("nan"), dtype=torch.bfloat16, device=gpu)
    svc(stage, dev(x_np, gpu), dev(ids_np, gpu), dev(w_np, gpu), out)
    torch.cuda.synchronize()
    return host(out)


def check_slots(ex_np, stage, x_np, ids_np, w_np, got):
    xq, xs = O.quantize_mxfp8(x_np)
    rows = x_np.shape[0]
    worst = 0.0
    want = np.zeros_like(got)
    by_expert = {}
    for r in range(rows):
        for k in range(3):
            by_expert.setdefault(int(ids_np[r, k]), []).append((r, k))
    for e, slots in by_expert.items():
        rr = np.array([r for r, _ in slots])
        wv = np.array([w_np[r, k] for r, k in slots], np.float32)
        ref = O.expert_ffn(ex_np[phys(stage, e)], xq[rr], xs[rr], wv, H, I, 10.0)
        for j, (r, k) in enumerate(slots):
            want[r, k] = ref[j]
            err = rel_l2(O.bf16_to_f32(got[r, k]), O.bf16_to_f32(ref[j]))
            worst = max(worst, err)
            assert err <= 5e-3, (stage, r, k, e, err)
    total = rel_l2(O.bf16_to_f32(got), O.bf16_to_f32(want))
    say(f"  output rel-L2 {total:.3e}, worst slot {worst:.3e}, bf16 exact {np.mean(got == want):.4f}")
    assert total <= 1e-3
    return worst


@pytest.mark.parametrize("rows,stage,pattern", [(1, 0, "fixture"), (3, 1, "fixture"), (5, 2, "random"),
                                                (8, 0, "random"), (5, 1, "shared")])
def test_target_experts_vs_oracle(gpu, rows, stage, pattern):
    import ds41_gfx950 as G
    O.set_threads(8)
    table, ex_np, _ = drafter_table(gpu)
    say(f"target experts rows={rows} stage={stage} ids={pattern}")
    svc = G.TargetExperts(table, 16, H, I)
    rng = np.random.default_rng(100 + 10 * rows + stage)
    x_np = O.bf16_bits(rng.standard_normal((rows, H)).astype(np.float32))
    if pattern == "fixture":  # the reference's service test routes (native_services.cpp:130-135)
        known = 17 + 40 * stage
        ids_np = np.array([[(known + (k + 3 - r % 3) % 3) % NE for k in range(3)] for r in range(rows)], np.int32)
    elif pattern == "shared":  # every row routes to the same three experts, in different slot orders
        base = np.array([5, 77, 120], np.int32)
        ids_np = np.stack([np.roll(base, r) for r in range(rows)]).astype(np.int32)
    else:
        ids_np = np.stack([rng.choice(NE, 3, replace=False) for _ in range(rows)]).astype(np.int32)
    w_np = rng.uniform(0.05, 1.2, (rows, 3)).astype(np.float32)
    got = run_case(gpu, svc, stage, x_np, ids_np, w_np)
    assert G.take_status() == 0
    assert not np.any(np.isnan(O.bf16_to_f32(got)))
    check_slots(ex_np, stage, x_np, ids_np, w_np, got)
    # a second call with fewer rows on the same handle: the workspace is recarved per call
    got2 = run_case(gpu, svc, stage, x_np[:1], ids_np[:1], w_np[:1])
    assert np.array_equal(got2[0], got[0])
    svc.close()


def test_target_experts_rejects_routes_on_device(gpu):
    """check_routes = 0: a duplicate or out-of-range id gives NaN in every slot and status bit 4,
    without a host wait; the next valid call is unaffected."""
    import ds41_gfx950 as G
    table, ex_np, _ = drafter_table(gpu)
    svc = G.TargetExperts(table, 16, H, I)
    rng = np.random.default_rng(5)
    x_np = O.bf16_bits(rng.standard_normal((2, H)).astype(np.float32))
    w_np = np.full((2, 3), 0.5, np.float32)
    G.take_status()
    for bad in ([[1, 2, 3], [4, 4, 5]], [[1, 2, 128], [3, 4, 5]], [[-1, 2, 3], [3, 4, 5]]):
        got = run_case(gpu, svc, 0, x_np, np.array(bad, np.int32), w_np)
        assert np.all(np.isnan(O.bf16_to_f32(got))), bad
        assert G.take_status() & 4
    ids_np = np.array([[1, 2, 3], [4, 6, 5]], np.int32)
    got = run_case(gpu, svc, 0, x_np, ids_np, w_np)
    assert G.take_status() == 0
    check_slots(ex_np, 0, x_np, ids_np, w_np, got)


def test_target_experts_host_checks_and_poison(gpu):
    """check_routes = 1 rejects a duplicate route on the host (the reference's behaviour); bad
    arguments and the wrong stream fail; any failure poisons the handle (forward.cu:984-998)."""
    import torch
    import ds41_gfx950 as G
    table, _, _ = drafter_table(gpu)
    rng = np.random.default_rng(6)
    x = dev(O.bf16_bits(rng.standard_normal((2, H)).astype(np.float32)), gpu)
    w = torch.full((2, 3), 0.5, dtype=torch.float32, device=gpu)
    out = torch.empty((2, 3, H), dtype=torch.bfloat16, device=gpu)
    good = torch.tensor([[1, 2, 3], [4, 5, 6]], dtype=torch.int32, device=gpu)
    dup = torch.tensor([[1, 2, 3], [4, 4, 6]], dtype=torch.int32, device=gpu)
    svc = G.TargetExperts(table, 16, H, I, check_routes=True)
    assert svc.call_rc(0, x, good, w, out) == 0 and svc.error() == ""
    assert svc.call_rc(0, x, dup, w, out) == -1 and "duplicate" in svc.error()
    assert svc.call_rc(0, x, good, w, out) == -1 and "poisoned" in svc.error()
    for stage, rows in ((3, 2), (-1, 2), (0, 0), (0, 9)):
        s2 = G.TargetExperts(table, 16, H, I)
        assert s2.call_rc(stage, x, good, w, out, rows=rows) == -1 and "arguments" in s2.error()
        s2.close()
    other = torch.cuda.Stream()
    s3 = G.TargetExperts(table, 16, H, I, stream=other)
    assert s3.call_rc(0, x, good, w, out, stream=torch.cuda.current_stream()) == -1 and "stream" in s3.error()
    torch.cuda.synchronize()


def topk3_inputs():
    rng = np.random.default_rng(9)
    cases = {}
    cases["distinct"] = rng.standard_normal((8, NE)).astype(np.float32)
    cases["small_ints"] = rng.integers(0, 3, (8, NE)).astype(np.float32)
    cases["all_equal"] = np.full((4, NE), 0.25, np.float32)
    z = rng.integers(0, 2, (6, NE)).astype(np.float32)
    z[z == 0] = -0.0
    z[:, ::7] = 0.0
    cases["signed_zero"] = np.where(rng.random((6, NE)) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
    cases["zero_one"] = z
    nan = rng.standard_normal((8, NE)).astype(np.float32)
    nan[0, 0] = np.nan
    nan[1, [0, 1, 2]] = np.nan
    nan[2, 5:60] = np.nan
    nan[3, :] = np.nan
    nan[4, 1] = np.nan
    nan[5, [0, 1]] = np.nan
    nan[6, 64] = np.nan
    nan[7, 127] = np.inf
    cases["nan_inf"] = nan
    pair = np.zeros((3, NE), np.float32)
    pair[:, 10] = pair[:, 20] = 5.0
    pair[:, 30] = 1.0
    cases["tied_pair"] = pair
    cases["router_like"] = (np.sqrt(np.log1p(np.exp(rng.standard_normal((5, NE)))))
                            + rng.choice([0.0, 0.01, 0.02], (5, NE))).astype(np.float32)
    return cases


@pytest.mark.parametrize("name", sorted(topk3_inputs()))
def test_spark_topk3_vs_oracle(gpu, name):
    import ds41_gfx950 as G
    s = topk3_inputs()[name]
    for m in sorted({1, 2, s.shape[0]}):
        sub = np.ascontiguousarray(s[:m])
        got = host(G.spark_topk3(dev(sub, gpu)))
        want = O.spark_topk3(sub)
        assert np.array_equal(got, want), (name, m, got.tolist(), want.tolist())


def tiled_drafter_table(gpu):
    """The same DISTINCT experts as drafter_table, as canonical slabs tiled by ds41_expert_slab_tile,
    behind the same 3 x 128 entries."""
    if "tiled" in _cache:
        return _cache["tiled"]
    import torch
    import ds41_gfx950 as G
    _, _, P = drafter_table(gpu)
    off, slab = G.slab_layout(H, I)
    src = torch.zeros((DISTINCT, slab), dtype=torch.uint8, device=gpu)
    for d in range(DISTINCT):
        for name, o in zip(("gate", "gate_scale", "up", "up_scale", "down", "down_scale"), off):
            t = P[name][d].reshape(-1)
            src[d, o:o + t.numel()] = t
    dst = torch.empty_like(src)
    G.slab_tile(src, dst, H, I, DISTINCT)
    entries = [G.DeviceExpert() for _ in range(16)] + [G.slab_entry(dst[phys(s, e)].data_ptr(), off)
                                                      for s in range(3) for e in range(NE)]
    table = torch.frombuffer(bytearray(b"".join(bytes(e) for e in entries)), dtype=torch.uint8).to(gpu)
    _cache["tiled"] = (table, src, dst)
    return _cache["tiled"]


@pytest.mark.parametrize("rows,stage", [(1, 2), (5, 0), (8, 1)])
def test_target_experts_tiled_weights_bitexact(gpu, rows, stage):
    """weight_layout = 1 over tiled slabs gives the row-major service's output bit for bit."""
    import ds41_gfx950 as G
    table, _, _ = drafter_table(gpu)
    ttable, _, _ = tiled_drafter_table(gpu)
    say(f"target experts tiled vs row-major rows={rows} stage={stage}")
    rng = np.random.default_rng(300 + 10 * rows + stage)
    x_np = O.bf16_bits(rng.standard_normal((rows, H)).astype(np.float32))
    ids_np = np.stack([rng.choice(NE, 3, replace=False) for _ in range(rows)]).astype(np.int32)
    w_np = rng.uniform(0.05, 1.2, (rows, 3)).astype(np.float32)
    svc = G.TargetExperts(table, 16, H, I)
    tsvc = G.TargetExperts(ttable, 16, H, I, weight_layout=1)
    want = run_case(gpu, svc, stage, x_np, ids_np, w_np)
    got = run_case(gpu, tsvc, stage, x_np, ids_np, w_np)
    assert G.take_status() == 0
    assert not np.any(np.isnan(O.bf16_to_f32(got)))
    assert np.array_equal(got, want)
    svc.close()
    tsvc.close()
