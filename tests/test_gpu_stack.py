"""Verify step through a stack of MoE layers with a pinned-host expert tier
(ds41_verify_stack_*), through the C ABI.

The host tier changes where a routed expert's bytes come from (a staging slot
filled by hipMemcpyAsync instead of its HBM slab), never the arithmetic: the
same step with every expert resident must give bit-identical outputs, ids and
weights. Each layer's output is also checked against the oracle's MoE layer
(rel-L2 1e-3) given the layer's input and routing."""
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
FIELDS = ("gate", "gate_scale", "up", "up_scale", "down", "down_scale")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def host(t):
    import torch
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.sum((a - b) ** 2) / max(np.sum(b ** 2), 1e-300)))


def shapes(H, I):
    return [(I, H // 2), (I, H // 32), (I, H // 2), (I, H // 32), (H, I // 2), (H, I // 32)]


class Stack:
    """L layers of E routed + 1 shared expert (index E) in canonical slabs on the device; `host_sets[l]`
    lists the routed ids of layer l that live only in pinned host slabs for the tiered stack."""

    def __init__(self, gpu, seed, L, H, I, E, K, Tmax, host_sets):
        import torch
        import ds41_gfx950 as G
        self.L, self.H, self.I, self.E, self.K = L, H, I, E, K
        self.off, self.slab = G.slab_layout(H, I)
        g = torch.Generator(device=gpu).manual_seed(seed)
        rng = np.random.default_rng(seed)
        self.slabs, self.layers_all, self.layers_tier, self.keep = [], [], [], []
        for l in range(L):
            s = torch.randint(0, 256, (E + 1, self.slab), dtype=torch.uint8, device=gpu, generator=g)
            for i in (1, 3, 5):
                n = shapes(H, I)[i][0] * shapes(H, I)[i][1]
                s[:, self.off[i]:self.off[i] + n].random_(119, 124, generator=g)
            self.slabs.append(s)
            entries = [G.slab_entry(s[e].data_ptr(), self.off, e) for e in range(E + 1)]
            table_all = torch.frombuffer(bytearray(b"".join(bytes(e) for e in entries)), dtype=torch.uint8).to(gpu)
            hs = list(host_sets[l])
            hidx = np.full(E, -1, np.int32)
            hidx[hs] = np.arange(len(hs), dtype=np.int32)
            tier_entries = [G.DeviceExpert() if e in hs else entries[e] for e in range(E + 1)]  # never read
            table_tier = torch.frombuffer(bytearray(b"".join(bytes(e) for e in tier_entries)),
                                          dtype=torch.uint8).to(gpu)
            pinned = torch.empty((max(len(hs), 1), self.slab), dtype=torch.uint8, pin_memory=True)
            if hs:
                pinned[:len(hs)].copy_(s[hs].cpu())
            wg = torch.from_numpy((rng.standard_normal((E, H)) * 0.02).astype(np.float32)).to(gpu)
            bias = torch.zeros(E, dtype=torch.float32, device=gpu)
            base = dict(router_w=wg, router_bias=bias, expert_base=0, shared_index=E)
            self.layers_all.append(dict(base, table=table_all))
            self.layers_tier.append(dict(base, table=table_tier, host_index=torch.from_numpy(hidx).to(gpu),
                                         host_slabs=pinned))
        self.host_sets = [set(h) for h in host_sets]
        self.tier = G.VerifyStack(self.layers_tier, Tmax, H, I, E, K, slab_bytes=self.slab)
        self.all = G.VerifyStack(self.layers_all, Tmax, H, I, E, K, slab_bytes=self.slab)

    def expert_np(self, l, e):
        s = self.slabs[l][e].cpu().numpy()
        return {f: s[o:o + a * b].reshape(a, b) for f, o, (a, b) in zip(FIELDS, self.off, shapes(self.H, self.I))}

    def run(self, which, x, route_ids=None):
        import torch
        T = x.shape[0]
        st = self.tier if which == "tier" else self.all
        y = torch.empty((T, self.H), dtype=torch.bfloat16, device=x.device)
        lo = torch.empty((self.L, T, self.H), dtype=torch.bfloat16, device=x.device)
        ids = torch.empty((self.L, T, self.K), dtype=torch.int32, device=x.device)
        w = torch.empty((self.L, T, self.K), dtype=torch.float32, device=x.device)
        st.step(x, y, route_ids=route_ids, layer_out=lo, ids_out=ids, weights_out=w)
        torch.cuda.synchronize()
        return host(y), host(lo), host(ids), host(w)


def rand_x(gpu, seed, T, H):
    import torch
    g = torch.Generator(device=gpu).manual_seed(seed)
    return torch.randn((T, H), generator=g, device=gpu, dtype=torch.float32).to(torch.bfloat16)


def check_same(a, b):
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))


def test_stack_host_tier_bitexact_vs_resident_router(gpu):
    import ds41_gfx950 as G
    L, H, I, E, K, T = 3, 512, 256, 32, 6, 4
    say(f"stack L={L} H={H} I={I} E={E} T={T}: host tier 8 experts/layer, router routing")
    st = Stack(gpu, 21, L, H, I, E, K, T, [range(3 * l, 3 * l + 8) for l in range(L)])
    x = rand_x(gpu, 5, T, H)
    G.take_status()  # clear bits left by earlier tests
    before = st.tier.stats()
    a = st.run("tier", x)
    b = st.run("all", x)
    check_same(a, b)
    assert G.take_status() == 0
    ids = a[2]
    fetched = sum(len(set(ids[l].ravel().tolist()) & st.host_sets[l]) for l in range(L))
    resident = sum(len(set(ids[l].ravel().tolist()) - st.host_sets[l]) for l in range(L))
    s = st.tier.stats()
    say(f"  host experts fetched {fetched}, resident routed {resident}, stats {s}")
    assert s["host_fetched"] - before["host_fetched"] == fetched and fetched > 0
    assert s["resident_routed"] - before["resident_routed"] == resident
    assert s["h2d_bytes"] - before["h2d_bytes"] == fetched * st.slab and s["invalid_layers"] == 0


@pytest.mark.parametrize("T", [1, 4, 8])
def test_stack_route_ids_reproduce_router_routes(gpu, T):
    """Given the route ids its router chose, a step plans beside the router and forms the route
    weights in the gate/up epilogue (the shared expert an ordinary gate/up job), not in a plan
    launch after the router: outputs, ids and weights must be bit-identical to the router-routed
    step, with and without the host tier. T = 8 plans two tokens per wave."""
    import torch
    import ds41_gfx950 as G
    L, H, I, E, K = 3, 1024, 256, 32, 6
    say(f"stack route ids = router routes L={L} H={H} I={I} E={E} T={T}")
    st = Stack(gpu, 31, L, H, I, E, K, 8, [range(3 * l, 3 * l + 8) for l in range(L)])
    x = rand_x(gpu, 12 + T, T, H)
    G.take_status()
    routed = st.run("all", x)
    rid = torch.from_numpy(np.ascontiguousarray(routed[2])).to(gpu)
    check_same(st.run("all", x, rid), routed)
    check_same(st.run("tier", x, rid), routed)
    assert G.take_status() == 0


def test_stack_layers_vs_oracle(gpu):
    L, H, I, E, K, T = 3, 512, 256, 32, 6, 4
    say(f"stack vs oracle L={L} H={H} I={I} E={E} T={T}")
    st = Stack(gpu, 22, L, H, I, E, K, T, [range(0, E, 4) for _ in range(L)])
    x = rand_x(gpu, 6, T, H)
    y, lo, ids, w = st.run("tier", x)
    xin = host(x)
    for l in range(L):
        out = y if l == L - 1 else lo[l]
        experts = [None] * E
        for e in sorted(set(ids[l].ravel().tolist())):
            experts[e] = st.expert_np(l, e)
        ref = O.moe_layer_routed(xin, ids[l], w[l], experts, st.expert_np(l, E), H, I)
        err = rel_l2(O.bf16_to_f32(out), O.bf16_to_f32(ref))
        say(f"  layer {l}: rel-L2 {err:.3e}, weights sum {w[l].sum(axis=1)}")
        assert err <= 1e-3
        assert np.allclose(w[l].sum(axis=1), 1.5, rtol=1e-5)
        for t in range(T):
            assert len(set(ids[l][t].tolist())) == K
        xin = out


def test_stack_route_ids_all_host(gpu):
    """Given ids that route every slot to a host-tier expert: up to T*K = 24 staging slots in one layer."""
    import torch
    L, H, I, E, K, T = 2, 512, 256, 32, 6, 4
    hosts = list(range(4, 28))
    st = Stack(gpu, 23, L, H, I, E, K, T, [hosts, hosts])
    rid = np.array([[hosts[t * K:(t + 1) * K] for t in range(T)], [hosts[::-1][t * K:(t + 1) * K] for t in range(T)]],
                   np.int32)
    say(f"stack route ids all-host: {len(hosts)} host-tier experts per layer")
    r = torch.from_numpy(rid).to(gpu)
    x = rand_x(gpu, 7, T, H)
    before = st.tier.stats()
    a = st.run("tier", x, r)
    b = st.run("all", x, r)
    check_same(a, b)
    assert np.array_equal(a[2], rid)
    s = st.tier.stats()
    assert s["host_fetched"] - before["host_fetched"] == 2 * len(hosts)
    assert s["resident_routed"] - before["resident_routed"] == 0


def test_stack_single_token_and_repeat(gpu):
    """T=1 and T=4 steps interleaved on one stack: staging reuse across steps and layers leaves no trace."""
    L, H, I, E, K = 4, 512, 256, 32, 6
    st = Stack(gpu, 24, L, H, I, E, K, 4, [range(l, E, 3) for l in range(L)])
    x4, x1 = rand_x(gpu, 8, 4, H), rand_x(gpu, 9, 1, H)
    first = st.run("tier", x4)
    one = st.run("tier", x1)
    again = st.run("tier", x4)
    check_same(first, again)
    check_same(one, st.run("all", x1))
    check_same(first, st.run("all", x4))


def test_stack_invalid_route_ids_give_nan(gpu):
    import torch
    import ds41_gfx950 as G
    L, H, I, E, K, T = 2, 512, 256, 32, 6, 2
    st = Stack(gpu, 25, L, H, I, E, K, T, [range(0, 8), range(8, 16)])
    rid = np.tile(np.arange(K, dtype=np.int32), (L, T, 1))
    rid[0, 1, 3] = rid[0, 1, 2]  # duplicate route in layer 0, token 1
    x = rand_x(gpu, 10, T, H)
    G.take_status()
    before = st.tier.stats()
    y, lo, _, w = st.run("tier", x, torch.from_numpy(rid).to(gpu))
    assert np.all(np.isnan(O.bf16_to_f32(lo[0])))
    # the rejected layer's weights are still each token's normalised scores times the route scale
    assert np.allclose(w[0].sum(axis=-1), 1.5, rtol=1e-5) and np.all(w[0] > 0)
    assert G.take_status() & 4
    assert st.tier.stats()["invalid_layers"] - before["invalid_layers"] == 1
    ok = st.run("tier", x)  # the stack recovers on the next step
    check_same(ok, st.run("all", x))


def test_stack_layer_entry_matches_step(gpu):
    """ds41_verify_stack_layer called layer by layer (as an engine with attention in between would)
    gives the step's bytes; y aliasing x is allowed."""
    import torch
    L, H, I, E, K, T = 3, 512, 256, 32, 6, 3
    st = Stack(gpu, 26, L, H, I, E, K, 4, [range(l, E, 5) for l in range(L)])
    x = rand_x(gpu, 11, T, H)
    y, lo, ids, w = st.run("tier", x)
    cur = x.clone()
    for l in range(L):
        i = torch.empty((T, K), dtype=torch.int32, device=gpu)
        st.tier.layer(l, cur, cur, ids_out=i)
        torch.cuda.synchronize()
        assert np.array_equal(host(i), ids[l])
        assert np.array_equal(host(cur).view(np.uint8), (y if l == L - 1 else lo[l]).view(np.uint8))


def host_demand(ids_l, host_set, l, E, model):
    """The host-tier experts of layer l in the order the stack hands them to its pool: the ones the
    cache already holds (the plan's HBM jobs), then the others, each ascending by expert id, as
    flattened ids l * E + e. `model` is a pool in the stack pool's state."""
    want = [l * E + e for e in sorted(set(ids_l.ravel().tolist()) & host_set)]
    return [f for f in want if model.residency(f) >= 0] + [f for f in want if model.residency(f) < 0]


@pytest.mark.parametrize("slots,budget", [(24, None), (40, (10, 18, 12))])
def test_stack_cache_bitexact_and_policy(gpu, slots, budget):
    """An HBM cache in front of the host tier (ds41_verify_stack_cache): over 10 steps with fresh
    host-heavy routes every output equals the all-resident stack's bit for bit, and the hits,
    misses and evictions equal those of the library's slot pool replaying the same demands."""
    import torch
    import ds41_gfx950 as G
    L, H, I, E, K, T = 3, 512, 256, 32, 6, 4
    host_sets = [range(l, E, 2) for l in range(L)]  # 16 host-tier experts per layer
    say(f"stack cache slots={slots} budget={budget} L={L} E={E} T={T}")
    st = Stack(gpu, 31, L, H, I, E, K, T, host_sets)
    placement = None
    if budget is not None:
        placement = G.make_placement(L, list(budget), recent=2, decay=4)
    st.tier.cache(slots, placement)
    model = G.ExpertPool(slots, [E] * L, recent=6 if placement is None else 2, decay=32 if placement is None else 4)
    if placement is not None:
        assert model.policy(placement) == 0
    rng = np.random.default_rng(32)
    hits = misses = evictions = 0
    G.take_status()
    for step in range(10):
        hs = [sorted(st.host_sets[l]) for l in range(L)]
        rid = np.empty((L, T, K), np.int32)
        for l in range(L):
            for t in range(T):  # mostly host-tier experts, some resident ones
                pool = hs[l][:10] if step % 2 else hs[l]
                n_host = int(rng.integers(3, 6))
                pick = list(rng.choice(pool, n_host, replace=False))
                rest = [e for e in range(E) if e not in st.host_sets[l]]
                pick += list(rng.choice(rest, K - n_host, replace=False))
                rid[l, t] = pick
        route = torch.from_numpy(rid).to(gpu)
        x = rand_x(gpu, 40 + step, T, H)
        a = st.run("tier", x, route)
        b = st.run("all", x, route)
        check_same(a, b)
        for l in range(L):
            want = host_demand(rid[l], st.host_sets[l], l, E, model)
            if not want:
                continue
            rc, got = model.acquire(want)
            assert rc == len(want)
            hits += sum(g[2] for g in got)
            misses += sum(not g[2] for g in got)
            evictions += sum(g[3] >= 0 for g in got)
            assert model.release(got) == 0
    assert G.take_status() == 0
    cs = st.tier.cache_stats()
    say(f"  cache {cs}")
    assert cs["hits"] == hits and cs["misses"] == misses and cs["evictions"] == evictions
    assert cs["requests"] == hits + misses and cs["h2d_bytes"] == misses * st.slab
    assert hits > 0 and evictions > 0
    ss = st.tier.stats()
    assert ss["cached_routed"] == hits  # every hit was found in the map by the plan (no prefetch here)


def random_routes(rng, st, L, T, K, E, step):
    rid = np.empty((L, T, K), np.int32)
    for l in range(L):
        hs = sorted(st.host_sets[l])
        for t in range(T):  # mostly host-tier experts, some resident ones
            pool = hs[:10] if step % 2 else hs
            n_host = int(rng.integers(3, 6))
            pick = list(rng.choice(pool, n_host, replace=False))
            rest = [e for e in range(E) if e not in st.host_sets[l]]
            pick += list(rng.choice(rest, K - n_host, replace=False))
            rid[l, t] = pick
    return rid


def test_stack_cache_prefetch_bitexact(gpu):
    """Prefetch (ds41_verify_stack_prefetch) of each step's routes into a small HBM cache before the
    step: every output equals the all-resident stack's bit for bit, every routed host-tier expert is
    served from the cache (found by its layer's plan, or a prefetch that landed after the plan:
    never a demand miss), and the prefetch copies and evictions equal the library's slot pool
    replaying the same prefetch-then-demand sequence."""
    import torch
    import ds41_gfx950 as G
    L, H, I, E, K, T, slots = 3, 512, 256, 32, 6, 4, 40
    say(f"stack cache + prefetch slots={slots} L={L} E={E} T={T}")
    st = Stack(gpu, 33, L, H, I, E, K, T, [range(l, E, 2) for l in range(L)])
    st.tier.cache(slots)
    model = G.ExpertPool(slots, [E] * L)
    rng = np.random.default_rng(34)
    copies = evictions = demand = 0
    G.take_status()
    c0, s0 = st.tier.cache_stats(), st.tier.stats()
    for step in range(10):
        rid = random_routes(rng, st, L, T, K, E, step)
        st.tier.prefetch_routes(rid)
        want = []  # the prefetch batch: per layer in order, first-seen host-tier ids
        for l in range(L):
            for e in rid[l].ravel().tolist():
                f = l * E + e
                if e in st.host_sets[l] and f not in want:
                    want.append(f)
        rc, pref = model.acquire(want, prefetch=True)
        assert rc == len(want)
        copies += sum(not g[2] for g in pref)
        evictions += sum(g[3] >= 0 for g in pref)
        route = torch.from_numpy(rid).to(gpu)
        x = rand_x(gpu, 60 + step, T, H)
        a = st.run("tier", x, route)
        b = st.run("all", x, route)
        check_same(a, b)
        for l in range(L):
            dem = host_demand(rid[l], st.host_sets[l], l, E, model)
            if dem:
                rc, got = model.acquire(dem)
                assert rc == len(dem) and all(g[2] for g in got)
                demand += len(dem)
                assert model.release(got) == 0
            assert model.release([g for g in pref if g[0] // E == l]) == 0
    assert G.take_status() == 0
    c1, s1 = st.tier.cache_stats(), st.tier.stats()
    d = {k: c1[k] - c0[k] for k in c1 if k != "slots"}
    say(f"  cache {d}")
    assert d["misses"] == 0 and d["hits"] == demand and d["requests"] == demand
    assert d["prefetch_copies"] == copies and d["evictions"] == evictions and evictions > 0
    assert d["h2d_bytes"] == copies * st.slab
    assert s1["cached_routed"] - s0["cached_routed"] == demand  # served from the cache, none copied on demand


def test_stack_prefetch_rejects_bad_pairs(gpu):
    L, H, I, E, K, T = 2, 512, 256, 32, 6, 4
    st = Stack(gpu, 35, L, H, I, E, K, T, [range(0, 8), range(8, 16)])
    assert st.tier.prefetch_rc([0], [1]) == 1  # no cache yet
    st.tier.cache(24)
    assert st.tier.prefetch_rc([2], [1]) == 1 and st.tier.prefetch_rc([0], [E]) == 1
    assert st.tier.prefetch_rc([0, 1], [20, 3]) == 0  # both HBM-resident: nothing to fetch
    many = list(range(0, 8)) + list(range(8, 16)) + list(range(0, 8))
    assert st.tier.prefetch_rc([0] * 8 + [1] * 8, many[:16]) == 0
    cs = st.tier.cache_stats()
    assert cs["prefetch_requests"] == 16 and cs["prefetch_copies"] == 16
    x = rand_x(gpu, 70, T, H)
    check_same(st.run("tier", x), st.run("all", x))  # leases end as the layers run
