"""configs[4]'s layer shape through the verify stack (ds41_verify_stack_*), through the C ABI: T=4,
H=4096, I=2880, 384 routed experts top-6 + 1 shared, 18,800,640-byte canonical slabs. Per layer
the Zipf(1.1)-hottest 320 experts (ranks of a seeded permutation) and the shared expert sit in HBM
and the other 64 in pinned host memory (hipHostMalloc'd by torch), as the bench's 40-layer stack
has them; three layers here.

Bars:
- outputs, ids and weights bit-identical to the same stack with every expert resident, for router
  routing and for Zipf(1.1)-drawn ids, without a cache and with an HBM cache fed by prefetches
  (the host tier moves bytes, never arithmetic);
- each layer within rel-L2 1e-3 of oracle.moe_layer_routed given its input and routing, and every
  token within rel-L2 1e-2 (one moved MXFP8 activation code costs a token about 0.125/sqrt(I), so
  a token's error is a few such steps at most)."""
import numpy as np
import pytest

import oracle as O
from test_gpu_stack import Stack, check_same, host, rand_x, rel_l2, say

pytestmark = pytest.mark.gpu

L, T, H, I, E, K, RES = 3, 4, 4096, 2880, 384, 6, 320


def zipf_ids(rng, perm, s=1.1):
    """T tokens x K distinct experts, ranks drawn from Zipf(s) over 1..E (Gumbel top-K of log p)."""
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    out = np.empty((T, K), np.int32)
    for t in range(T):
        ranks = np.argsort(-(logp + rng.gumbel(size=E)))[:K]
        out[t] = perm[ranks]
    return out


@pytest.fixture(scope="module")
def stack4(gpu):
    perms = [np.random.default_rng([81, l]).permutation(E) for l in range(L)]
    host_sets = [sorted(p[RES:].tolist()) for p in perms]  # Zipf ranks 321..384
    say(f"configs[4] layer shape: L={L} T={T} H={H} I={I} E={E}, {RES}+1 resident, {E - RES} host per layer")
    st = Stack(gpu, 80, L, H, I, E, K, T, host_sets)
    return st, perms


def oracle_check(st, x, res):
    y, lo, ids, w = res
    xin = host(x)
    for l in range(L):
        out = y if l == L - 1 else lo[l]
        experts = [None] * E
        for e in sorted(set(ids[l].ravel().tolist())):
            experts[e] = st.expert_np(l, e)
        ref = O.moe_layer_routed(xin, ids[l], w[l], experts, st.expert_np(l, E), H, I)
        a, b = O.bf16_to_f32(out), O.bf16_to_f32(ref)
        err = rel_l2(a, b)
        tok = [rel_l2(a[t], b[t]) for t in range(T)]
        n_host = len(set(ids[l].ravel().tolist()) & st.host_sets[l])
        say(f"  layer {l}: rel-L2 {err:.3e}, per token max {max(tok):.3e}, host-tier experts routed {n_host}")
        assert err <= 1e-3
        assert max(tok) <= 1e-2
        xin = out


def test_config4_shape_router_routing(gpu, stack4):
    import ds41_gfx950 as G
    st, _ = stack4
    x = rand_x(gpu, 82, T, H)
    G.take_status()
    before = st.tier.stats()
    a = st.run("tier", x)
    b = st.run("all", x)
    check_same(a, b)
    assert G.take_status() == 0
    fetched = sum(len(set(a[2][l].ravel().tolist()) & st.host_sets[l]) for l in range(L))
    s = st.tier.stats()
    say(f"  router routing: host-tier experts copied {s['host_fetched'] - before['host_fetched']} (routed {fetched})")
    assert s["host_fetched"] - before["host_fetched"] == fetched
    oracle_check(st, x, a)


def test_config4_shape_zipf_ids(gpu, stack4):
    import torch
    import ds41_gfx950 as G
    st, perms = stack4
    rng = np.random.default_rng(83)
    for rep in range(2):
        rid = np.stack([zipf_ids(rng, perms[l]) for l in range(L)])
        rid[:, 0, 0] = [perms[l][RES + 3 * rep + l] for l in range(L)]  # at least one host-tier expert per layer
        for l in range(L):
            assert len(set(rid[l, 0].tolist())) == K, "forced id repeated another route of the token"
        route = torch.from_numpy(rid).to(gpu)
        x = rand_x(gpu, 84 + rep, T, H)
        a = st.run("tier", x, route)
        b = st.run("all", x, route)
        check_same(a, b)
        assert np.array_equal(a[2], rid)
        assert G.take_status() == 0
        if rep == 0:
            oracle_check(st, x, a)


def test_config4_shape_cache_with_prefetch(gpu, stack4):
    """An HBM cache of 48 slots in front of the 3 x 64 host-tier experts: each step's Zipf routes
    are prefetched before the step; three steps of router routing (no prefetch, demand misses)
    are interleaved. Every step equals the all-resident stack bit for bit."""
    import torch
    import ds41_gfx950 as G
    st, perms = stack4
    st.tier.cache(48)
    rng = np.random.default_rng(86)
    c0 = st.tier.cache_stats()
    for step in range(6):
        x = rand_x(gpu, 90 + step, T, H)
        if step % 2 == 0:
            rid = np.stack([zipf_ids(rng, perms[l]) for l in range(L)])
            rid[:, 1, 2] = [perms[l][RES + step + l] for l in range(L)]
            if any(len(set(rid[l, 1].tolist())) != K for l in range(L)):
                continue
            st.tier.prefetch_routes(rid)
            route = torch.from_numpy(rid).to(gpu)
        else:
            route = None
        a = st.run("tier", x, route)
        b = st.run("all", x, route)
        check_same(a, b)
        assert G.take_status() == 0
    c1 = st.tier.cache_stats()
    d = {k: c1[k] - c0[k] for k in c1 if k != "slots"}
    say(f"  cache {d}")
    assert d["prefetch_copies"] > 0 and d["hits"] > 0
