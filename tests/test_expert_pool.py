"""The library's expert slot pool (ds41_pool_*, host code: runs without a GPU) against the
reference's own SlotPool and placement parser (components/moe/src/store.cpp, manifest.cpp),
compiled from the reference sources into oracle/_ref by `make -C oracle ref`, on random
operation traces; and against hand-derived outcomes of the LFU rules, which hold with or
without the compiled reference."""
import os
import tempfile

import numpy as np
import pytest

import ds41_gfx950 as G
import oracle as O

LAYERS = G.REFERENCE_LAYERS
FIRST = np.concatenate([[0], np.cumsum(LAYERS)]).astype(np.int64)
N_IDS = int(FIRST[-1])
REF_PROFILES = "/root/reference/profiles"

needs_ref = pytest.mark.skipif(O.refpool() is None, reason="oracle/_ref not built (needs the reference sources)")


class RefPool:
    """ctypes view of the compiled reference SlotPool with the library wrapper's method shapes."""

    def __init__(self, slots, recent=6, decay=32, distinct=True):
        self.R = O.refpool()
        self.h = self.R.refpool_create(slots, recent, decay, int(distinct))

    def _allocs(self, fn, ids, *extra):
        ids_a = np.ascontiguousarray(ids, np.uint32)
        out = np.zeros((max(len(ids), 1), 4), np.int64)
        rc = fn(self.h, ids_a.ctypes.data, len(ids), *extra, out.ctypes.data)
        return rc, [(int(a), int(b), bool(c), int(d)) for a, b, c, d in out[:max(rc, 0)]]

    def acquire(self, ids, prefetch=False):
        return self._allocs(self.R.refpool_acquire, ids, int(prefetch))

    def borrow(self, ids):
        return self._allocs(self.R.refpool_borrow, ids)

    def release(self, lease):
        arr = np.array([[e, s, int(h), ev] for e, s, h, ev in lease] or [[0, 0, 0, 0]], np.int64)
        return self.R.refpool_release(self.h, arr.ctypes.data, len(lease))

    def touch(self, ids):
        ids_a = np.ascontiguousarray(ids, np.uint32)
        return self.R.refpool_touch(self.h, ids_a.ctypes.data, len(ids))

    def policy(self, budget, hard=False, pins=(), recent=6, decay=32, distinct=True):
        b = np.zeros(43, np.uint32)
        b[:len(budget)] = budget
        p = np.ascontiguousarray(list(pins) or [0], np.uint32)
        return self.R.refpool_policy(self.h, b.ctypes.data, int(hard), p.ctypes.data, len(pins), recent, decay,
                                     int(distinct))

    def pin(self, e):
        return self.R.refpool_pin(self.h, e)

    def unpin(self, e):
        return self.R.refpool_unpin(self.h, e)

    def residency(self, e):
        return self.R.refpool_residency(self.h, e)

    def reset_history(self):
        self.R.refpool_reset(self.h)
        return 0

    def __del__(self):
        try:
            self.R.refpool_destroy(self.h)
        except Exception:
            pass


def zipf_ids(rng, layer, n, s=1.1):
    E = LAYERS[layer]
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    return (FIRST[layer] + rng.choice(E, size=n, p=p)).astype(np.int64).tolist()


def run_trace(ours, ref, rng, ops, layers, max_ids):
    """Applies the same random operations to both pools; every return value must match."""
    held = []
    for step in range(ops):
        r = rng.random()
        if r < 0.70:
            ls = rng.choice(layers, size=rng.integers(1, 3))
            ids = []
            for l in ls:
                ids += zipf_ids(rng, int(l), int(rng.integers(1, max_ids + 1)))
            pre = bool(rng.random() < 0.1)
            a, b = ours.acquire(ids, pre), ref.acquire(ids, pre)
            assert a == b, (step, "acquire", ids, a, b)
            if a[0] > 0:
                held.append(a[1])
        elif r < 0.78:
            ids = zipf_ids(rng, int(rng.choice(layers)), 4)
            a, b = ours.borrow(ids), ref.borrow(ids)
            assert a == b, (step, "borrow", a, b)
            if a[0] > 0:
                held.append(a[1])
        elif r < 0.86:
            ids = zipf_ids(rng, int(rng.choice(layers)), int(rng.integers(1, 6)))
            assert ours.touch(ids) == ref.touch(ids) == 0
        elif r < 0.92:
            e = zipf_ids(rng, int(rng.choice(layers)), 1)[0]
            if rng.random() < 0.6:
                assert ours.pin(e) == ref.pin(e), (step, "pin", e)
            else:
                assert ours.unpin(e) == ref.unpin(e)
        elif r < 0.93:
            assert ours.reset_history() == ref.reset_history() == 0
        # keep at most two leases outstanding, release the oldest
        while len(held) > (2 if rng.random() < 0.5 else 0):
            lease = held.pop(0)
            assert ours.release(lease) == ref.release(lease) == 0
    for l in layers:
        for e in range(FIRST[l], FIRST[l + 1]):
            assert ours.residency(int(e)) == ref.residency(int(e)), (l, e)


POLICIES = {
    "default": dict(recent=6, decay=32, distinct=True, budget=None),
    "recent2_budgets": dict(recent=2, decay=32, distinct=True, budget={0: 6, 1: 10, 2: 4}),
    "multiplicity": dict(recent=6, decay=8, distinct=False, budget=None),
    "no_recent_no_decay": dict(recent=0, decay=0, distinct=True, budget={1: 3}),
    "drafter_layers": dict(recent=2, decay=4, distinct=True, budget={40: 8, 41: 8}),
}


@needs_ref
@pytest.mark.parametrize("name", sorted(POLICIES))
def test_pool_matches_reference_slotpool(name):
    cfg = POLICIES[name]
    layers = [40, 41, 42] if name == "drafter_layers" else [0, 1, 2]
    slots = 24
    for seed in range(3):
        rng = np.random.default_rng(1000 * seed + len(name))
        ours = G.ExpertPool(slots, recent=cfg["recent"], decay=cfg["decay"], distinct=cfg["distinct"])
        ref = RefPool(slots, cfg["recent"], cfg["decay"], cfg["distinct"])
        if cfg["budget"] is not None:
            budget = [0] * 43
            for l, b in cfg["budget"].items():
                budget[l] = b
            p = G.make_placement(43, budget, recent=cfg["recent"], decay=cfg["decay"], distinct=cfg["distinct"])
            assert ours.policy(p) == 0
            assert ref.policy(budget, recent=cfg["recent"], decay=cfg["decay"], distinct=cfg["distinct"]) == 0
        run_trace(ours, ref, rng, 600, layers, 8)


@needs_ref
def test_pool_hard_budgets_match_reference():
    """Hard pools deal every slot to a layer (pins + budget, layer by layer); a layer can only use
    its own slots. Pins are loaded and pinned first, as OffloadStore::place does."""
    budget = [0] * 43
    budget[0], budget[1], budget[2] = 5, 7, 4
    pins = [FIRST[0] + 3, FIRST[0] + 9, FIRST[1] + 0, FIRST[2] + 100]
    slots = sum(budget) + len(pins)
    for seed in range(3):
        rng = np.random.default_rng(77 + seed)
        ours, ref = G.ExpertPool(slots, recent=2, decay=16), RefPool(slots, 2, 16)
        assert ours.policy(G.make_placement(43, budget, hard=True, recent=2, decay=16, pins=pins)) == 0
        assert ref.policy(budget, hard=True, pins=pins, recent=2, decay=16) == 0
        a, b = ours.acquire(pins), ref.acquire(pins)
        assert a == b and a[0] == len(pins)
        for e in pins:
            assert ours.pin(int(e)) == ref.pin(int(e)) == 0
        assert ours.release(a[1]) == ref.release(b[1]) == 0
        run_trace(ours, ref, rng, 500, [0, 1, 2], 6)
        # a layer's demand beyond its own slots is rejected by both, before any state change
        big = list(range(FIRST[2], FIRST[2] + 6))
        assert ours.acquire(big)[0] == ref.acquire(big)[0] == -1
    bad = [1] * 43
    assert G.ExpertPool(slots).policy(G.make_placement(43, bad, hard=True, pins=pins)) == -4
    assert RefPool(slots).policy(bad, hard=True, pins=pins) == -4


@needs_ref
def test_pool_errors_match_reference():
    ours, ref = G.ExpertPool(3), RefPool(3)
    assert ours.acquire([N_IDS])[0] == ref.acquire([N_IDS])[0] == -2
    a, b = ours.acquire([1, 2, 3]), ref.acquire([1, 2, 3])
    assert a == b
    assert ours.acquire([4])[0] == ref.acquire([4])[0] == -1  # all slots leased
    assert ours.release([(9, 0, False, -1)]) == ref.release([(9, 0, False, -1)]) == -3
    assert ours.pin(77) == ref.pin(77) == -3  # not resident
    assert ours.release(a[1]) == ref.release(b[1]) == 0
    assert ours.release(a[1]) == ref.release(b[1]) == -3  # already released


IMPLS = ["library"] + (["reference"] if O.refpool() is not None else [])


@pytest.fixture(params=IMPLS)
def impl(request):
    return request.param


def make_pool(impl, slots, recent=0, decay=0):
    if impl == "library":
        return G.ExpertPool(slots, recent=recent, decay=decay)
    return RefPool(slots, recent, decay)


def test_lfu_evicts_least_frequent_then_oldest(impl):
    """recent 0, decay 0: A used three times, B once, C once -> D evicts the least-used, oldest
    stamp first (B, acquired before C); then E evicts C."""
    p = make_pool(impl, 3)
    A, B, C, D, E = 10, 11, 12, 13, 14
    for _ in range(3):
        rc, a = p.acquire([A])
        p.release(a)
    for e in (B, C):
        rc, a = p.acquire([e])
        p.release(a)
    rc, a = p.acquire([D])
    assert a == [(D, 1, False, B)]
    p.release(a)
    rc, a = p.acquire([E])
    assert a == [(E, 2, False, C)]
    p.release(a)
    assert p.residency(A) == 0 and p.residency(B) == -1


def test_recent_window_protects_then_yields(impl):
    """recent 2: an expert used within the last 2 ticks of its layer is skipped while any other
    victim exists; when every candidate is recent, the LFU order decides anyway."""
    p = make_pool(impl, 2, recent=2)
    A, B, C = 1, 2, 3
    for _ in range(4):  # A: count 4, ticks 1..4
        _, a = p.acquire([A])
        p.release(a)
    _, a = p.acquire([B])  # tick 5: B count 1, recent
    p.release(a)
    _, a = p.acquire([C])  # tick 6: A (last 4, 4+2 >= 6 -> recent) and B (recent) -> pass 1: B (count 1)
    assert a == [(C, 1, False, B)]
    p.release(a)
    for _ in range(3):  # ticks 7..9 with other ids of the layer: A and C age out of the window
        p.touch([50])
    _, a = p.acquire([B])  # tick 10: A count 4, C count 1, neither recent -> C
    assert a == [(B, 1, False, C)]


def test_decay_halves_counts_of_the_layer(impl):
    """decay 4: every 4th tick of a layer halves its experts' counts before the tick's own
    counts are added, so an early burst loses to steady recent use."""
    p = make_pool(impl, 2, decay=4)
    A, B, C = 100, 101, 102
    for _ in range(3):  # ticks 1-3: A count 3
        _, a = p.acquire([A])
        p.release(a)
    _, a = p.acquire([B])  # tick 4: halve (A 3 -> 1), then B 1
    p.release(a)
    _, a = p.acquire([B])  # tick 5: B 2
    p.release(a)
    _, a = p.acquire([C])  # tick 6: A 1 < B 2 -> A goes
    assert a == [(C, 0, False, A)]


def test_soft_budget_prefers_over_budget_layer(impl):
    """budget layer 0: 1 slot. With two layer-0 experts resident, a new layer-1 expert evicts a
    layer-0 slot even though the layer-1 resident has the lower count."""
    p = make_pool(impl, 3)
    budget = [0] * 43
    budget[0] = 1
    budget[1] = 2
    if impl == "library":
        assert p.policy(G.make_placement(43, budget, recent=0, decay=0)) == 0
    else:
        assert p.policy(budget, recent=0, decay=0) == 0
    a0, a1, b0 = 5, 6, FIRST[1] + 7
    for e, n in ((a0, 3), (a1, 3), (b0, 1)):
        for _ in range(n):
            _, a = p.acquire([int(e)])
            p.release(a)
    _, a = p.acquire([int(FIRST[1] + 8)])
    assert a[0][3] in (a0, a1) and p.residency(int(b0)) >= 0


def test_capacity_rejection_changes_nothing(impl):
    p = make_pool(impl, 2)
    _, lease = p.acquire([1, 2])
    assert p.acquire([3])[0] == -1
    assert p.residency(3) == -1 and p.residency(1) == 0 and p.residency(2) == 1
    assert p.release(lease) == 0
    _, a = p.acquire([3])
    assert a == [(3, 0, False, 1)]  # counts equal (1 each), A's stamp is older


@needs_ref
@pytest.mark.skipif(not os.path.isdir(REF_PROFILES), reason="reference profiles absent")
@pytest.mark.parametrize("name", ["p80-mtp48.placement", "k3-p80.placement"])
def test_placement_profiles_match_reference_parser(name):
    path = os.path.join(REF_PROFILES, name)
    ours, vram, host = G.load_placement(path)
    R = O.refpool()
    u = np.zeros(4, np.uint32)
    b, hb = np.zeros(43, np.uint32), np.zeros(43, np.uint32)
    v, h = np.zeros(1 << 16, np.uint32), np.zeros(1 << 16, np.uint32)
    nv, nh = np.zeros(1, np.int32), np.zeros(1, np.int32)
    assert R.refplacement_load(path.encode(), u.ctypes.data, b.ctypes.data, hb.ctypes.data, v.ctypes.data,
                               nv.ctypes.data, 1 << 16, h.ctypes.data, nh.ctypes.data, 1 << 16) == 0
    assert [ours.recent_window, ours.decay_interval, ours.distinct_lfu, ours.hard_budgets] == u.tolist()
    assert list(ours.budget[:43]) == b.tolist() and list(ours.host_budget[:43]) == hb.tolist()
    assert vram == v[:nv[0]].tolist() and host == h[:nh[0]].tolist()
    assert len(vram) > 1000 and len(host) > 1000


BAD_PLACEMENTS = ["vram 5\nvram 5\n", "vram 5\nhost 5\n", "pools medium\n", "budget 43 1\n", "budget 40 129\n",
                  "budget 0 385\n", "recent -\n", "lfu sometimes\n", "vram 15744\n", "frobnicate 1\n",
                  "recent 2 3\n", "decay 4294967296\n"]
GOOD_PLACEMENTS = ["# c\n\nrecent 2\ndecay 256\npools hard\nlfu multiplicity\nbudget 40 128\nhost_budget 3 7\n"
                   "vram 15743\nhost 0\n", ""]


@needs_ref
@pytest.mark.parametrize("text", BAD_PLACEMENTS + GOOD_PLACEMENTS)
def test_placement_accepts_and_rejects_like_reference(text):
    with tempfile.NamedTemporaryFile("w", suffix=".placement", delete=False) as f:
        f.write(text)
        path = f.name
    try:
        R = O.refpool()
        u, b, hb = np.zeros(4, np.uint32), np.zeros(43, np.uint32), np.zeros(43, np.uint32)
        v, h, nv, nh = np.zeros(16, np.uint32), np.zeros(16, np.uint32), np.zeros(1, np.int32), np.zeros(1, np.int32)
        ref_ok = R.refplacement_load(path.encode(), u.ctypes.data, b.ctypes.data, hb.ctypes.data, v.ctypes.data,
                                     nv.ctypes.data, 16, h.ctypes.data, nh.ctypes.data, 16) == 0
        try:
            ours, vram, host = G.load_placement(path)
            ok = True
        except ValueError:
            ok = False
        assert ok == ref_ok == (text in GOOD_PLACEMENTS)
        if ok:
            assert [ours.recent_window, ours.decay_interval, ours.distinct_lfu, ours.hard_budgets] == u.tolist()
            assert list(ours.budget[:43]) == b.tolist() and list(ours.host_budget[:43]) == hb.tolist()
            assert vram == v[:nv[0]].tolist() and host == h[:nh[0]].tolist()
    finally:
        os.unlink(path)
