"""Two-tier extensions of the library's expert slot pool (host code, no GPU): retention tokens,
reserve/drained, peer scoring with exclusive host pools and late target layers,
switch_target_layer, and the drift controller. Every return value and allocation is compared with
the reference's own SlotPool and DriftPolicy (components/moe/src/store.cpp:56-66,130-255),
compiled from the reference sources into oracle/_ref by `make -C oracle ref`, on random traces
that exercise them; plus hand-derived outcomes that hold without the compiled reference."""
import numpy as np
import pytest

import ds41_gfx950 as G
import oracle as O
from test_expert_pool import FIRST, LAYERS, RefPool, needs_ref, zipf_ids

class RefTierPool(RefPool):
    """The compiled reference SlotPool with the extension calls."""

    def retain(self, e):
        import ctypes
        rcv = ctypes.c_int(0)
        t = self.R.refpool_retain(self.h, e, ctypes.addressof(rcv))
        return rcv.value, (t if rcv.value == 0 else None)

    def token_release(self, t):
        self.R.refpool_token_release(t)
        return 0

    def reserve(self, target, wanted=()):
        w = np.ascontiguousarray(list(wanted) or [0], np.uint32)
        out = np.zeros((max(int(target), 1), 4), np.int64)
        rc = self.R.refpool_reserve(self.h, int(target), w.ctypes.data, len(wanted), out.ctypes.data)
        return rc, [(int(a), int(b), bool(c), int(d)) for a, b, c, d in out[:max(rc, 0)]]

    def drained(self, slot):
        return self.R.refpool_drained(self.h, int(slot))

    def peer(self, other, host):
        return self.R.refpool_peer(self.h, other.h if other is not None else None, int(host))

    def exclusive(self, on):
        return self.R.refpool_exclusive(self.h, int(on))

    def decay_interval(self, d):
        return self.R.refpool_decay_interval(self.h, int(d))

    def fast_minima(self, on):
        return self.R.refpool_fast_minima(self.h, int(on))

    def switch_target_layer(self, pins, layer):
        p = np.ascontiguousarray(list(pins) or [0], np.uint32)
        return self.R.refpool_switch_target_layer(self.h, p.ctypes.data, len(pins), int(layer))


class RefDrift:
    def __init__(self, pins, vram, ram, recent=2, decay=256, distinct=True, hard=False):
        import ctypes
        self.R = O.refpool()
        p = np.ascontiguousarray(list(pins) or [0], np.uint32)
        rc = ctypes.c_int(0)
        self._keep = (vram, ram)
        self.h = self.R.refdrift_create(p.ctypes.data, len(pins), recent, decay, int(distinct), int(hard), vram.h,
                                        ram.h, ctypes.addressof(rc))
        self.rc = rc.value

    def before(self, ids):
        a = np.ascontiguousarray(list(ids) or [0], np.uint32)
        return self.R.refdrift_before(self.h, a.ctypes.data, len(ids))

    def after(self, ids):
        a = np.ascontiguousarray(list(ids) or [0], np.uint32)
        return self.R.refdrift_after(self.h, a.ctypes.data, len(ids))

    def active(self):
        return self.R.refdrift_active(self.h)

    def completed_tokens(self):
        return self.R.refdrift_tokens(self.h)

    def __del__(self):
        try:
            if self.h:
                self.R.refdrift_destroy(self.h)
        except Exception:
            pass


def placement_with_pins(pins, recent=6, decay=32, budget=None):
    return G.make_placement(43, budget, recent=recent, decay=decay, pins=pins)


def same_residency(a, b, layers):
    for l in layers:
        for e in range(FIRST[l], FIRST[l + 1]):
            assert a.residency(int(e)) == b.residency(int(e)), (l, e)


def run_tier_trace(pairs, rng, ops, layers, pins, fast):
    """pairs: [(ours, ref)] for the VRAM pool then the RAM pool, peered. Same ops on both sides."""
    (ov, rv), (orr, rr) = pairs
    tokens = {0: [], 1: []}    # retention tokens per pool side: (ours, ref)
    leases = {0: [], 1: []}
    draining = {0: set(), 1: set()}
    pl = placement_with_pins(pins)
    for step in range(ops):
        side = int(rng.random() < 0.4)
        o, r = pairs[side]
        x = rng.random()
        if x < 0.50:
            ids = []
            for l in rng.choice(layers, size=rng.integers(1, 3)):
                ids += zipf_ids(rng, int(l), int(rng.integers(1, 7)))
            pre = bool(rng.random() < 0.15)
            a, b = o.acquire(ids, pre), r.acquire(ids, pre)
            assert a == b, (step, side, "acquire", ids, a, b)
            if a[0] > 0:
                leases[side].append(a[1])
        elif x < 0.60:
            e = zipf_ids(rng, int(rng.choice(layers)), 1)[0]
            a, b = o.retain(e), r.retain(e)
            assert a[0] == b[0], (step, side, "retain", e, a[0], b[0])
            if a[0] == 0:
                tokens[side].append((a[1], b[1]))
        elif x < 0.68:
            if tokens[side]:
                t_o, t_r = tokens[side].pop(int(rng.integers(len(tokens[side]))))
                assert G.ExpertPool.token_release(t_o) == 0
                r.token_release(t_r)
        elif x < 0.75:
            target = int(rng.integers(0, 8))
            wanted = zipf_ids(rng, int(rng.choice(layers)), int(rng.integers(0, 4)))
            a, b = o.reserve(target, wanted), r.reserve(target, wanted)
            assert a == b, (step, side, "reserve", target, a, b)
            for _, slot, _, _ in a[1]:
                draining[side].add(slot)
        elif x < 0.81:
            if draining[side] and rng.random() < 0.85:
                slot = sorted(draining[side])[int(rng.integers(len(draining[side])))]
                draining[side].discard(slot)
            else:
                slot = int(rng.integers(0, 8))  # mostly not draining: an error on both sides
            assert o.drained(slot) == r.drained(slot), (step, side, "drained", slot)
        elif x < 0.85:
            ids = zipf_ids(rng, int(rng.choice(layers)), int(rng.integers(1, 5)))
            assert o.touch(ids) == r.touch(ids) == 0
        elif x < 0.88:
            on = int(rng.random() < 0.5)
            assert o.exclusive(on) == r.exclusive(on) == 0
        elif x < 0.91:
            layer = int(rng.choice(list(layers) + [41, 39]))
            assert o.switch_target_layer(pl, layer) == r.switch_target_layer(pins, layer) == 0
        elif x < 0.94:
            e = int(rng.choice(pins)) if pins and rng.random() < 0.7 else zipf_ids(rng, int(rng.choice(layers)), 1)[0]
            if rng.random() < 0.6:
                assert o.pin(e) == r.pin(e), (step, side, "pin", e)
            else:
                assert o.unpin(e) == r.unpin(e)
        elif x < 0.95:
            d = int(rng.choice([0, 4, 32, 256]))
            assert o.decay_interval(d) == r.decay_interval(d) == 0
        else:
            ids = zipf_ids(rng, int(rng.choice(layers)), 4)
            a, b = o.borrow(ids), r.borrow(ids)
            assert a == b, (step, side, "borrow", a, b)
            if a[0] > 0:
                leases[side].append(a[1])
        for s in (0, 1):
            while len(leases[s]) > (2 if rng.random() < 0.5 else 0):
                lease = leases[s].pop(0)
                oo, rr_ = pairs[s]
                assert oo.release(lease) == rr_.release(lease) == 0, (step, s, "release")
        if step % 100 == 99:
            for o2, r2 in pairs:
                same_residency(o2, r2, layers)
    for s in (0, 1):
        for t_o, t_r in tokens[s]:
            G.ExpertPool.token_release(t_o)
            pairs[s][1].token_release(t_r)
    for o2, r2 in pairs:
        same_residency(o2, r2, layers)


@needs_ref
@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_tiers_match_reference_slotpool(seed, fast):
    """VRAM pool (24 slots) and RAM pool (40 slots) peered both ways, with pins, budgets, late
    layers, exclusive toggles, retention tokens and draining slots; fast_minima on the reference
    side (and accepted on ours) must not change a decision."""
    rng = np.random.default_rng(77 + seed)
    layers = [0, 1, 2, 40]
    pins = [int(FIRST[0] + 5), int(FIRST[0] + 17), int(FIRST[1] + 2), int(FIRST[2] + 200)]
    budget = [0] * 43
    budget[0], budget[1], budget[2] = 6, 4, 5
    ov, rv = G.ExpertPool(24), RefTierPool(24)
    orr, rr = G.ExpertPool(40), RefTierPool(40)
    p = placement_with_pins(pins, budget=budget)
    assert ov.policy(p) == 0 and rv.policy(budget, pins=pins) == 0
    for o, r in ((ov, rv), (orr, rr)):
        assert o.fast_minima(int(fast)) == r.fast_minima(int(fast)) == 0
    assert ov.peer(orr, False) == rv.peer(rr, False) == 0
    assert orr.peer(ov, True) == rr.peer(rv, True) == 0
    # load and pin the VRAM pins first, as a placement does
    a, b = ov.acquire(pins), rv.acquire(pins)
    assert a == b
    assert ov.release(a[1]) == rv.release(b[1]) == 0
    for e in pins:
        assert ov.pin(e) == rv.pin(e) == 0
    run_tier_trace([(ov, rv), (orr, rr)], rng, 1500, layers, pins, fast)


@needs_ref
@pytest.mark.parametrize("seed", [0, 1])
def test_drift_controller_matches_reference(seed):
    """Token-major traversal of the 40 target layers (plus a drafter layer, which the controller
    ignores) over a VRAM pool whose pins cover few of the demanded experts: the pinned hit rate
    falls below one half, and after 128 tokens the controller turns every target layer late in
    both pools. Decisions, activation time and every allocation must match the reference."""
    rng = np.random.default_rng(500 + seed)
    pins = [int(FIRST[l] + k) for l in range(40) for k in (0, 1)]
    ov, rv = G.ExpertPool(160, recent=2, decay=256), RefTierPool(160, 2, 256)
    orr, rr = G.ExpertPool(320, recent=2, decay=256), RefTierPool(320, 2, 256)
    p = placement_with_pins(pins, recent=2, decay=256)
    assert ov.policy(p) == 0 and rv.policy([0] * 43, pins=pins, recent=2, decay=256) == 0
    a, b = ov.acquire(pins), rv.acquire(pins)
    assert a == b
    assert ov.release(a[1]) == rv.release(b[1]) == 0
    for e in pins:
        assert ov.pin(e) == rv.pin(e) == 0
    od, rd = G.DriftControl(p, ov, orr), RefDrift(pins, rv, rr)
    assert od.rc == rd.rc == 0
    switched_at = None
    for tok in range(140):
        for l in list(range(40)) + [40]:
            E = LAYERS[l]
            ids = (FIRST[l] + rng.choice(E, size=4, replace=False)).tolist()
            if rng.random() < 0.2:
                ids[0] = int(FIRST[l])  # a pinned hit now and then
            assert od.before(ids) == rd.before(ids) == 0, (tok, l)
            for o, r in ((ov, rv), (orr, rr)):
                x, y = o.acquire(ids), r.acquire(ids)
                assert x == y, (tok, l)
                assert o.release(x[1]) == r.release(y[1]) == 0
            assert od.after(ids) == rd.after(ids) == 0, (tok, l)
        assert od.completed_tokens() == rd.completed_tokens() == tok + 1
        assert od.active() == rd.active()
        if od.active() and switched_at is None:
            switched_at = tok
    assert switched_at == 128  # the window fills after 128 tokens; the switch is at token 129's layer 0
    for l in range(40):
        assert ov.late(l) == 1 and orr.late(l) == 1
    assert ov.late(40) == 0
    for o, r in ((ov, rv), (orr, rr)):
        same_residency(o, r, list(range(0, 40, 7)) + [40])


@needs_ref
def test_drift_errors_match_reference():
    pins = [int(FIRST[0])]
    ov, rv = G.ExpertPool(16, recent=2, decay=256), RefTierPool(16, 2, 256)
    orr, rr = G.ExpertPool(16, recent=2, decay=256), RefTierPool(16, 2, 256)
    bad = placement_with_pins(pins, recent=6, decay=32)
    od_bad, rd_bad = G.DriftControl(bad, ov, orr), RefDrift(pins, rv, rr, recent=6, decay=32)
    assert od_bad.rc == rd_bad.rc == -4
    p = placement_with_pins(pins, recent=2, decay=256)
    od, rd = G.DriftControl(p, ov, orr), RefDrift(pins, rv, rr)
    l1 = [int(FIRST[1]) + 3]
    assert od.before(l1) == rd.before(l1) == -4                                       # out of order
    assert od.after([int(FIRST[0])]) == rd.after([int(FIRST[0])]) == -3               # unpaired
    assert od.before([int(FIRST[0]), int(FIRST[1])]) == rd.before([int(FIRST[0]), int(FIRST[1])]) == -4  # mixed
    assert od.before([]) == rd.before([]) == -4                                       # empty
    assert od.before([int(FIRST[0])]) == rd.before([int(FIRST[0])]) == 0
    assert od.before([int(FIRST[0])]) == rd.before([int(FIRST[0])]) == -4             # twice
    assert od.after([int(FIRST[40])]) == rd.after([int(FIRST[40])]) == 0              # drafter: ignored
    assert od.after([int(FIRST[0])]) == rd.after([int(FIRST[0])]) == 0


@pytest.mark.parametrize("impl", ["ours"] + (["ref"] if O.refpool() is not None else []))
def test_retained_slot_is_never_evicted_nor_usable(impl):
    """Hand-derived: 2 slots, both occupied; a token on one leaves the other as the only victim,
    and a need set of two new experts is then rejected (capacity 1) without state change."""
    mk = (lambda: G.ExpertPool(2)) if impl == "ours" else (lambda: RefTierPool(2))
    pool = mk()
    a, b = int(FIRST[0] + 1), int(FIRST[0] + 2)
    rc, lease = pool.acquire([a, b])
    assert rc == 2 and pool.release(lease) == 0
    rc, tok = pool.retain(a)
    assert rc == 0
    rc, got = pool.acquire([int(FIRST[0] + 3)])
    assert rc == 1 and got[0][3] == b  # b evicted, a kept
    assert pool.release(got) == 0
    rc, _ = pool.acquire([int(FIRST[0] + 4), int(FIRST[0] + 5)])
    assert rc == -1
    assert pool.residency(a) == 0
    if impl == "ours":
        assert G.ExpertPool.token_release(tok) == 0
    else:
        pool.token_release(tok)
    rc, got = pool.acquire([int(FIRST[0] + 4), int(FIRST[0] + 5)])
    assert rc == 2 and {g[3] for g in got} == {a, int(FIRST[0] + 3)}


@pytest.mark.parametrize("impl", ["ours"] + (["ref"] if O.refpool() is not None else []))
def test_reserve_drains_victims_until_drained(impl):
    """Hand-derived: 4 slots full with counts 3, 1, 2, 1 (ids a..d); reserve(2) drains the two
    count-1 experts in stamp order (b, then d); their slots take no allocation until drained()."""
    pool = G.ExpertPool(4, recent=0) if impl == "ours" else RefTierPool(4, 0)
    ids = [int(FIRST[2] + k) for k in range(4)]
    for e, n in zip(ids, (3, 1, 2, 1)):
        for _ in range(n):
            rc, got = pool.acquire([e])
            assert rc == 1 and pool.release(got) == 0
    rc, drained = pool.reserve(2)
    assert rc == 2 and [d[3] for d in drained] == [ids[1], ids[3]]
    assert pool.residency(ids[1]) == pool.residency(ids[3]) == -1
    rc, _ = pool.acquire([int(FIRST[2] + 9), int(FIRST[2] + 10), int(FIRST[2] + 11)])
    assert rc == -1  # draining slots are not capacity: two usable slots for three new experts
    slot = drained[0][1]
    assert pool.drained(slot) == 0
    assert pool.drained(slot) == -3
    rc, got = pool.acquire([int(FIRST[2] + 9)])
    assert rc == 1 and got[0][1] == slot and got[0][3] == -1
