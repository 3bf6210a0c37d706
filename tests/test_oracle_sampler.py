"""Pins the oracle's acceptance sampler (oracle/sampler_oracle.c) against the
reference: the Philox v2 known answers of engine/tests/core.cpp:21-31, golden
vectors written by the reference's own compiled sampler (tests/golden/*.json),
the closed forms of core.cpp:35-60, and the distribution-preservation property
of core.cpp:44-76 (rejection sampling with the residual max(0, p - q) emits
tokens distributed as p)."""
import hashlib
import json
import math
import os
import sys

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_accept_golden import logits_for  # noqa: E402  (numpy-only logits generator)

TARGET, DRAFT, ACCEPT, RESIDUAL = 0, 1, 2, 3


def test_philox_known_answers():
    L = O.lib()
    assert [L.oracle_philox_word_v2(0, 0, 0, TARGET, d) for d in range(4)] == \
        [0xE0481467, 0x8DDFD609, 0xB08E446F, 0x1852B5AB]
    assert L.oracle_uniform_v2(0, 0, 0, TARGET, 0) == 0.8760998513862246
    assert L.oracle_philox_word_v2(0, 0, 0, TARGET, 0) != L.oracle_philox_word_v2(0, 0, 0, DRAFT, 0)
    assert L.oracle_philox_word_v2(0, 1, 0, TARGET, 0) != L.oracle_philox_word_v2(0, 0, 0, TARGET, 0)
    assert L.oracle_philox_word_v2(0, 0, 1, TARGET, 0) != L.oracle_philox_word_v2(0, 0, 0, TARGET, 0)


def test_philox_golden_grid():
    rows = json.load(open(os.path.join(HERE, "golden", "philox_v2.json")))["rows"]
    L = O.lib()
    for seed, step, slot, purpose, draw, word, uhex in rows:
        assert L.oracle_philox_word_v2(seed, step, slot, purpose, draw) == word
        assert L.oracle_uniform_v2(seed, step, slot, purpose, draw) == float.fromhex(uhex)


def test_probabilities_closed_forms():
    assert np.all(O.probabilities(np.zeros(4, np.float32), 1, 1) == 0.25)
    assert list(O.probabilities(np.array([2, 1, 0], np.float32), 0, 1)) == [1, 0, 0]
    assert list(O.probabilities(np.zeros(4, np.float32), 1, 0.5)) == [0.5, 0.5, 0, 0]
    for bad in (np.array([np.nan], np.float32),):
        with pytest.raises(ValueError):
            O.probabilities(bad, 1, 1)
    with pytest.raises(ValueError):
        O.probabilities(np.zeros(1, np.float32), -1, 1)
    # ties at the maximum: the first occurrence is the argmax (one-hot at T=0)
    x = np.array([1, 3, 3, 2], np.float32)
    assert list(O.probabilities(x, 0, 1)) == [0, 1, 0, 0]
    # top-p keeps the lower id first among equal probabilities (stable order)
    p = O.probabilities(np.array([0, 1, 1, 0], np.float32), 1, 0.3)
    assert p[1] == 1.0 and p[2] == 0.0


def test_verify_greedy_cases():
    # core.cpp:50-60
    rows = np.array([[0, 0, 1, 0], [0, 1, 0, 0], [1, 0, 0, 0]], np.float64)
    for seed in (0, 1, 42, 99):
        r = O.verify_v2(np.array([2, 0], np.int32), None, rows, 2, 4, 1, seed, 100)
        assert r.as_tuple() == ((2, 1), 1, 2, 1)
        r = O.verify_v2(np.array([2], np.int32), None, rows[:2], 1, 4, 1, seed, 100)
        assert r.as_tuple() == ((2, 1), 1, 2, 0)


def test_verify_rejects_invalid_rows():
    p = np.array([[0.5, 0.5], [0.5, 0.6]])
    with pytest.raises(ValueError):
        O.verify_v2(np.array([0], np.int32), np.array([[0.5, 0.5]]), p, 1, 2, 0, 0, 0)
    with pytest.raises(ValueError):  # draft impossible under q
        O.verify_v2(np.array([0], np.int32), np.array([[0.0, 1.0]]), np.array([[0.5, 0.5], [0.5, 0.5]]), 1, 2, 0,
                    0, 0)


def test_rejection_sampling_preserves_target_distribution():
    # core.cpp:44-76 with fewer trials: emitted token ~ p within 6 sigma
    pairs = [([.1, .2, .3, .4], [.4, .3, .2, .1]), ([.2, .3, .5, 0], [0, 0, 0, 1]),
             ([.25, .25, .25, .25], [.25, .25, .25, .25])]
    trials = 20000
    pos = 0
    for p, q in pairs:
        p = np.array(p, np.float64)
        q = np.array(q, np.float64)
        counts = np.zeros(4, int)
        for _ in range(trials):
            d = O.sample_v2(q, 0, pos, 0, DRAFT)
            r = O.verify_v2(np.array([d], np.int32), q[None], np.stack([p, p]), 1, 4, 0, 0, pos)
            counts[r.tokens[0]] += 1
            pos += 1
        for j in range(4):
            e = trials * p[j]
            assert abs(counts[j] - e) < 6 * math.sqrt(e * (1 - p[j])) + 2


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


GOLD = json.load(open(os.path.join(HERE, "golden", "accept_v2.json")))


@pytest.mark.parametrize("case", GOLD["cases"], ids=[c["name"] for c in GOLD["cases"]])
def test_accept_golden_vs_reference(case):
    V, k, T, top_p, seed = case["vocab"], case["drafts"], case["temperature"], case["top_p"], case["seed"]
    t = max(T, 1e-5) if T > 0 else T
    for entry in case["results"]:
        step = entry["step"]
        target, draft = logits_for(case, step)
        p = np.stack([O.probabilities(target[r], t, top_p) for r in range(k + 1)])
        assert [_sha(p[r]) for r in range(k + 1)] == entry["p_sha256"], (case["name"], step)
        if T == 0:
            drafts = [int(np.argmax(draft[j])) for j in range(k)]
            q = None
        else:
            q = np.stack([O.probabilities(draft[j], t, top_p) for j in range(k)])
            assert [_sha(q[j]) for j in range(k)] == entry["q_sha256"], (case["name"], step)
            drafts = [O.sample_v2(q[j], seed, step, j, DRAFT) for j in range(k)]
        assert drafts == entry["drafts"]
        r = O.verify_v2(np.array(drafts, np.int32), q, p, k, V, 1 if T == 0 else 0, seed, step)
        assert list(r.tokens[:r.emitted]) == entry["tokens"] and r.accepted_drafts == entry["accepted"] and \
            r.rejected == entry["rejected"], (case["name"], step)
        # the fused logits path gives the same result
        r2 = O.accept_logits(target, draft if T != 0 else None, np.array(drafts, np.int32), T, top_p, seed, step)
        assert r2.as_tuple() == r.as_tuple()


@pytest.mark.skipif(O.ref() is None, reason="oracle/_ref not built (needs the reference sources)")
def test_probabilities_bitwise_vs_compiled_reference():
    # engine/tests/sampling_parallel.cpp-style inputs against the reference build itself
    R = O.ref()
    rng = np.random.default_rng(20261018)
    for n in (4096, 4097, 65537):
        for t in (1.0, 0.7, 1e-7, 2.5):
            for trial in range(4):
                x = (rng.standard_normal(n) * (40 if trial == 3 else 4)).astype(np.float32)
                if trial == 1:
                    m = x.max() + 1
                    x[[n // 3, n // 2, n - 1]] = m
                if trial == 2:
                    x[::7] = np.round(x[::7])
                for top_p in (1.0, 0.9):
                    tt = max(t, 1e-5)
                    ref = np.empty(n, np.float64)
                    assert R.ds41_spark_probabilities(x.ctypes.data, ref.ctypes.data, n, tt, top_p) == 0
                    assert np.array_equal(O.probabilities(x, tt, top_p).view(np.uint64), ref.view(np.uint64))


# ---- the reference's GPU sampler over fp32 measures (sampling.cu:6-39) -------------------------
def exact_measure(rng, n, hi, m=None):
    """fp32 integer measure whose total is a power of two: every fp64 sum of it and of its
    normalisation is exact, in any order."""
    x = rng.integers(0, hi, n).astype(np.int64)
    x[rng.integers(0, n)] += 1
    s = int(x.sum())
    total = 1 << (s - 1).bit_length() if m is None else m
    x[rng.integers(0, n)] += total - s
    return x.astype(np.float32), float(total)


@pytest.mark.skipif(O.ref() is None, reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("n", [1, 7, 256, 300, 4097, 129280])
def test_gpu_sampler_equals_host_sampler_when_sums_are_exact(n):
    """Where every fp64 sum is exact, the GPU sampler's chunked/strided orders cannot matter: its
    decisions must equal the compiled reference host sampler's on the normalised measures."""
    import ctypes
    R = O.ref()
    rng = np.random.default_rng(n)
    k = 3 if n > 6 else 1
    for trial in range(12):
        hi = 16 if trial % 3 else 3  # few levels: many ties for greedy and for draws
        p32 = np.empty((k + 1, n), np.float32)
        q32 = np.empty((k, n), np.float32)
        p64 = np.empty((k + 1, n))
        q64 = np.empty((k, n))
        for r in range(k + 1):
            p32[r], z = exact_measure(rng, n, hi)
            p64[r] = p32[r].astype(np.float64) / z
        for r in range(k):
            q32[r], z = exact_measure(rng, n, hi)
            q64[r] = q32[r].astype(np.float64) / z
        seed, step = int(rng.integers(0, 1 << 62)), int(rng.integers(0, 1 << 40))
        d = []
        for j in range(k):
            tok = ctypes.c_int32(-1)
            assert R.ds41_spark_sample_v2(q64[j].ctypes.data, n, seed, step, j, 1, ctypes.byref(tok)) == 0
            d.append(tok.value)
            assert O.sample_gpu_v2(q32[j], seed, step, j, 1) == tok.value
        d = np.array(d, np.int32)
        for greedy in (0, 1):
            want = O.SparkResult()
            assert R.ds41_spark_verify_v2(d.ctypes.data, q64.ctypes.data, p64.ctypes.data, k, n, greedy, seed, step,
                                          ctypes.byref(want)) == 0
            got = O.verify_gpu_v2(d, q32, p32, k, n, greedy, seed, step)
            assert got.as_tuple() == want.as_tuple(), (n, trial, greedy)


def test_gpu_sampler_closed_forms_and_invalid_rows():
    n = 1000
    rng = np.random.default_rng(5)
    p = rng.random((2, n)).astype(np.float32)
    # p == q: the acceptance ratio is exactly 1, every draft is accepted
    for step in range(20):
        d = np.array([rng.integers(0, n)], np.int32)
        r = O.verify_gpu_v2(d, p[:1], p, 1, n, 0, 7, step)
        assert r.as_tuple()[:2] == ((int(d[0]), r.tokens[1]), 1) and r.rejected == 0
    # greedy: accept iff the draft is the first argmax; on reject the argmax is emitted
    p2 = np.zeros((2, 8), np.float32)
    p2[0, [2, 5]] = 3.0
    p2[1, 4] = 1.0
    assert O.verify_gpu_v2(np.array([2], np.int32), None, p2, 1, 8, 1, 0, 0).as_tuple() == ((2, 4), 1, 2, 0)
    assert O.verify_gpu_v2(np.array([5], np.int32), None, p2, 1, 8, 1, 0, 0).as_tuple() == ((2,), 0, 1, 1)
    # invalid rows / ids: emitted -1
    bad = p.copy()
    bad[1, 3] = np.nan
    assert O.verify_gpu_v2(np.array([0], np.int32), p[:1], bad, 1, n, 0, 0, 0).emitted == -1
    neg = p.copy()
    neg[0, 9] = -1e-30
    assert O.verify_gpu_v2(np.array([0], np.int32), p[:1], neg, 1, n, 0, 0, 0).emitted == -1
    q0 = p[:1].copy()
    q0[0, 11] = 0
    assert O.verify_gpu_v2(np.array([11], np.int32), q0, p, 1, n, 0, 0, 0).emitted == -1
    assert O.verify_gpu_v2(np.array([n], np.int32), p[:1], p, 1, n, 0, 0, 0).emitted == -1
    assert O.verify_gpu_v2(np.array([0], np.int32), p[:1], np.zeros((2, n), np.float32), 1, n, 0, 0, 0).emitted == -1
    assert O.sample_gpu_v2(np.zeros(n, np.float32), 0, 0, 0, 0) == -1
    with pytest.raises(ValueError):
        O.verify_gpu_v2(None, p[:1], p, 1, n, 0, 0, 0)


def test_gpu_sampler_preserves_target_distribution():
    """Rejection sampling with the GPU sampler's residual max(0, p/pz - q/qz) emits tokens
    distributed as p (core.cpp:44-76 style), on unnormalised fp32 measures."""
    pairs = [([1, 2, 3, 4], [4, 3, 2, 1]), ([2, 3, 5, 0], [0, 0, 0, 7]), ([1, 1, 1, 1], [3, 1, 2, 5])]
    trials = 20000
    pos = 0
    for p, q in pairs:
        p = np.array(p, np.float32)
        q = np.array(q, np.float32)
        pn = p.astype(np.float64) / p.sum()
        counts = np.zeros(4, int)
        for _ in range(trials):
            d = O.sample_gpu_v2(q, 3, pos, 0, DRAFT)
            r = O.verify_gpu_v2(np.array([d], np.int32), q[None], np.stack([p, p]), 1, 4, 0, 3, pos)
            counts[r.tokens[0]] += 1
            pos += 1
        for j in range(4):
            e = trials * pn[j]
            assert abs(counts[j] - e) < 6 * math.sqrt(e * (1 - pn[j])) + 2
