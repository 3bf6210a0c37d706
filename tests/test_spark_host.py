"""The product library's host sampler C ABI (ds41_spark_probabilities / _sample_v2 / _verify_v2 /
_uniform_v2 / _rng_word_v2, spark.h:115-132), on the CPU.

Bars, all bit-exact:
- the committed golden fixtures written by the reference's own compiled sampler
  (tests/golden/philox_v2.json words and uniforms; tests/golden/accept_v2.json: SHA-256 of every
  fp64 probability row, the sampled draft tokens and the verify results);
- the reference's libds41_spark compiled from its sources (oracle/_ref, when built) on rows the
  fixtures do not cover: ties at the top-p cut, tiny temperatures, greedy rows, invalid inputs;
- the reference engine's own accept step (engine/src/sampling.cpp through oracle/_ref, when
  built): draft tokens from q and the reject_sample result."""
import ctypes
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
from make_accept_golden import logits_for  # noqa: E402

GOLD = json.load(open(os.path.join(HERE, "golden", "accept_v2.json")))
DRAFT, TARGET = 1, 0


def G():
    import ds41_gfx950
    return ds41_gfx950


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_philox_words_and_uniforms_match_golden():
    rows = json.load(open(os.path.join(HERE, "golden", "philox_v2.json")))["rows"]
    for seed, step, slot, purpose, draw, word, u in rows:
        assert G().spark_rng_word_v2(seed, step, slot, purpose, draw) == word
        assert G().spark_uniform_v2(seed, step, slot, purpose, draw) == float.fromhex(u)
    assert G().spark_rng_word_v2(0, 0, 6, 0, 0) == 0 and G().spark_error()
    assert math.isnan(G().spark_uniform_v2(0, 0, 0, 4, 0))
    assert math.isnan(G().spark_uniform_v2(0, 0, 0, 0, 1 << 33))


@pytest.mark.parametrize("case", GOLD["cases"], ids=[c["name"] for c in GOLD["cases"]])
def test_host_sampler_reproduces_golden(case):
    """Probability rows (SHA-256), draft tokens and verify results of every golden step."""
    V, k, T, top_p, seed = case["vocab"], case["drafts"], case["temperature"], case["top_p"], case["seed"]
    greedy = 1 if T == 0 else 0
    t = max(T, 1e-5) if T > 0 else T
    steps = case["results"][:12] if V > 10000 else case["results"]
    for e in steps:
        target, draft = logits_for(case, e["step"])
        p = np.stack([G().spark_probabilities(target[r], t, top_p) for r in range(k + 1)])
        assert [sha(p[r]) for r in range(k + 1)] == e["p_sha256"]
        q = None
        if greedy:
            drafts = [int(np.argmax(draft[j])) for j in range(k)]
        else:
            q = np.stack([G().spark_probabilities(draft[j], t, top_p) for j in range(k)])
            assert [sha(q[j]) for j in range(k)] == e["q_sha256"]
            drafts = [G().spark_sample_v2(q[j], seed, e["step"], j, DRAFT) for j in range(k)]
        assert drafts == e["drafts"]
        res = G().spark_verify_v2(np.array(drafts, np.int32), q, p, greedy, seed, e["step"])
        assert res == (tuple(e["tokens"]), e["accepted"], e["accepted"] + 1, e["rejected"])


def _ref_probabilities(R, x, t, top_p):
    p = np.empty(x.shape[0], np.float64)
    rc = R.ds41_spark_probabilities(x.ctypes.data, p.ctypes.data, x.shape[0], t, top_p)
    return p if rc == 0 else None


def _ref_sample(R, p, seed, step, slot, purpose):
    tok = ctypes.c_int32(-1)
    rc = R.ds41_spark_sample_v2(p.ctypes.data, p.shape[0], seed, step, slot, purpose, ctypes.byref(tok))
    return tok.value if rc == 0 else None


def _ref_verify(R, d, q, p, greedy, seed, step):
    k, V = p.shape[0] - 1, p.shape[1]
    res = O.SparkResult()
    rc = R.ds41_spark_verify_v2(None if not k else np.ascontiguousarray(d, np.int32).ctypes.data,
                                None if q is None else np.ascontiguousarray(q).ctypes.data,
                                np.ascontiguousarray(p).ctypes.data, k, V, greedy, seed, step, ctypes.byref(res))
    return res.as_tuple() if rc == 0 else None


def _rows(rng, kind, V):
    if kind == "ties":  # many equal logits, some at the top-p cut
        x = np.round(rng.standard_normal(V) * 2).astype(np.float32)
    elif kind == "flat":
        x = np.zeros(V, np.float32)
        x[::5] = 1.0
    elif kind == "dominant":
        x = (rng.standard_normal(V) * 0.1).astype(np.float32)
        x[V // 3] = 40.0
    else:
        x = (rng.standard_normal(V) * 3).astype(np.float32)
    return x


@pytest.mark.parametrize("kind", ["normal", "ties", "flat", "dominant"])
@pytest.mark.parametrize("V", [1, 7, 4096, 40000])
def test_host_sampler_matches_reference_library(kind, V):
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    rng = np.random.default_rng(V + len(kind))
    for T in (0.0, 1e-7, 0.5, 1.0, 3.0):
        for top_p in (1.0, 0.95, 0.5, 0.1, 1e-9):
            x = _rows(rng, kind, V)
            a, b = G().spark_probabilities(x, T, top_p), _ref_probabilities(R, x, T, top_p)
            assert a is not None and b is not None
            assert a.tobytes() == b.tobytes(), (T, top_p)
            for slot, purpose, step in ((0, DRAFT, 3), (5, TARGET, 1 << 40), (2, 3, 12345)):
                assert G().spark_sample_v2(a, 7, step, slot, purpose) == _ref_sample(R, b, 7, step, slot, purpose)
    # verify_v2 on rows of this shape: drafts from q, greedy and sampled
    for greedy in (0, 1):
        for step in range(6):
            k = 3
            p = np.stack([G().spark_probabilities(_rows(rng, kind, V), 1.0, 0.9) for _ in range(k + 1)])
            q = np.stack([G().spark_probabilities(_rows(rng, kind, V), 1.0, 0.9) for _ in range(k)])
            d = np.array([G().spark_sample_v2(q[j], 5, step, j, DRAFT) for j in range(k)], np.int32)
            qq = None if greedy else q
            assert G().spark_verify_v2(d, qq, p, greedy, 5, step) == _ref_verify(R, d, qq, p, greedy, 5, step)


def test_host_sampler_rejects_what_the_reference_rejects():
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    V = 64
    x = np.linspace(-1, 1, V).astype(np.float32)
    bad_x = x.copy()
    bad_x[5] = np.inf
    for args in ((bad_x, 1.0, 1.0), (x, -1.0, 1.0), (x, 1.0, 0.0), (x, 1.0, 1.5), (x, np.nan, 1.0)):
        assert G().spark_probabilities(*args) is None and _ref_probabilities(R, *args) is None
    p = G().spark_probabilities(x, 1.0, 1.0)
    for row in (p * 2, -p, np.where(np.arange(V) == 3, np.nan, p)):
        row = np.ascontiguousarray(row)
        assert G().spark_sample_v2(row, 0, 0, 0, 0) is None and _ref_sample(R, row, 0, 0, 0, 0) is None
    assert G().spark_sample_v2(p, 0, 0, 6, 0) is None and _ref_sample(R, p, 0, 0, 6, 0) is None
    assert G().spark_sample_v2(p, 0, 0, 0, 4) is None and _ref_sample(R, p, 0, 0, 0, 4) is None
    k = 2
    P = np.stack([p] * (k + 1))
    q = np.zeros((k, V))
    q[:, 0] = 1.0  # the drafts below have no mass under q
    for d, qq, greedy in (([3, 4], q, 0), ([V, 0], P[:k], 1), ([-1, 0], P[:k], 0)):
        d = np.array(d, np.int32)
        assert G().spark_verify_v2(d, qq, P, greedy, 1, 2) is None and _ref_verify(R, d, qq, P, greedy, 1, 2) is None
    assert G().spark_error() != ""


def test_host_sampler_matches_reference_engine_accept_step():
    """SpeculativeStep's accept arithmetic (engine/src/speculation.cpp:116-182) in the reference
    engine's own code vs the product's host ABI, at configs[2]'s shape."""
    if O.refengine() is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    k, V = 3, 129280
    rng = np.random.default_rng(5)
    for T, top_p, steps in ((1.0, 1.0, 6), (1.0, 0.95, 2), (0.0, 1.0, 2), (0.8, 1.0, 3)):
        for step in range(steps):
            target = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
            draft = (target[:k] + rng.standard_normal((k, V)) * 0.5).astype(np.float32)
            ref = O.ref_accept_step(target, draft, k, T, top_p, 11, step)
            t = max(T, 1e-5) if T > 0 else 0.0
            p = np.stack([G().spark_probabilities(target[r], t, top_p) for r in range(k + 1)])
            if T == 0:
                d, q = [int(np.argmax(draft[j])) for j in range(k)], None
            else:
                q = np.stack([G().spark_probabilities(draft[j], t, top_p) for j in range(k)])
                d = [G().spark_sample_v2(q[j], 11, step, j, DRAFT) for j in range(k)]
            res = G().spark_verify_v2(np.array(d, np.int32), q, p, 1 if T == 0 else 0, 11, step)
            assert ref == (d, res), (T, top_p, step)
