"""Writes the acceptance-sampling golden fixtures from the REFERENCE's own host
sampler (engine/third_party/spark/src/sampling.cpp, compiled from its sources by
`make -C oracle ref` into oracle/_ref/libds41_spark_ref.so).

Fixtures are data only: Philox v2 words/uniforms for a grid of counters, and per
accept case the generator spec of its logits (numpy PCG64 seeds; the logits are
regenerated bit-identically by the tests) with the reference's outputs: draft
tokens sampled from q (purpose Draft, slot k, as engine/src/speculation.cpp:149-155
does), the verify_v2 result, and SHA-256 digests of the fp64 probability rows.

    python tests/golden/make_accept_golden.py
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

DRAFT, TARGET = 1, 0


def logits_for(case, step):
    """Target rows N(0, sigma^2) [count+1][V]; draft rows = target[:count] + N(0, noise^2)."""
    rng = np.random.default_rng([case["seed_logits"], step])
    V, k = case["vocab"], case["drafts"]
    target = (rng.standard_normal((k + 1, V)) * case["sigma"]).astype(np.float32)
    draft = (target[:k] + rng.standard_normal((k, V)) * case["noise"]).astype(np.float32)
    if case.get("ties"):  # equal maxima: the first occurrence must win
        m = float(target.max()) + 1.0
        target[:, [V // 3, V // 2, V - 1]] = m
        draft[:, [V // 5, V - 2]] = float(draft.max()) + 1.0
    if case.get("rounded"):
        target[:, ::7] = np.round(target[:, ::7])
    return target, draft


def ref_probabilities(R, x, t, top_p):
    p = np.empty(x.shape[0], np.float64)
    rc = R.ds41_spark_probabilities(x.ctypes.data, p.ctypes.data, x.shape[0], t, top_p)
    assert rc == 0, R.ds41_spark_error()
    return p


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_case(R, case):
    V, k, T, top_p, seed = case["vocab"], case["drafts"], case["temperature"], case["top_p"], case["seed"]
    t = max(T, 1e-5) if T > 0 else T  # engine/src/sampling.cpp:208-210 floor
    greedy = 1 if T == 0 else 0
    steps = []
    for step in range(case["first_step"], case["first_step"] + case["steps"]):
        target, draft = logits_for(case, step)
        p = np.stack([ref_probabilities(R, target[r], t, top_p) for r in range(k + 1)])
        if greedy:
            q = None
            drafts = [int(np.argmax(draft[j])) for j in range(k)]  # speculation.cpp:149 argmax
        else:
            q = np.stack([ref_probabilities(R, draft[j], t, top_p) for j in range(k)])
            drafts = []
            for j in range(k):
                tok = ctypes.c_int32(-1)
                assert R.ds41_spark_sample_v2(q[j].ctypes.data, V, seed, step, j, DRAFT, ctypes.byref(tok)) == 0
                drafts.append(tok.value)
        d = np.array(drafts, np.int32)
        res = O.SparkResult()
        rc = R.ds41_spark_verify_v2(d.ctypes.data, 0 if q is None else q.ctypes.data, p.ctypes.data, k, V, greedy,
                                    seed, step, ctypes.byref(res))
        assert rc == 0, R.ds41_spark_error()
        entry = {"step": step, "drafts": drafts, "tokens": list(res.tokens[:res.emitted]),
                 "accepted": res.accepted_drafts, "rejected": res.rejected,
                 "p_sha256": [sha(p[r]) for r in range(k + 1)],
                 "q_sha256": [] if q is None else [sha(q[j]) for j in range(k)],
                 "p_at_drafts": [float(p[j][drafts[j]]) for j in range(k)],
                 "q_at_drafts": [] if q is None else [float(q[j][drafts[j]]) for j in range(k)]}
        steps.append(entry)
    return steps


CASES = [
    dict(name="v129280_t1_p1", vocab=129280, drafts=3, sigma=2.5, noise=0.5, temperature=1.0, top_p=1.0,
         seed=0, seed_logits=11, first_step=0, steps=48),
    dict(name="v129280_t1_p095", vocab=129280, drafts=3, sigma=2.5, noise=0.5, temperature=1.0, top_p=0.95,
         seed=0, seed_logits=12, first_step=0, steps=8),
    dict(name="v129280_greedy", vocab=129280, drafts=3, sigma=2.5, noise=0.5, temperature=0.0, top_p=1.0,
         seed=0, seed_logits=13, first_step=0, steps=8),
    dict(name="v129280_t07_p1_far", vocab=129280, drafts=3, sigma=2.5, noise=0.5, temperature=0.7, top_p=1.0,
         seed=0x5eed, seed_logits=14, first_step=(1 << 40) + 3, steps=16),
    dict(name="v4097_ties_t1_p1", vocab=4097, drafts=5, sigma=4.0, noise=1.0, temperature=1.0, top_p=1.0,
         seed=42, seed_logits=15, first_step=100, steps=64, ties=True, rounded=True),
    dict(name="v4097_t25_p09", vocab=4097, drafts=2, sigma=4.0, noise=2.0, temperature=2.5, top_p=0.9,
         seed=7, seed_logits=16, first_step=0, steps=64, rounded=True),
    dict(name="v50_tiny_temp", vocab=50, drafts=1, sigma=1.0, noise=0.1, temperature=1e-7, top_p=1.0,
         seed=3, seed_logits=17, first_step=0, steps=16),
]


def main():
    R = O.ref()
    if R is None:
        sys.exit("oracle/_ref/libds41_spark_ref.so is not built: make -C oracle ref")
    words = []
    for seed in (0, 1, 0xDEADBEEF, (1 << 63) + 5):
        for step in (0, 1, 12345, (1 << 40) + 3):
            for slot in range(6):
                for purpose in range(4):
                    for draw in (0, 1, 3, 7):
                        w = R.ds41_spark_rng_word_v2(seed, step, slot, purpose, draw)
                        u = R.ds41_spark_uniform_v2(seed, step, slot, purpose, draw)
                        words.append([seed, step, slot, purpose, draw, int(w), float(u).hex()])
    with open(os.path.join(HERE, "philox_v2.json"), "w") as f:
        json.dump({"source": "reference ds41_spark_rng_word_v2 / ds41_spark_uniform_v2 (compiled from "
                             "engine/third_party/spark/src/sampling.cpp)",
                   "fields": ["seed", "step", "slot", "purpose", "draw", "word", "uniform_hex"],
                   "rows": words}, f)
    out = {"source": "reference ds41_spark_probabilities / ds41_spark_sample_v2 / ds41_spark_verify_v2 "
                     "(engine/third_party/spark/src/sampling.cpp, compiled from its sources)",
           "logits": "numpy default_rng([seed_logits, step]); target = N(0,1)*sigma [drafts+1][V] float32; "
                     "draft = float32(target[:drafts] + N(0,1)*noise); see logits_for()",
           "cases": []}
    for case in CASES:
        print("case", case["name"], flush=True)
        c = dict(case)
        c["results"] = run_case(R, case)
        out["cases"].append(c)
    with open(os.path.join(HERE, "accept_v2.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
