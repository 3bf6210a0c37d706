"""GPU acceptance sampler vs the reference's host sampler, through the C ABI.

Bar: accept/reject decisions and resampled token ids are
bit-exact given identical fp32 logits and Philox uniforms. The golden results
come from the reference's own compiled sampler (tests/golden/accept_v2.json);
the sequential exact path (flags bit 0) must give the same answers."""
import json
import os
import sys
import zlib

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_accept_golden import logits_for  # noqa: E402

GOLD = json.load(open(os.path.join(HERE, "golden", "accept_v2.json")))
SUPPORTED = GOLD["cases"]
TOP_P = [c for c in GOLD["cases"] if c["top_p"] < 1.0 and c["temperature"] > 0.0]


def run_case(case, gpu, flags, max_steps=None):
    import torch
    import ds41_gfx950 as G
    k, V, T = case["drafts"], case["vocab"], case["temperature"]
    ws = G.accept_workspace(k, V, gpu)
    out = torch.zeros(16, dtype=torch.int32, device=gpu)
    got, want = [], []
    for entry in case["results"][:max_steps]:
        target, draft = logits_for(case, entry["step"])
        td = torch.from_numpy(target).to(gpu)
        dd = torch.from_numpy(draft).to(gpu) if T > 0 else None
        ids = torch.tensor(entry["drafts"], dtype=torch.int32, device=gpu)
        G.verify_logits(td, dd, ids, T, case["top_p"], case["seed"], entry["step"], out, ws, flags=flags)
        torch.cuda.synchronize()
        got.append(G.result_tuple(out))
        want.append((tuple(entry["tokens"]), entry["accepted"], entry["accepted"] + 1, entry["rejected"]))
    return got, want, G.accept_fallbacks(ws, k, V)


@pytest.mark.parametrize("case", SUPPORTED, ids=[c["name"] for c in SUPPORTED])
def test_accept_matches_reference_golden(gpu, case):
    got, want, fallbacks = run_case(case, gpu, flags=0)
    print(f"{case['name']}: {len(got)} steps, sequential-path steps {fallbacks}", flush=True)
    assert got == want


@pytest.mark.parametrize("case", SUPPORTED[:1] + TOP_P + SUPPORTED[-1:], ids=lambda c: c["name"])
def test_accept_exact_path_matches_reference_golden(gpu, case):
    got, want, fallbacks = run_case(case, gpu, flags=1, max_steps=6)
    assert got == want
    assert fallbacks == len(got) or case["temperature"] == 0.0


def test_accept_random_sweep_vs_oracle(gpu):
    """200 fresh steps at the config-2 shape (k=3, V=129280, T=1) against the oracle."""
    import torch
    import ds41_gfx950 as G
    k, V = 3, 129280
    ws = G.accept_workspace(k, V, gpu)
    out = torch.zeros(16, dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(99)
    mism = 0
    for step in range(200):
        target = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
        draft = (target[:k] + rng.standard_normal((k, V)) * 0.5).astype(np.float32)
        q = np.stack([O.probabilities(draft[j], 1.0, 1.0) for j in range(k)])
        drafts = np.array([O.sample_v2(q[j], 5, step, j, 1) for j in range(k)], np.int32)
        ref = O.accept_logits(target, draft, drafts, 1.0, 1.0, 5, step).as_tuple()
        G.verify_logits(torch.from_numpy(target).to(gpu), torch.from_numpy(draft).to(gpu),
                        torch.from_numpy(drafts).to(gpu), 1.0, 1.0, 5, step, out, ws)
        torch.cuda.synchronize()
        mism += G.result_tuple(out) != ref
    print(f"sweep: 200 steps, mismatches {mism}, sequential-path steps {G.accept_fallbacks(ws, k, V)}", flush=True)
    assert mism == 0


def test_accept_rejects_bad_input(gpu):
    import torch
    import ds41_gfx950 as G
    k, V = 1, 4097
    ws = G.accept_workspace(k, V, gpu)
    out = torch.zeros(16, dtype=torch.int32, device=gpu)
    t = torch.zeros((2, V), dtype=torch.float32, device=gpu)
    t[1, 5] = float("nan")
    d = torch.zeros((1, V), dtype=torch.float32, device=gpu)
    G.verify_logits(t, d, torch.tensor([3], dtype=torch.int32, device=gpu), 1.0, 1.0, 0, 0, out, ws)
    torch.cuda.synchronize()
    assert G.result_tuple(out)[1] == -1
    G.take_status()
    for top_p in (0.0, 1.5, float("nan")):
        with pytest.raises(RuntimeError):
            G.verify_logits(t, d, torch.tensor([3], dtype=torch.int32, device=gpu), 1.0, top_p, 0, 0, out, ws)


def oracle_tuple(target, draft, drafts, T, top_p, seed, step):
    """The oracle's result, with the host's input errors (a draft outside q's support) as emitted -1."""
    try:
        return O.accept_logits(target, draft, drafts, T, top_p, seed, step).as_tuple()
    except ValueError:
        return ((), -1, -1, -1)


def sweep_logits(rng, k, V, sigma, noise, shape):
    target = (rng.standard_normal((k + 1, V)) * sigma).astype(np.float32)
    draft = (target[:k] + rng.standard_normal((k, V)) * noise).astype(np.float32)
    if shape == "rounded":  # many exact ties in x, so cuts fall inside tie groups
        target = np.round(target * 2) / 2
        draft = np.round(draft * 2) / 2
    elif shape == "bf16":  # logits that came out of a bf16 GEMM
        target = (target.view(np.uint32) & 0xFFFF0000).view(np.float32)
        draft = (draft.view(np.uint32) & 0xFFFF0000).view(np.float32)
    elif shape == "dominant":  # one token holds nearly all the mass
        target[:, 7] = target.max() + 12.0
        draft[:, 7] = draft.max() + 12.0
    return np.ascontiguousarray(target), np.ascontiguousarray(draft)


TOP_P_SWEEP = [
    # name, drafts, V, T, top_p, sigma, noise, logits shape, steps, drafts drawn from q
    ("v129280_t1_p095", 3, 129280, 1.0, 0.95, 2.5, 0.5, "normal", 24, True),
    ("v4097_t07_p05_rounded", 5, 4097, 0.7, 0.5, 2.0, 0.7, "rounded", 60, True),
    ("v4097_t1_p09_bf16", 2, 4097, 1.0, 0.9, 2.5, 0.4, "bf16", 60, True),
    ("v1000_tiny_t_p09", 1, 1000, 1e-6, 0.9, 1.0, 0.3, "normal", 30, True),
    ("v50000_t13_p099_random_drafts", 4, 50000, 1.3, 0.99, 2.0, 0.5, "normal", 30, False),
    ("v3_p06", 1, 3, 1.0, 0.6, 1.0, 0.5, "normal", 40, True),
    ("v8192_p09_dominant", 2, 8192, 1.0, 0.9, 1.0, 0.5, "dominant", 30, True),
    ("v129280_t2_p03_bf16", 3, 129280, 2.0, 0.3, 3.0, 0.3, "bf16", 12, True),
]


@pytest.mark.parametrize("spec", TOP_P_SWEEP, ids=[s[0] for s in TOP_P_SWEEP])
def test_accept_top_p_sweep_vs_oracle(gpu, spec):
    """Top-p < 1: fresh steps against the oracle (pinned to the reference's compiled sampler), over
    ties, bf16-rounded logits, underflowing temperatures, one dominant token and drafts outside q's
    kept set (an invalid input on the host)."""
    import torch
    import ds41_gfx950 as G
    name, k, V, T, top_p, sigma, noise, shape, steps, from_q = spec
    t = max(T, 1e-5)
    ws = G.accept_workspace(k, V, gpu)
    out = torch.zeros(16, dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    mism, invalid = [], 0
    for step in range(steps):
        target, draft = sweep_logits(rng, k, V, sigma, noise, shape)
        if from_q:
            q = [O.probabilities(draft[j], t, top_p) for j in range(k)]
            drafts = np.array([O.sample_v2(q[j], 11, step, j, 1) for j in range(k)], np.int32)
        else:
            drafts = rng.integers(0, V, k).astype(np.int32)
        ref = oracle_tuple(target, draft, drafts, T, top_p, 11, step)
        invalid += ref[1] == -1
        G.verify_logits(torch.from_numpy(target).to(gpu), torch.from_numpy(draft).to(gpu),
                        torch.from_numpy(drafts).to(gpu), T, top_p, 11, step, out, ws)
        torch.cuda.synchronize()
        got = G.result_tuple(out)
        if got != ref:
            mism.append((step, got, ref))
    print(f"{name}: {steps} steps, invalid inputs {invalid}, sequential-path steps "
          f"{G.accept_fallbacks(ws, k, V)}, mismatches {mism[:3]}", flush=True)
    assert not mism


def test_accept_top_p_exact_path_matches_parallel(gpu):
    """flags bit 0 (every decision on the sequential path: host sort and sums) against the parallel path."""
    import torch
    import ds41_gfx950 as G
    k, V, T, top_p = 3, 20000, 1.0, 0.9
    ws = G.accept_workspace(k, V, gpu)
    a = torch.zeros(16, dtype=torch.int32, device=gpu)
    b = torch.zeros(16, dtype=torch.int32, device=gpu)
    rng = np.random.default_rng(5)
    for step in range(12):
        target, draft = sweep_logits(rng, k, V, 2.0, 0.5, "rounded" if step % 2 else "normal")
        q = [O.probabilities(draft[j], T, top_p) for j in range(k)]
        drafts = np.array([O.sample_v2(q[j], 3, step, j, 1) for j in range(k)], np.int32)
        args = (torch.from_numpy(target).to(gpu), torch.from_numpy(draft).to(gpu), torch.from_numpy(drafts).to(gpu),
                T, top_p, 3, step)
        G.verify_logits(*args, a, ws)
        G.verify_logits(*args, b, ws, flags=1)
        torch.cuda.synchronize()
        ref = oracle_tuple(target, draft, drafts, T, top_p, 3, step)
        assert G.result_tuple(a) == G.result_tuple(b) == ref


def bonus_draws(gpu, target, T, top_p, steps):
    """Bonus-token draws (no drafts) over `steps` Philox steps: GPU vs oracle."""
    import torch
    import ds41_gfx950 as G
    V = target.shape[1]
    ws = G.accept_workspace(0, V, gpu)
    out = torch.zeros(16, dtype=torch.int32, device=gpu)
    td = torch.from_numpy(target).to(gpu)
    got, want = [], []
    for step in range(steps):
        G.verify_logits(td, None, None, T, top_p, 8, step, out, ws)
        torch.cuda.synchronize()
        got.append(G.result_tuple(out)[0])
        want.append(oracle_tuple(target, None, None, T, top_p, 8, step)[0])
    return got, want, G.accept_fallbacks(ws, 0, V)


def test_accept_top_p_signed_zero_ties(gpu):
    """-0.0 and +0.0 are one logit value: the cut inside their tie group keeps the lowest indices."""
    x = np.full((1, 64), -60.0, np.float32)
    x[0, 5:21] = np.where(np.arange(16) % 2, 0.0, -0.0).astype(np.float32)  # 16 zeros, p = 1/16 each
    got, want, _ = bonus_draws(gpu, x, 1.0, 0.3, 64)  # keeps the first 5 zeros (5/16 >= 0.3)
    assert got == want
    assert set(t[0] for t in got) <= set(range(5, 10)) and len(set(t[0] for t in got)) == 5


def test_accept_top_p_distinct_logits_equal_p(gpu):
    """Distinct tiny logits next to a large maximum give exactly equal p on the host; the host's
    stable sort then orders them by index, not by value, and the cut inside that group must follow."""
    x = np.full((1, 32), -80.0, np.float32)
    x[0, 0] = 1.0
    x[0, 1], x[0, 2], x[0, 3] = 1e-30, 3e-30, 2e-30  # one p value on the host, order by index: 1, 2, 3
    got, want, fallbacks = bonus_draws(gpu, x, 1.0, 0.75, 48)  # keeps {0, 1, 2}
    assert got == want
    assert set(t[0] for t in got) == {0, 1, 2}
    assert fallbacks == len(got)  # the near-tie check sends every step down the exact path


def test_accept_top_p_crossing_bin_beyond_lds_list(gpu):
    """Logits within one coarse bin (x in [1, 1.25): the first digit of the key cannot separate them)
    over 20,000 elements: the crossing bin holds far more than the 6,144 elements the finish kernel
    lists in LDS, so its later passes histogram the whole row instead. Draws must still be the
    host's."""
    rng = np.random.default_rng(31)
    x = (1.0 + rng.random((1, 20000)) * 0.2499).astype(np.float32)
    got, want, _ = bonus_draws(gpu, x, 1.0, 0.4, 24)
    assert got == want


def test_accept_top_p_vocabulary_rows_listed_path(gpu):
    """Vocabulary-sized rows (V = 129,280, logits N(0, 2.5^2)): the crossing bin of the first pass
    holds a few hundred elements, listed in LDS for the later passes; draws are the host's at
    top-p 0.95, 0.9 and 0.5."""
    rng = np.random.default_rng(32)
    x = (rng.standard_normal((1, 129280)) * 2.5).astype(np.float32)
    for top_p in (0.95, 0.9, 0.5):
        got, want, _ = bonus_draws(gpu, x, 1.0, top_p, 6)
        assert got == want, top_p


@pytest.mark.parametrize("cluster", [40, 200])
def test_accept_top_p_cluster_of_adjacent_logits(gpu, cluster):
    """`cluster` distinct logits one ulp apart from 5.0 upward (the rest far below) share every key
    bit above the lowest ten, so the first pass leaves exactly that cluster in its crossing bin. With
    40 the finish kernel resolves the range directly; with 200 it is more than the 64 it resolves
    directly, so its histogram passes go on. Draws must be the host's either way."""
    x = np.full((1, 4096), -30.0, np.float32)
    x[0, 100:100 + cluster] = (np.float32(5.0).view(np.uint32) + np.arange(cluster, dtype=np.uint32)).view(np.float32)
    got, want, _ = bonus_draws(gpu, x, 1.0, 0.5, 24)
    assert got == want
    assert all(100 <= t[0] < 100 + cluster for t in got)
