"""Token sampling from fp32 logits on the device (ds41_spark_sample_logits_gpu_v2): the engine's
sample(probabilities(x, T, top_p), rng, step, slot, purpose), which SpeculativeStep uses to draw each
draft token (engine/src/speculation.cpp:147-155), through the C ABI.

Bar: tokens bit-exact.
- Every draft token of the committed golden fixtures (tests/golden/accept_v2.json, written by the
  reference's own compiled sampler) on the parallel path and on the forced sequential path.
- The product's host sampler ABI (itself pinned to the reference in test_spark_host.py) on rows with
  ties at the top-p cut, dominant tokens, tiny temperatures, every slot and purpose.
- Invalid rows give -1 and bad arguments are rejected."""
import json
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_accept_golden import logits_for  # noqa: E402

GOLD = json.load(open(os.path.join(HERE, "golden", "accept_v2.json")))
DRAFT = 1


@pytest.mark.parametrize("case", GOLD["cases"], ids=[c["name"] for c in GOLD["cases"]])
def test_draft_tokens_match_reference_golden(gpu, case):
    import torch
    import ds41_gfx950 as G
    k, V, T = case["drafts"], case["vocab"], case["temperature"]
    ws = G.sample_workspace(k, V, gpu)
    out = torch.full((k,), -7, dtype=torch.int32, device=gpu)
    n_exact = 4 if V > 10000 else 16
    for i, e in enumerate(case["results"]):
        _, draft = logits_for(case, e["step"])
        dd = torch.from_numpy(draft).to(gpu)
        for flags in ((0, 1) if i < n_exact else (0,)):
            G.sample_logits(dd, T, case["top_p"], case["seed"], e["step"], 0, DRAFT, out, ws, flags=flags)
            torch.cuda.synchronize()
            assert out.cpu().tolist() == e["drafts"], (e["step"], flags)
    print(f"{case['name']}: {len(case['results'])} steps of {k} draft tokens", flush=True)


def _row(rng, kind, V):
    if kind == "ties":
        return np.round(rng.standard_normal(V) * 2).astype(np.float32)
    if kind == "dominant":
        x = (rng.standard_normal(V) * 0.1).astype(np.float32)
        x[V // 3] = 40.0
        return x
    if kind == "flat":
        x = np.zeros(V, np.float32)
        x[::7] = 0.5
        return x
    return (rng.standard_normal(V) * 2.5).astype(np.float32)


@pytest.mark.parametrize("V", [3, 2049, 129280])
def test_sampling_matches_host_sampler(gpu, V):
    import torch
    import ds41_gfx950 as G
    rng = np.random.default_rng(V)
    rows = 3
    ws = G.sample_workspace(rows, V, gpu)
    out = torch.zeros(rows, dtype=torch.int32, device=gpu)
    checked = 0
    for kind in ("normal", "ties", "dominant", "flat"):
        for T, top_p in ((1.0, 1.0), (1.0, 0.95), (0.7, 0.5), (2.0, 0.999), (1e-6, 1.0), (0.0, 1.0)):
            x = np.stack([_row(rng, kind, V) for _ in range(rows)])
            slot0, purpose, step, seed = int(rng.integers(0, 4)), int(rng.integers(0, 4)), int(rng.integers(1 << 40)), 99
            G.sample_logits(torch.from_numpy(x).to(gpu), T, top_p, seed, step, slot0, purpose, out, ws)
            torch.cuda.synchronize()
            got = out.cpu().tolist()
            t = max(T, 1e-5) if T > 0 else 0.0
            want = []
            for r in range(rows):
                if T == 0:
                    want.append(int(np.argmax(x[r])))
                else:
                    p = G.spark_probabilities(x[r], t, top_p)
                    want.append(G.spark_sample_v2(p, seed, step, slot0 + r, purpose))
            assert got == want, (kind, T, top_p)
            checked += rows
    print(f"V={V}: {checked} tokens equal the host sampler's", flush=True)


def test_sampling_invalid_rows_and_arguments(gpu):
    import torch
    import ds41_gfx950 as G
    V = 5000
    ws = G.sample_workspace(2, V, gpu)
    out = torch.zeros(2, dtype=torch.int32, device=gpu)
    x = np.random.default_rng(1).standard_normal((2, V)).astype(np.float32)
    x[1, 17] = np.nan
    G.sample_logits(torch.from_numpy(x).to(gpu), 1.0, 1.0, 1, 2, 0, DRAFT, out, ws)
    torch.cuda.synchronize()
    got = out.cpu().tolist()
    assert got[1] == -1 and got[0] == G.spark_sample_v2(G.spark_probabilities(x[0], 1.0, 1.0), 1, 2, 0, DRAFT)
    d = torch.from_numpy(x).to(gpu)
    assert G.sample_logits_rc(d, 1.0, 1.0, 1, 2, 5, DRAFT, out, ws) == 1  # slot 5 + 1 row > 5
    assert G.sample_logits_rc(d, 1.0, 1.0, 1, 2, 0, 4, out, ws) == 1      # purpose 4
    assert G.sample_logits_rc(d, -1.0, 1.0, 1, 2, 0, DRAFT, out, ws) == 1
    assert G.sample_logits_rc(d, 1.0, 0.0, 1, 2, 0, DRAFT, out, ws) == 1
    small = torch.zeros(16, dtype=torch.uint8, device=gpu)
    assert G.sample_logits_rc(d, 1.0, 1.0, 1, 2, 0, DRAFT, out, small) == 1
