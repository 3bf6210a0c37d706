"""The spark GPU sampler over fp32 measures (ds41_spark_verify_gpu_v2 /
ds41_spark_sample_gpu_v2, engine/third_party/spark/src/sampling.cu:6-49) on the
GPU against the oracle's restatement of the reference kernel, through the C ABI.

Bar: accept/reject decisions and token ids bit-exact.
The measures are random fp32 rows whose fp64 sums round, so the kernel's
summation orders (strided mass + tree, chunked draw prefix) are exercised; the
oracle itself is pinned to the compiled reference host sampler on exact sums
(tests/test_oracle_sampler.py)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def measures(rng, rows, V, kind):
    if kind == "softmax":
        x = rng.standard_normal((rows, V)) * 2.5
        return np.exp(x - x.max(axis=1, keepdims=True)).astype(np.float32)
    if kind == "sparse":  # long zero runs: empty chunks, fallbacks to the last positive index
        m = (rng.random((rows, V)) * (rng.random((rows, V)) < 0.01)).astype(np.float32)
        m[:, 0] += 1e-3
        return m
    return rng.random((rows, V)).astype(np.float32) * 1e-3 + np.float32(1e-30)


def run_gpu(gpu, d, q, p, greedy, seed, step):
    import torch
    import ds41_gfx950 as G
    out = torch.full((10,), 7, dtype=torch.int32, device=gpu)
    dd = torch.from_numpy(np.ascontiguousarray(d, np.int32)).to(gpu) if d is not None and len(d) else None
    qd = torch.from_numpy(np.ascontiguousarray(q)).to(gpu) if q is not None else None
    G.verify_gpu_v2(dd, qd, torch.from_numpy(np.ascontiguousarray(p)).to(gpu), greedy, seed, step, out)
    torch.cuda.synchronize()
    return G.result_raw(out)


@pytest.mark.parametrize("V,k,kind", [(129280, 3, "softmax"), (129280, 5, "uniform"), (4097, 2, "sparse"),
                                      (300, 1, "softmax"), (257, 4, "sparse"), (7, 2, "uniform"), (1, 0, "uniform")])
def test_verify_gpu_v2_bitexact_vs_oracle(gpu, V, k, kind):
    rng = np.random.default_rng(V * 10 + k)
    steps = 40 if V > 10000 else 120
    mism = 0
    for step in range(steps):
        p = measures(rng, k + 1, V, kind)
        q = measures(rng, k, V, kind) if k else None
        greedy = int(step % 5 == 4)
        seed = int(rng.integers(0, 1 << 63))
        # drafts as the drafter samples them: from q (slot j, purpose Draft) with the same sampler
        d = np.array([O.sample_gpu_v2(q[j], seed, step, j, 1) for j in range(k)], np.int32)
        want = O.verify_gpu_v2(d, q, p, k, V, greedy, seed, step).raw()
        got = run_gpu(gpu, d, None if greedy else q, p, greedy, seed, step)
        mism += got != want
    assert mism == 0


def test_verify_gpu_v2_invalid_inputs_match_oracle(gpu):
    rng = np.random.default_rng(3)
    V = 5000
    p = measures(rng, 3, V, "softmax")
    q = measures(rng, 2, V, "softmax")
    d = np.array([10, 20], np.int32)
    # a row is checked when the step reaches it (sampling.cu:29-33): row 0 and draft 0 always are
    cases = []
    bad = p.copy(); bad[0, 77] = np.nan; cases.append((d, q, bad))
    neg = p.copy(); neg[0, 5] = -1.0; cases.append((d, q, neg))
    qz = q.copy(); qz[0, 10] = 0.0; cases.append((d, qz, p))
    cases.append((np.array([V, 10], np.int32), q, p))
    zero = p.copy(); zero[0] = 0.0; cases.append((d, q, zero))
    qnan = q.copy(); qnan[0, 3] = np.inf; cases.append((d, qnan, p))
    for dd, qq, pp in cases:
        want = O.verify_gpu_v2(dd, qq, pp, 2, V, 0, 1, 2).raw()
        assert run_gpu(gpu, dd, qq, pp, 0, 1, 2) == want
        assert want[1] == -1
    # an invalid row past the step's end is never read: the step is valid
    late = p.copy(); late[2, 9] = np.nan
    want = O.verify_gpu_v2(np.array([0, 1], np.int32), q, late, 2, V, 0, 1, 2).raw()
    assert run_gpu(gpu, np.array([0, 1], np.int32), q, late, 0, 1, 2) == want


def test_sample_gpu_v2_bitexact_vs_oracle(gpu):
    import torch
    import ds41_gfx950 as G
    rng = np.random.default_rng(4)
    out = torch.zeros(1, dtype=torch.int32, device=gpu)
    for V, kind in ((129280, "softmax"), (1000, "sparse"), (3, "uniform")):
        for step in range(30):
            p = measures(rng, 1, V, kind)[0]
            seed, slot, purpose = int(rng.integers(0, 1 << 63)), step % 6, step % 4
            G.sample_gpu_v2(torch.from_numpy(p).to(gpu), seed, step, slot, purpose, out)
            torch.cuda.synchronize()
            assert int(out.item()) == O.sample_gpu_v2(p, seed, step, slot, purpose), (V, kind, step)
    with pytest.raises(RuntimeError):
        G.sample_gpu_v2(torch.zeros(4, device=gpu), 0, 0, 6, 0, out)  # slot > 5
