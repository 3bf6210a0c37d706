"""Pins the oracle's MoE arithmetic: the W4A8 group-serial GEMM against a
pure-Python restatement and closed forms, top-k against a brute-force sort,
the route-weight summation order against its formula, the route plan against
the invariants of the reference's engine/tests/route_plan.cpp, and the ordered
reduction against an explicit loop."""
import numpy as np
import pytest

import oracle as O

E2M1 = [0, .5, 1, 1.5, 2, 3, 4, 6]


def e2m1(c):
    return (-1 if c & 8 else 1) * E2M1[c & 7]


def e4m3(b):
    s, e, m = b >> 7, (b >> 3) & 15, b & 7
    v = m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10)
    return -v if s else v


def rand_mx(rng, n, k, scale_lo=119, scale_hi=123):
    w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = rng.integers(scale_lo, scale_hi + 1, (n, k // 32), dtype=np.uint8)
    return w, s


def rand_x8(rng, m, k):
    x = rng.integers(0, 256, (m, k), dtype=np.uint8)
    x[(x & 0x7F) == 0x7F] = 0x00  # no NaN codes
    xs = rng.integers(120, 130, (m, k // 32), dtype=np.uint8)
    return x, xs


def python_gemm(w, ws, x, xs, m, n, k):
    """mxfp4.cu:46-95 restated with Python floats: exact group dot, one fp32 rounding,
    two fp32 scalings, serial fp32 add."""
    f = np.float32
    out = np.zeros((m, n), np.float32)
    for t in range(m):
        for r in range(n):
            acc = f(0)
            for g in range(k // 32):
                dot = 0.0
                for i in range(32):
                    byte = int(w[r, g * 16 + i // 2])
                    nib = byte >> 4 if i & 1 else byte & 15
                    dot += e4m3(int(x[t, g * 32 + i])) * e2m1(nib)
                sx = f(2.0 ** (int(xs[t, g]) - 127))
                sw = f(2.0 ** (int(ws[r, g]) - 127))
                acc = f(acc + f(f(f(dot) * sx) * sw))
            out[t, r] = acc
    return out


@pytest.mark.parametrize("m,n,k", [(1, 3, 32), (2, 5, 96), (3, 4, 160)])
def test_gemm_vs_python(m, n, k):
    rng = np.random.default_rng(m * 100 + n)
    w, ws = rand_mx(rng, n, k)
    x, xs = rand_x8(rng, m, k)
    acc, out = O.mxfp4_gemm(w, ws, x, xs, m, n, k)
    ref = python_gemm(w, ws, x, xs, m, n, k)
    assert np.array_equal(acc, ref)
    assert np.array_equal(out, O.bf16_bits(ref))


def test_gemm_one_hot_picks_activation_and_scales():
    # weight one-hot 1.0 (code 2) at element j of row r -> out = x[j] * 2^(sx-127) * 2^(sw-127)
    k, n = 64, 64
    w = np.zeros((n, k // 2), np.uint8)
    for r in range(n):
        j = r
        w[r, j // 2] = (2 << 4) if j & 1 else 2
    ws = np.full((n, k // 32), 127, np.uint8)
    ws[:, 1] = 129
    x = np.arange(k, dtype=np.uint8).reshape(1, k) % 0x7E
    xs = np.array([[125, 131]], np.uint8)
    acc, _ = O.mxfp4_gemm(w, ws, x, xs, 1, n, k)
    for r in range(n):
        g = r // 32
        expect = e4m3(int(x[0, r])) * 2.0 ** (int(xs[0, g]) - 127) * 2.0 ** (int(ws[r, g]) - 127)
        assert acc[0, r] == np.float32(expect)


def test_gemm_scale_linearity():
    rng = np.random.default_rng(11)
    w, ws = rand_mx(rng, 8, 128)
    x, xs = rand_x8(rng, 2, 128)
    a0, _ = O.mxfp4_gemm(w, ws, x, xs, 2, 8, 128)
    a1, _ = O.mxfp4_gemm(w, ws + 1, x, xs, 2, 8, 128)
    assert np.array_equal(a1, a0 * 2)  # power-of-two rescaling is exact


def test_gemm_rejects_bad_k():
    with pytest.raises(ValueError):
        O.mxfp4_gemm(np.zeros((1, 8), np.uint8), np.zeros((1, 1), np.uint8), np.zeros((1, 16), np.uint8),
                      np.zeros((1, 1), np.uint8), 1, 1, 16)


def test_topk_vs_bruteforce_with_ties():
    rng = np.random.default_rng(5)
    for trial in range(50):
        b = rng.standard_normal((4, 384)).astype(np.float32)
        b[:, rng.integers(0, 384, 40)] = b[0, 3]  # ties, lower id must win
        if trial % 3 == 0:
            b = np.round(b, 1).astype(np.float32)
        ids = O.topk(b, 6)
        for r in range(4):
            order = sorted(range(384), key=lambda i: (-float(b[r, i]), i))
            assert list(ids[r]) == order[:6]


def test_route_weights_order():
    f = np.float32
    rng = np.random.default_rng(9)
    u = (rng.random((64, 16)) * 3).astype(np.float32)
    ids = np.stack([rng.permutation(16)[:6] for _ in range(64)]).astype(np.int32)
    w = O.route_weights(u, ids, 1.5)
    differs = 0
    for r in range(64):
        s = [u[r, i] for i in ids[r]]
        total = f(f(f(f(s[0] + s[4]) + s[2]) + f(f(s[1] + s[5]) + s[3])) + f(1e-20))
        for i in range(6):
            assert w[r, i] == f(f(s[i] / total) * f(1.5))
        naive = f(0)
        for v in s:
            naive = f(naive + v)
        differs += naive != f(f(f(s[0] + s[4]) + s[2]) + f(f(s[1] + s[5]) + s[3]))
    assert differs > 0  # the fixed order is observable on these inputs
    # k = 3: (v0 + v2) + v1
    ids3 = ids[:, :3].copy()
    w3 = O.route_weights(u, ids3, 1.5)
    for r in range(64):
        s = [u[r, i] for i in ids3[r]]
        total = f(f(f(s[0] + s[2]) + s[1]) + f(1e-20))
        assert all(w3[r, i] == f(f(s[i] / total) * f(1.5)) for i in range(3))


def test_router_scores_closed_form():
    z = np.array([[-30, -5, -1e-3, 0, 1e-3, 5, 19.99, 20, 20.5, 80]], np.float32)
    bias = np.linspace(-1, 1, 10).astype(np.float32)
    u, b = O.router_scores(z, bias)
    zz = z.astype(np.float64)
    ref = np.sqrt(np.where(zz > 20, zz, np.log1p(np.exp(zz))))
    assert np.allclose(u, ref, rtol=2e-7, atol=0)
    assert u[0, 8] == np.float32(np.sqrt(np.float32(20.5)))  # pass-through above 20
    assert np.array_equal(b, (u + bias).astype(np.float32))
    us, _ = O.router_scores(z, bias, mode=1)
    assert np.allclose(us, 1 / (1 + np.exp(-zz)), rtol=2e-7, atol=1e-30)


def test_router_logits_double_sum():
    rng = np.random.default_rng(1)
    x = O.bf16_bits(rng.standard_normal((2, 256)).astype(np.float32))
    wg = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    got = O.router_logits(x, wg)
    ref = (O.bf16_to_f32(x).astype(np.float64) @ wg.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(got, ref)


def test_plan_routes_invariants():
    # engine/tests/route_plan.cpp: random routings, every slot once, ids ascending, rows contiguous
    rng = np.random.default_rng(2026)
    for _ in range(2000):
        rows = int(rng.integers(1, 7))
        sel = np.stack([rng.permutation(384)[:6] for _ in range(rows)]).astype(np.int32)
        if rng.random() < 0.5:  # concentrate on few experts to force sharing
            sel = np.stack([rng.permutation(12)[:6] for _ in range(rows)]).astype(np.int32)
        ids, begin, count, src, dst = O.plan_routes(sel, 384)
        assert np.all(np.diff(ids) > 0)
        assert sorted(dst.tolist()) == list(range(rows * 6))
        assert np.all(src == dst // 6)
        assert begin[0] == 0 and np.all(begin[1:] == np.cumsum(count)[:-1]) and count.sum() == rows * 6
        flat = sel.ravel()
        for e, b0, c in zip(ids, begin, count):
            seg = dst[b0:b0 + c]
            assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)  # stable within an expert


def test_plan_routes_rejects_duplicates_and_range():
    with pytest.raises(ValueError):
        O.plan_routes(np.array([[1, 2, 3, 4, 5, 1]], np.int32), 384)
    with pytest.raises(ValueError):
        O.plan_routes(np.array([[1, 2, 3, 4, 5, 384]], np.int32), 384)
    O.plan_routes(np.array([[1, 2, 3, 4, 5, 6], [1, 2, 3, 4, 5, 6]], np.int32), 384)  # across tokens: fine


def test_reduce_ascending_order_and_shared_last():
    f = np.float32
    rng = np.random.default_rng(4)
    rows, k, h = 3, 6, 16
    routed = O.bf16_bits((rng.standard_normal((rows, k, h)) * 10.0 ** rng.integers(-3, 4, (rows, k, 1))).astype(np.float32))
    shared = O.bf16_bits(rng.standard_normal((rows, h)).astype(np.float32))
    ids = np.stack([rng.permutation(384)[:6] for _ in range(rows)]).astype(np.int32)
    out = O.reduce_experts(routed, ids, shared)
    rv = O.bf16_to_f32(routed)
    sv = O.bf16_to_f32(shared)
    for t in range(rows):
        order = np.argsort(ids[t], kind="stable")
        for j in range(h):
            acc = f(0)
            for i in order:
                acc = f(acc + rv[t, i, j])
            acc = f(acc + sv[t, j])
            assert out[t, j] == O.bf16_bits(np.array([acc], np.float32))[0]
    with pytest.raises(ValueError):
        O.reduce_experts(routed, np.array([[1, 1, 2, 3, 4, 5]] * rows, np.int32), shared)


def test_swiglu_formula():
    f = np.float32
    rng = np.random.default_rng(8)
    g = O.bf16_bits((rng.standard_normal((4, 64)) * 8).astype(np.float32))
    u = O.bf16_bits((rng.standard_normal((4, 64)) * 8).astype(np.float32))
    w = rng.random(4).astype(np.float32)
    out = O.swiglu(g, u, w, 10.0)
    gv, uv = O.bf16_to_f32(g), O.bf16_to_f32(u)
    ref = np.empty((4, 64), np.float32)
    for r in range(4):
        for c in range(64):
            gg = min(gv[r, c], f(10))
            uu = min(f(10), max(f(-10), uv[r, c]))
            den = f(1 + np.exp(-np.float64(gg)))  # fp64 exp, fp32 rounding
            ref[r, c] = f(w[r] * f(f(gg / den) * uu))
    # expf(-g) in fp32 vs fp64-then-round can differ by 1 ulp; bf16 outputs agree
    diff = np.abs(O.bf16_to_f32(out) - O.bf16_to_f32(O.bf16_bits(ref)))
    assert np.mean(diff == 0) > 0.99
    assert np.all(diff <= np.abs(O.bf16_to_f32(out)) * 2 ** -7)


def test_spark_topk3_distinct_is_descending_top3():
    """Distinct scores: the drafter's top-3 is the three largest, largest first, for one row
    (4-entry network) and for several rows (32-entry network)."""
    rng = np.random.default_rng(41)
    for m in (1, 5):
        s = rng.permutation(np.arange(m * 128, dtype=np.float32)).reshape(m, 128) * np.float32(0.37) - 9.0
        want = np.argsort(-s, axis=1, kind="stable")[:, :3].astype(np.int32)
        assert np.array_equal(O.spark_topk3(s), want)


def test_spark_topk3_tie_orders():
    """The reference states (spark forward.cu:30-33) that the several-row network reverses a
    tied pair above the threshold; the one-row network keeps gather order for it. Equal
    values never change the chosen multiset of scores."""
    s = np.zeros((1, 128), np.float32)
    s[0, 10] = s[0, 20] = 5.0
    s[0, 30] = 1.0
    assert O.spark_topk3(s).tolist() == [[10, 20, 30]]
    assert O.spark_topk3(np.repeat(s, 3, 0)).tolist() == [[20, 10, 30]] * 3
    rng = np.random.default_rng(42)
    for m in (1, 2, 7):
        s = rng.integers(0, 4, (m, 128)).astype(np.float32)
        ids = O.spark_topk3(s)
        for r in range(m):
            vals = s[r, ids[r]]
            assert len(set(ids[r].tolist())) == 3
            assert np.all(vals[:-1] >= vals[1:])
            assert sorted(vals.tolist()) == sorted(np.sort(s[r])[-3:].tolist())


def rand_e4m3(rng, shape):
    """Random E4M3 codes without the NaN codes 0x7f / 0xff."""
    b = rng.integers(0, 256, shape, dtype=np.uint8)
    b[(b & 0x7F) == 0x7F] = 0x3C
    return b


def python_dense_fp8(w, ws, x, xs, m, n, k):
    """dense.cu:37-91 restated with Python floats: exact K32 dot of decoded E4M3 pairs, one fp32
    rounding, times the activation then the 32x32-block weight scale in fp32, serial fp32 add."""
    f = np.float32
    ng = k // 32
    out = np.zeros((m, n), np.float32)
    for t in range(m):
        for r in range(n):
            acc = f(0)
            for g in range(ng):
                dot = sum(e4m3(int(x[t, 32 * g + i])) * e4m3(int(w[r, 32 * g + i])) for i in range(32))
                sx = f(2.0 ** (int(xs[t, g]) - 127))
                sw = f(2.0 ** (int(ws[r // 32, g]) - 127))
                acc = f(acc + f(f(f(dot) * sx) * sw))
            out[t, r] = acc
    return out


@pytest.mark.parametrize("m,n,k", [(1, 32, 32), (3, 64, 96), (2, 96, 160)])
def test_dense_fp8_vs_python(m, n, k):
    rng = np.random.default_rng(m * 100 + n + k)
    w = rand_e4m3(rng, (n, k))
    ws = rng.integers(118, 130, (n // 32, k // 32), dtype=np.uint8)
    x = rand_e4m3(rng, (m, k))
    xs = rng.integers(118, 130, (m, k // 32), dtype=np.uint8)
    acc, bits = O.dense_fp8(w, ws, x, xs, m, n, k)
    want = python_dense_fp8(w, ws, x, xs, m, n, k)
    assert np.array_equal(acc.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(bits, O.bf16_bits(want))


def test_dense_fp8_one_hot_block_scales():
    """One nonzero weight (row r, column c) and one nonzero activation at c: y[r] is their product
    times 2^(sx-127) * 2^(sw-127) with sw the scale of block (r // 32, c // 32); other rows are 0."""
    m, n, k = 1, 96, 128
    for r, c in ((0, 0), (33, 70), (95, 127)):
        w = np.zeros((n, k), np.uint8)
        w[r, c] = 0x48  # 2^(9-7) * 1 = 4
        x = np.zeros((m, k), np.uint8)
        x[0, c] = 0xB4  # -(1 + 4/8) * 2^(6-7) = -0.75
        ws = np.arange(n // 32 * (k // 32), dtype=np.uint8).reshape(n // 32, k // 32) + 120
        xs = np.full((m, k // 32), 127, np.uint8)
        xs[0, c // 32] = 129
        acc, _ = O.dense_fp8(w, ws, x, xs, m, n, k)
        want = 4.0 * -0.75 * 2.0 ** 2 * 2.0 ** (int(ws[r // 32, c // 32]) - 127)
        assert acc[0, r] == np.float32(want)
        assert np.count_nonzero(acc) == 1
