"""ctypes/numpy wrapper of the C oracle (libds41_oracle.so) and of the
reference's own host sampler compiled from its sources (_ref/libds41_spark_ref.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this as the checker / CPU baseline. Product code never
imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libds41_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libds41_spark_ref.so")
_lib = None
_ref = None

P = ctypes.c_void_p


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_e2m1.restype = ctypes.c_float
        L.oracle_e8m0.restype = ctypes.c_float
        L.oracle_e4m3.restype = ctypes.c_float
        L.oracle_e4m3_from_f32.restype = ctypes.c_uint8
        L.oracle_e4m3_from_f32.argtypes = [ctypes.c_float]
        L.oracle_philox_word_v2.restype = ctypes.c_uint32
        L.oracle_philox_word_v2.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                            ctypes.c_uint64]
        L.oracle_uniform_v2.restype = ctypes.c_double
        L.oracle_uniform_v2.argtypes = L.oracle_philox_word_v2.argtypes
        L.oracle_error.restype = ctypes.c_char_p
        L.oracle_probabilities.argtypes = [P, P, ctypes.c_int, ctypes.c_double, ctypes.c_double]
        L.oracle_verify_v2.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                       ctypes.c_uint64, P]
        L.oracle_sample_v2.argtypes = [P, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                       ctypes.c_uint32, P]
        L.oracle_accept_logits.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                           ctypes.c_uint64, ctypes.c_uint64, P, P, P]
        L.oracle_swiglu.argtypes = [P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.oracle_spark_verify_gpu_v2.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                                 ctypes.c_uint64, P]
        L.oracle_spark_sample_gpu_v2.argtypes = [P, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                                 ctypes.c_uint32, P]
        L.oracle_route_weights.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, P]
        _lib = L
    return _lib


def ref():
    """The reference's engine/third_party/spark/src/sampling.cpp, compiled from its own
    sources by `make -C oracle ref`. None when it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = ctypes.CDLL(REF_PATH)
        R.ds41_spark_rng_word_v2.restype = ctypes.c_uint32
        R.ds41_spark_rng_word_v2.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.c_uint64]
        R.ds41_spark_uniform_v2.restype = ctypes.c_double
        R.ds41_spark_uniform_v2.argtypes = R.ds41_spark_rng_word_v2.argtypes
        R.ds41_spark_probabilities.argtypes = [P, P, ctypes.c_int, ctypes.c_double, ctypes.c_double]
        R.ds41_spark_verify_v2.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                           ctypes.c_uint64, P]
        R.ds41_spark_sample_v2.argtypes = [P, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                           ctypes.c_uint32, P]
        R.ds41_spark_error.restype = ctypes.c_char_p
        _ref = R
    return _ref


REFENGINE_PATH = os.path.join(HERE, "_ref", "libds41_refengine.so")
_refengine = None


def refengine():
    """The reference engine's accept sampler (engine/src/sampling.cpp with its 8-thread
    probabilities_rows) behind oracle/refengine_shim.cpp, compiled from the reference sources by
    `make -C oracle ref`. None when it was not built."""
    global _refengine
    if _refengine is None and os.path.exists(REFENGINE_PATH):
        R = ctypes.CDLL(REFENGINE_PATH)
        R.refeng_accept_step.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                         ctypes.c_uint64, ctypes.c_uint64, P, P]
        R.refeng_probabilities.argtypes = [P, ctypes.c_int, ctypes.c_double, ctypes.c_double, P]
        _refengine = R
    return _refengine


def ref_accept_step(target, draft, drafts, temperature, top_p, seed, step):
    """refeng_accept_step: (draft tokens, ds41_spark_result as a tuple), or None when it throws."""
    R = refengine()
    V = target.shape[1]
    d = np.full(max(drafts, 1), -1, np.int32)
    res = SparkResult()
    rc = R.refeng_accept_step(_ptr(np.ascontiguousarray(target, np.float32)),
                              _ptr(None if draft is None else np.ascontiguousarray(draft, np.float32)), drafts, V,
                              temperature, top_p, seed, step, _ptr(d), ctypes.byref(res))
    if rc:
        return None
    return d[:drafts].tolist(), res.as_tuple()


REFPOOL_PATH = os.path.join(HERE, "_ref", "libds41_refpool.so")
_refpool = None


def refpool():
    """The reference's SlotPool and placement parser (components/moe/src/store.cpp, manifest.cpp)
    behind oracle/refpool_shim.cpp, compiled from the reference sources by `make -C oracle ref`.
    None when it was not built."""
    global _refpool
    if _refpool is None and os.path.exists(REFPOOL_PATH):
        R = ctypes.CDLL(REFPOOL_PATH)
        R.refpool_create.restype = ctypes.c_void_p
        R.refpool_create.argtypes = [ctypes.c_size_t, ctypes.c_uint, ctypes.c_uint, ctypes.c_int]
        for f in ("refpool_destroy", "refpool_reset"):
            getattr(R, f).argtypes = [ctypes.c_void_p]
        R.refpool_policy.argtypes = [ctypes.c_void_p, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_uint, ctypes.c_uint,
                                     ctypes.c_int]
        R.refpool_acquire.argtypes = [ctypes.c_void_p, P, ctypes.c_int, ctypes.c_int, P]
        R.refpool_borrow.argtypes = [ctypes.c_void_p, P, ctypes.c_int, P]
        R.refpool_release.argtypes = [ctypes.c_void_p, P, ctypes.c_int]
        R.refpool_touch.argtypes = [ctypes.c_void_p, P, ctypes.c_int]
        for f in ("refpool_pin", "refpool_unpin", "refpool_residency"):
            getattr(R, f).argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        R.refplacement_load.argtypes = [ctypes.c_char_p, P, P, P, P, P, ctypes.c_int, P, P, ctypes.c_int]
        R.refrecords_load.argtypes = [ctypes.c_char_p, ctypes.c_int, P, ctypes.c_int, P, P, P]
        R.refpool_retain.restype = ctypes.c_void_p
        R.refpool_retain.argtypes = [ctypes.c_void_p, ctypes.c_uint32, P]
        R.refpool_token_release.argtypes = [ctypes.c_void_p]
        R.refpool_reserve.argtypes = [ctypes.c_void_p, ctypes.c_size_t, P, ctypes.c_int, P]
        R.refpool_drained.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        R.refpool_peer.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        for f in ("refpool_exclusive", "refpool_fast_minima"):
            getattr(R, f).argtypes = [ctypes.c_void_p, ctypes.c_int]
        R.refpool_decay_interval.argtypes = [ctypes.c_void_p, ctypes.c_uint]
        R.refpool_switch_target_layer.argtypes = [ctypes.c_void_p, P, ctypes.c_int, ctypes.c_uint]
        R.refdrift_create.restype = ctypes.c_void_p
        R.refdrift_create.argtypes = [P, ctypes.c_int, ctypes.c_uint, ctypes.c_uint, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p, P]
        R.refdrift_before.argtypes = [ctypes.c_void_p, P, ctypes.c_int]
        R.refdrift_after.argtypes = [ctypes.c_void_p, P, ctypes.c_int]
        R.refdrift_active.argtypes = [ctypes.c_void_p]
        R.refdrift_tokens.argtypes = [ctypes.c_void_p]
        R.refdrift_tokens.restype = ctypes.c_uint64
        R.refdrift_destroy.argtypes = [ctypes.c_void_p]
        _refpool = R
    return _refpool


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


class SparkResult(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_int32 * 6), ("emitted", ctypes.c_int), ("accepted_drafts", ctypes.c_int),
                ("accepted_input_rows", ctypes.c_int), ("rejected", ctypes.c_int)]

    def as_tuple(self):
        return (tuple(self.tokens[:self.emitted]), self.accepted_drafts, self.accepted_input_rows, self.rejected)

    def raw(self):
        """Every field, including those of an invalid step (emitted == -1)."""
        return (tuple(self.tokens), self.emitted, self.accepted_drafts, self.accepted_input_rows, self.rejected)


class Expert(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in ("gate", "gate_scale", "up", "up_scale", "down", "down_scale")]


class MoeConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("n_experts", ctypes.c_int),
                ("topk", ctypes.c_int), ("score_mode", ctypes.c_int), ("route_scale", ctypes.c_float),
                ("swiglu_limit", ctypes.c_float)]


# ---- formats ---------------------------------------------------------------------
def bf16_bits(x):
    """fp32 array -> bf16 bit patterns (RNE) via the oracle."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.array([lib().oracle_f32_to_bf16(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize_mxfp8(x_bf16_bits):
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // 32), np.uint8)
    if lib().oracle_quantize_mxfp8(_ptr(x), _ptr(q), _ptr(s), rows, cols):
        raise ValueError("oracle_quantize_mxfp8")
    return q, s


def dequant_mxfp4(w, s, n, k):
    out = np.empty((n, k), np.float32)
    lib().oracle_dequant_mxfp4(_ptr(np.ascontiguousarray(w)), _ptr(np.ascontiguousarray(s)), n, k, _ptr(out))
    return out


def mxfp4_gemm(w, ws, xq, xs, m, n, k):
    """Returns (fp32 accumulators [m][n], bf16 bits [m][n])."""
    acc = np.empty((m, n), np.float32)
    out = np.empty((m, n), np.uint16)
    rc = lib().oracle_mxfp4_gemm(_ptr(np.ascontiguousarray(w)), _ptr(np.ascontiguousarray(ws)),
                                 _ptr(np.ascontiguousarray(xq)), _ptr(np.ascontiguousarray(xs)), m, n, k,
                                 _ptr(acc), _ptr(out))
    if rc:
        raise ValueError("oracle_mxfp4_gemm")
    return acc, out


def set_threads(n):
    lib().oracle_set_threads(int(n))


def swiglu(g_bits, u_bits, w, limit):
    g = np.ascontiguousarray(g_bits, np.uint16)
    u = np.ascontiguousarray(u_bits, np.uint16)
    rows, cols = g.shape
    out = np.empty_like(g)
    wv = None if w is None else np.ascontiguousarray(w, np.float32)
    lib().oracle_swiglu(_ptr(g), _ptr(u), _ptr(wv), _ptr(out), rows, cols, limit)
    return out


# ---- router / plan / reduce ------------------------------------------------------
def router_logits(x_bits, wg):
    x = np.ascontiguousarray(x_bits, np.uint16)
    wg = np.ascontiguousarray(wg, np.float32)
    m, h = x.shape
    e = wg.shape[0]
    out = np.empty((m, e), np.float32)
    lib().oracle_router_logits(_ptr(x), _ptr(wg), m, e, h, _ptr(out))
    return out


def router_scores(logits, bias, mode=0):
    logits = np.ascontiguousarray(logits, np.float32)
    m, n = logits.shape
    u = np.empty_like(logits)
    b = np.empty_like(logits)
    lib().oracle_router_scores(_ptr(logits), _ptr(np.ascontiguousarray(bias, np.float32)), m, n, mode, _ptr(u),
                               _ptr(b))
    return u, b


def topk(b, k):
    b = np.ascontiguousarray(b, np.float32)
    m, n = b.shape
    ids = np.empty((m, k), np.int32)
    lib().oracle_topk(_ptr(b), m, n, k, _ptr(ids))
    return ids


def spark_topk3(scores):
    """Drafter router top-3 with CUDA torch.topk's tie order (spark forward.cu:28-40)."""
    s = np.ascontiguousarray(scores, np.float32)
    m = s.shape[0]
    assert s.shape[1] == 128
    ids = np.empty((m, 3), np.int32)
    lib().oracle_spark_topk3(_ptr(s), m, _ptr(ids))
    return ids


def route_weights(u, ids, scale=1.5):
    u = np.ascontiguousarray(u, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    m, n = u.shape
    k = ids.shape[1]
    w = np.empty((m, k), np.float32)
    lib().oracle_route_weights(_ptr(u), _ptr(ids), m, n, k, scale, _ptr(w))
    return w


def plan_routes(selected, n_experts):
    sel = np.ascontiguousarray(selected, np.int32)
    rows, topk_ = sel.shape
    total = rows * topk_
    ids, begin, count, src, dst = (np.empty(total, np.int32) for _ in range(5))
    u = lib().oracle_plan_routes(_ptr(sel), rows, topk_, n_experts, _ptr(ids), _ptr(begin), _ptr(count), _ptr(src),
                                 _ptr(dst))
    if u < 0:
        raise ValueError("invalid route")
    return ids[:u], begin[:u], count[:u], src, dst


def reduce_experts(routed_bits, ids, shared_bits):
    r = np.ascontiguousarray(routed_bits, np.uint16)
    rows, k, h = r.shape
    out = np.empty((rows, h), np.uint16)
    sh = None if shared_bits is None else np.ascontiguousarray(shared_bits, np.uint16)
    if lib().oracle_reduce_experts(_ptr(r), _ptr(np.ascontiguousarray(ids, np.int32)), _ptr(sh), _ptr(out), rows, k,
                                   h):
        raise ValueError("duplicate route ids")
    return out


def _expert_struct(e):
    return Expert(*[e[f].ctypes.data for f in ("gate", "gate_scale", "up", "up_scale", "down", "down_scale")])


def expert_ffn(e, xq, xs, route_w, hidden, inter, limit=10.0, return_acc=False):
    """One expert on quantised rows -> bf16 bits [m][hidden] (and, with return_acc, the down
    projection's fp32 accumulators [m][hidden] that round to them)."""
    m = xq.shape[0]
    out = np.empty((m, hidden), np.uint16)
    acc = np.empty((m, hidden), np.float32) if return_acc else None
    es = _expert_struct(e)
    wv = None if route_w is None else np.ascontiguousarray(route_w, np.float32)
    rc = lib().oracle_expert_ffn(ctypes.byref(es), _ptr(np.ascontiguousarray(xq)), _ptr(np.ascontiguousarray(xs)),
                                 _ptr(wv), m, hidden, inter, ctypes.c_float(limit), _ptr(out), _ptr(acc))
    if rc:
        raise ValueError("oracle_expert_ffn")
    return (out, acc) if return_acc else out


def dense_fp8(w, ws, xq, xs, m, n, k):
    """W8A8 FP8 projection (32 x 32 block weight scales) -> (fp32 acc, bf16 bits) [m][n]."""
    acc = np.empty((m, n), np.float32)
    out = np.empty((m, n), np.uint16)
    rc = lib().oracle_dense_fp8(_ptr(np.ascontiguousarray(w)), _ptr(np.ascontiguousarray(ws)),
                                _ptr(np.ascontiguousarray(xq)), _ptr(np.ascontiguousarray(xs)), m, n, k, _ptr(acc),
                                _ptr(out))
    if rc:
        raise ValueError("oracle_dense_fp8")
    return acc, out


def shared_fp8_ffn(e, xq, xs, hidden, inter):
    """FP8 shared expert on quantised rows -> bf16 bits [m][hidden]."""
    m = xq.shape[0]
    out = np.empty((m, hidden), np.uint16)
    es = _expert_struct(e)
    rc = lib().oracle_shared_fp8_ffn(ctypes.byref(es), _ptr(np.ascontiguousarray(xq)), _ptr(np.ascontiguousarray(xs)),
                                     m, hidden, inter, _ptr(out))
    if rc:
        raise ValueError("oracle_shared_fp8_ffn")
    return out


def moe_layer(x_bits, router_w, router_bias, experts, shared, hidden, inter, topk_=6, score_mode=0,
              route_scale=1.5, swiglu_limit=10.0, threads=0):
    """experts: list (len n_experts) of dicts of numpy arrays, or None for absent ones
    (an absent expert that gets routed raises). Returns (y bits, ids, weights, logits)."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    m = x.shape[0]
    E = len(experts)
    arr = (Expert * E)()
    for i, e in enumerate(experts):
        if e is not None:
            arr[i] = _expert_struct(e)
    cfg = MoeConfig(hidden, inter, E, topk_, score_mode, route_scale, swiglu_limit)
    y = np.empty((m, hidden), np.uint16)
    ids = np.empty((m, topk_), np.int32)
    w = np.empty((m, topk_), np.float32)
    logits = np.empty((m, E), np.float32)
    sh = ctypes.byref(_expert_struct(shared)) if shared is not None else ctypes.c_void_p(0)
    rc = lib().oracle_moe_layer(ctypes.byref(cfg), _ptr(x), _ptr(np.ascontiguousarray(router_w, np.float32)),
                                _ptr(np.ascontiguousarray(router_bias, np.float32)), arr, sh, m, _ptr(y), _ptr(ids),
                                _ptr(w), _ptr(logits), threads)
    if rc:
        raise ValueError("oracle_moe_layer")
    return y, ids, w, logits


def moe_layer_routed(x_bits, ids, weights, experts, shared, hidden, inter, swiglu_limit=10.0, threads=0):
    """Layer output given the routing (ids/weights [m][topk]); experts as in moe_layer."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    ids = np.ascontiguousarray(ids, np.int32)
    m, k = ids.shape
    E = len(experts)
    arr = (Expert * E)()
    for i, e in enumerate(experts):
        if e is not None:
            arr[i] = _expert_struct(e)
    cfg = MoeConfig(hidden, inter, E, k, 0, 1.5, swiglu_limit)
    y = np.empty((m, hidden), np.uint16)
    sh = ctypes.byref(_expert_struct(shared)) if shared is not None else ctypes.c_void_p(0)
    rc = lib().oracle_moe_layer_routed(ctypes.byref(cfg), _ptr(x), _ptr(ids),
                                       _ptr(np.ascontiguousarray(weights, np.float32)), arr, sh, m, _ptr(y), threads)
    if rc:
        raise ValueError("oracle_moe_layer_routed")
    return y


# ---- sampler -----------------------------------------------------------------------
def probabilities(x, t, top_p):
    x = np.ascontiguousarray(x, np.float32)
    p = np.empty(x.shape[0], np.float64)
    if lib().oracle_probabilities(_ptr(x), _ptr(p), x.shape[0], t, top_p):
        raise ValueError(lib().oracle_error().decode())
    return p


def verify_v2(d, q, p, count, n, greedy, seed, step):
    r = SparkResult()
    d = np.ascontiguousarray(d, np.int32) if d is not None else None
    q = np.ascontiguousarray(q, np.float64) if q is not None else None
    if lib().oracle_verify_v2(_ptr(d), _ptr(q), _ptr(np.ascontiguousarray(p, np.float64)), count, n, greedy, seed,
                              step, ctypes.byref(r)):
        raise ValueError(lib().oracle_error().decode())
    return r


def accept_logits(target, draft, drafts, temperature, top_p, seed, step):
    target = np.ascontiguousarray(target, np.float32)
    count = target.shape[0] - 1
    n = target.shape[1]
    r = SparkResult()
    dl = np.ascontiguousarray(draft, np.float32) if draft is not None and count else None
    d = np.ascontiguousarray(drafts, np.int32) if count else None
    if lib().oracle_accept_logits(_ptr(target), _ptr(dl), _ptr(d), count, n, temperature, top_p, seed, step,
                                  ctypes.byref(r), ctypes.c_void_p(0), ctypes.c_void_p(0)):
        raise ValueError(lib().oracle_error().decode())
    return r


def verify_gpu_v2(d, q, p, count, n, greedy, seed, step):
    """The reference GPU sampler's arithmetic over fp32 measures (sampling.cu:6-39)."""
    r = SparkResult()
    d = np.ascontiguousarray(d, np.int32) if d is not None else None
    q = np.ascontiguousarray(q, np.float32) if q is not None else None
    if lib().oracle_spark_verify_gpu_v2(_ptr(d), _ptr(q), _ptr(np.ascontiguousarray(p, np.float32)), count, n,
                                        greedy, seed, step, ctypes.byref(r)):
        raise ValueError(lib().oracle_error().decode())
    return r


def sample_gpu_v2(p, seed, step, slot, purpose):
    out = ctypes.c_int32(-2)
    p = np.ascontiguousarray(p, np.float32)
    if lib().oracle_spark_sample_gpu_v2(_ptr(p), p.shape[0], seed, step, slot, purpose, ctypes.byref(out)):
        raise ValueError(lib().oracle_error().decode())
    return out.value


def sample_v2(p, seed, step, slot, purpose):
    out = ctypes.c_int32(-1)
    p = np.ascontiguousarray(p, np.float64)
    if lib().oracle_sample_v2(_ptr(p), p.shape[0], seed, step, slot, purpose, ctypes.byref(out)):
        raise ValueError(lib().oracle_error().decode())
    return out.value
