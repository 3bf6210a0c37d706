"""ctypes binding of libds41_gfx950.so (the gfx950 verify-path library).

The C ABI (include/ds41_moe_gfx950.h, include/ds41_accept_gfx950.h) takes plain
device pointers; torch is used here only to own device memory and streams.
Every call raises if the library is missing or returns a HIP error: there is
no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libds41_gfx950.so")
_lib = None

PROJ_GATE, PROJ_UP, PROJ_DOWN = 0, 1, 2


class DeviceExpert(ctypes.Structure):
    """components/moe/include/ds41/store.hpp:110-117 (64 bytes)."""
    _fields_ = [("gate", ctypes.c_void_p), ("gate_scale", ctypes.c_void_p),
                ("up", ctypes.c_void_p), ("up_scale", ctypes.c_void_p),
                ("down", ctypes.c_void_p), ("down_scale", ctypes.c_void_p),
                ("ready", ctypes.c_void_p), ("generation", ctypes.c_uint32),
                ("slot", ctypes.c_int32)]


class GemmJob(ctypes.Structure):
    """components/moe/include/ds41/kernels.cuh:8-13 (32 bytes)."""
    _fields_ = [("expert", ctypes.c_uint32), ("tokens", ctypes.c_int32),
                ("x", ctypes.c_void_p), ("x_scale", ctypes.c_void_p),
                ("output", ctypes.c_void_p)]


ABI_VERSION = 1  # DS41_GFX950_ABI_VERSION
_ABI_FIELDS = [("abi_version", ctypes.c_uint32), ("struct_bytes", ctypes.c_uint32)]


class _Versioned(ctypes.Structure):
    """A struct that begins with abi_version and struct_bytes (filled in here; the other fields
    follow positionally or by name)."""

    def __init__(self, *args, **kw):
        super().__init__(ABI_VERSION, ctypes.sizeof(type(self)), *args, **kw)

    @classmethod
    def data_fields(cls):
        return [f for f, _ in cls._fields_ if f not in ("abi_version", "struct_bytes")]


class MoeLayerArgs(_Versioned):
    _fields_ = _ABI_FIELDS + [("x_bf16", ctypes.c_void_p), ("router_w", ctypes.c_void_p),
                ("router_bias", ctypes.c_void_p), ("table", ctypes.c_void_p),
                ("expert_base", ctypes.c_int32), ("shared_index", ctypes.c_int32),
                ("tokens", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("inter", ctypes.c_int32), ("n_experts", ctypes.c_int32),
                ("topk", ctypes.c_int32), ("score_mode", ctypes.c_int32),
                ("route_scale", ctypes.c_float), ("swiglu_limit", ctypes.c_float),
                ("y_bf16", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_size_t), ("ids_out", ctypes.c_void_p),
                ("weights_out", ctypes.c_void_p), ("logits_out", ctypes.c_void_p),
                ("stage_events", ctypes.c_void_p), ("stage_mask", ctypes.c_uint32),
                ("shared_fp8", ctypes.c_void_p), ("weight_layout", ctypes.c_int32)]


class MoePrefillArgs(ctypes.Structure):
    _fields_ = [("x_bf16", ctypes.c_void_p), ("ids", ctypes.c_void_p), ("weights", ctypes.c_void_p),
                ("table", ctypes.c_void_p), ("expert_base", ctypes.c_int32), ("shared_index", ctypes.c_int32),
                ("tokens", ctypes.c_int32), ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
                ("n_experts", ctypes.c_int32), ("topk", ctypes.c_int32), ("swiglu_limit", ctypes.c_float),
                ("y_bf16", ctypes.c_void_p), ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("stage_events", ctypes.c_void_p)]


class ExpertLayout(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_uint64 * 6), ("bytes", ctypes.c_uint64)]


class StackLayer(ctypes.Structure):
    _fields_ = [("router_w", ctypes.c_void_p), ("router_bias", ctypes.c_void_p), ("table", ctypes.c_void_p),
                ("expert_base", ctypes.c_int32), ("shared_index", ctypes.c_int32),
                ("host_index", ctypes.c_void_p), ("host_slabs", ctypes.c_void_p),
                ("host_slab_count", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class StackDesc(_Versioned):
    _fields_ = _ABI_FIELDS + [("layers", ctypes.c_int32), ("max_tokens", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("inter", ctypes.c_int32), ("n_experts", ctypes.c_int32), ("topk", ctypes.c_int32),
                ("score_mode", ctypes.c_int32), ("route_scale", ctypes.c_float), ("swiglu_limit", ctypes.c_float),
                ("layer", ctypes.POINTER(StackLayer)), ("weight_layout", ctypes.c_int32)]


class StackStats(_Versioned):
    _fields_ = _ABI_FIELDS + [("steps", ctypes.c_uint64), ("layers", ctypes.c_uint64), ("resident_routed", ctypes.c_uint64),
                ("host_fetched", ctypes.c_uint64), ("h2d_bytes", ctypes.c_uint64),
                ("invalid_layers", ctypes.c_uint64), ("cached_routed", ctypes.c_uint64)]


assert ctypes.sizeof(DeviceExpert) == 64 and ctypes.sizeof(GemmJob) == 32
assert ctypes.sizeof(StackLayer) == 56 and ctypes.sizeof(ExpertLayout) == 56


class SparkResult(ctypes.Structure):
    """engine/third_party/spark/include/ds41/spark.h ds41_spark_result."""
    _fields_ = [("tokens", ctypes.c_int32 * 6), ("emitted", ctypes.c_int),
                ("accepted_drafts", ctypes.c_int), ("accepted_input_rows", ctypes.c_int),
                ("rejected", ctypes.c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.ds41_moe_layer_workspace_bytes.restype = ctypes.c_size_t
        _lib.ds41_moe_layer_noalloc_max_bytes.restype = ctypes.c_size_t
        _lib.ds41_drift_completed_tokens.restype = ctypes.c_uint64
        _lib.ds41_drift_error.restype = ctypes.c_char_p
        _lib.ds41_moe_prefill_workspace_bytes.restype = ctypes.c_size_t
        _lib.ds41_gfx950_version.restype = ctypes.c_char_p
        _lib.ds41_spark_accept_workspace_bytes.restype = ctypes.c_size_t
        _lib.ds41_spark_sample_workspace_bytes.restype = ctypes.c_size_t
        _lib.ds41_spark_sample_logits_gpu_v2.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_uint64,
            ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
            ctypes.c_int, ctypes.c_void_p]
        _lib.ds41_spark_error.restype = ctypes.c_char_p
        _lib.ds41_spark_rng_word_v2.restype = ctypes.c_uint32
        _lib.ds41_spark_uniform_v2.restype = ctypes.c_double
        _lib.ds41_spark_verify_gpu_v2.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64,
                                                  ctypes.c_void_p, ctypes.c_void_p]
        _lib.ds41_spark_sample_gpu_v2.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64,
                                                  ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
        _lib.ds41_pool_error.restype = ctypes.c_char_p
        _lib.ds41_pool_error.argtypes = [ctypes.c_void_p]
        _lib.ds41_placement_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                             ctypes.c_char_p, ctypes.c_size_t]
        _lib.ds41_target_experts_error.restype = ctypes.c_char_p
        _lib.ds41_target_experts_error.argtypes = [ctypes.c_void_p]
        _lib.ds41_target_experts.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        _lib.ds41_spark_verify_logits_gpu_v2.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_double,
            ctypes.c_double, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
            ctypes.c_int, ctypes.c_void_p]
    return _lib


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def take_status():
    v = ctypes.c_uint32(0)
    check(lib().ds41_take_status(ctypes.byref(v)), "ds41_take_status")
    return v.value


# ---- formats -------------------------------------------------------------------
def quantize_mxfp8(x, stream=None):
    import torch
    rows, cols = x.shape
    q = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, cols // 32), dtype=torch.uint8, device=x.device)
    check(lib().ds41_quantize_mxfp8(_p(x), _p(q), _p(s), rows, cols, _stream(stream)), "quantize_mxfp8")
    return q, s


def dequant_mxfp4(w, s, n, k, stream=None):
    import torch
    out = torch.empty((n, k), dtype=torch.float32, device=w.device)
    check(lib().ds41_dequant_mxfp4(_p(w), _p(s), _p(out), n, k, _stream(stream)), "dequant_mxfp4")
    return out


# ---- projections ----------------------------------------------------------------
def mxfp4_raw(w, ws, xq, xs, m, n, k, out=None, stream=None):
    """ds41_mxfp4_native_parallel_raw: out[m][n] bf16."""
    import torch
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=w.device)
    check(lib().ds41_mxfp4_native_parallel_raw(_p(w), _p(ws), _p(xq), _p(xs), _p(out), m, n, k,
                                               _stream(stream)), "mxfp4_raw")
    return out


def device_table(experts, device="cuda"):
    """experts: list of dicts with gate, gate_scale, up, up_scale, down, down_scale tensors
    (or None entries). Returns (device uint8 tensor holding DeviceExpert[len], host array)."""
    import torch
    arr = (DeviceExpert * len(experts))()
    for i, e in enumerate(experts):
        if e is None:
            continue
        for f in ("gate", "gate_scale", "up", "up_scale", "down", "down_scale"):
            t = e.get(f)
            setattr(arr[i], f, 0 if t is None else t.data_ptr())
        arr[i].ready = e.get("ready", 0) or 0
        arr[i].generation = e.get("generation", 0)
        arr[i].slot = e.get("slot", i)
    raw = bytes(arr)
    host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
    return host.to(device), arr


def device_jobs(jobs, device="cuda"):
    import torch
    arr = (GemmJob * len(jobs))()
    for i, (expert, tokens, x, xs, out) in enumerate(jobs):
        arr[i].expert, arr[i].tokens = expert, tokens
        arr[i].x, arr[i].x_scale, arr[i].output = x.data_ptr(), xs.data_ptr(), out.data_ptr()
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.to(device)


def grouped(table, jobs, count, projection, n, k, entry="ds41_grouped_mxfp4_native_parallel", stream=None):
    check(getattr(lib(), entry)(_p(table), _p(jobs), count, projection, n, k, _stream(stream)), entry)


def swiglu(g, u, w, limit, stream=None):
    import torch
    rows, cols = g.shape
    out = torch.empty_like(g)
    check(lib().ds41_swiglu(_p(g), _p(u), _p(w), _p(out), rows, cols, ctypes.c_float(limit), _stream(stream)),
          "swiglu")
    return out


def reduce_experts(routed, ids, shared, stream=None):
    import torch
    rows, topk, hidden = routed.shape
    out = torch.empty((rows, hidden), dtype=torch.bfloat16, device=routed.device)
    check(lib().ds41_reduce_experts(_p(routed), _p(ids), _p(shared), _p(out), rows, topk, hidden,
                                    _stream(stream)), "reduce_experts")
    return out


# ---- router ---------------------------------------------------------------------
def router_logits(x, w, stream=None):
    import torch
    M, K = x.shape
    N = w.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    check(lib().ds41_router_logits(_p(x), _p(w), _p(out), M, N, K, _stream(stream)), "router_logits")
    return out


def router_scores(logits, bias, stream=None):
    import torch
    M, N = logits.shape
    u = torch.empty_like(logits)
    b = torch.empty_like(logits)
    check(lib().ds41_dense_router_scores(_p(logits), _p(bias), _p(u), _p(b), M, N, _stream(stream)),
          "router_scores")
    return u, b


def router_topk(b, k, stream=None):
    import torch
    M, N = b.shape
    ids = torch.empty((M, k), dtype=torch.int32, device=b.device)
    check(lib().ds41_router_topk(_p(b), _p(ids), M, N, k, _stream(stream)), "router_topk")
    return ids


def router_weights(u, ids, scale=1.5, stream=None):
    import torch
    M, N = u.shape
    k = ids.shape[1]
    w = torch.empty((M, k), dtype=torch.float32, device=u.device)
    check(lib().ds41_dense_router_weights(_p(u), _p(ids), _p(w), M, N, k, ctypes.c_float(scale),
                                          _stream(stream)), "router_weights")
    return w


# ---- fused layer ------------------------------------------------------------------
def hbm_read_probe(buf, sink, blocks, stream=None):
    """Streams buf (a uint8 CUDA tensor, 16-byte multiple) once with `blocks` workgroups; sink
    holds blocks * 256 uint32 words. Time it to get the device's streaming-read ceiling."""
    f = lib().ds41_hbm_read_probe
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    check(f(buf.data_ptr(), buf.numel(), sink.data_ptr(), blocks, _stream(stream)), "ds41_hbm_read_probe")


def hbm_read_probe_ex(buf, sink, blocks, loads_in_flight, nontemporal, stream=None):
    """hbm_read_probe with loads_in_flight (4, 8, 16) 16-byte loads per thread in flight, plain or
    non-temporal loads."""
    f = lib().ds41_hbm_read_probe_ex
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_void_p]
    check(f(buf.data_ptr(), buf.numel(), sink.data_ptr(), blocks, loads_in_flight, int(nontemporal),
            _stream(stream)), "ds41_hbm_read_probe_ex")


def layer_workspace_bytes(T, H, I, E, K):
    return lib().ds41_moe_layer_workspace_bytes(T, H, I, E, K)


def make_layer_args(x, router_w, router_bias, table, expert_base, shared_index, T, H, I, E, K, y,
                    workspace, score_mode=0, route_scale=1.5, swiglu_limit=10.0, ids_out=None,
                    weights_out=None, logits_out=None):
    a = MoeLayerArgs()
    a.x_bf16, a.router_w, a.router_bias, a.table = x.data_ptr(), router_w.data_ptr(), \
        router_bias.data_ptr(), table.data_ptr()
    a.expert_base, a.shared_index = expert_base, shared_index
    a.tokens, a.hidden, a.inter, a.n_experts, a.topk = T, H, I, E, K
    a.score_mode, a.route_scale, a.swiglu_limit = score_mode, route_scale, swiglu_limit
    a.y_bf16, a.workspace, a.workspace_bytes = y.data_ptr(), workspace.data_ptr(), workspace.numel()
    a.ids_out = 0 if ids_out is None else ids_out.data_ptr()
    a.weights_out = 0 if weights_out is None else weights_out.data_ptr()
    a.logits_out = 0 if logits_out is None else logits_out.data_ptr()
    return a


def fp8_expert(e):
    """Host DeviceExpert for an FP8 shared expert given a dict of device tensors (gate, gate_scale,
    up, up_scale, down, down_scale); keep the returned object alive while the layer args use it."""
    d = DeviceExpert()
    for f in ("gate", "gate_scale", "up", "up_scale", "down", "down_scale"):
        setattr(d, f, e[f].data_ptr())
    d.slot = -1
    return d


def dense_quant(x, stream=None):
    import torch
    M, K = x.shape
    a = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    check(lib().ds41_dense_quant(_p(x), _p(a), _p(s), M, K, _stream(stream)), "ds41_dense_quant")
    return a, s


def dense_fp8(a, as_, w, ws, N, variant=-1, stream=None):
    import torch
    M, K = a.shape
    y = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    check(lib().ds41_dense_fp8(_p(a), _p(as_), _p(w), _p(ws), _p(y), M, N, K, variant, _stream(stream)),
          "ds41_dense_fp8")
    return y


def dense_shared_act(g, u, stream=None):
    import torch
    M, K = g.shape
    z = torch.empty_like(g)
    a = torch.empty((M, K), dtype=torch.uint8, device=g.device)
    s = torch.empty((M, K // 32), dtype=torch.uint8, device=g.device)
    check(lib().ds41_dense_shared_act(_p(g), _p(u), _p(z), _p(a), _p(s), M, K, _stream(stream)),
          "ds41_dense_shared_act")
    return z, a, s


def moe_layer(args, stream=None):
    check(lib().ds41_moe_verify_layer(ctypes.byref(args), _stream(stream)), "moe_verify_layer")


def moe_layer_noalloc_rc(args, stream=None):
    """ds41_moe_verify_layer_noalloc: the layer on the library's fixed device workspace (the
    args' workspace fields are ignored). Returns the HIP error code."""
    return lib().ds41_moe_verify_layer_noalloc(ctypes.byref(args), _stream(stream))


def moe_layer_noalloc_max_bytes():
    return lib().ds41_moe_layer_noalloc_max_bytes()


class Events:
    """n hipEvents owned by the library (timing on a given stream)."""

    def __init__(self, n):
        self.n = n
        self.arr = (ctypes.c_void_p * n)()
        check(lib().ds41_events_create(self.arr, n), "ds41_events_create")

    def ptr(self, i=0):
        return ctypes.cast(ctypes.byref(self.arr, i * ctypes.sizeof(ctypes.c_void_p)), ctypes.c_void_p).value

    def record(self, i, stream=None):
        check(lib().ds41_event_record(ctypes.c_void_p(self.arr[i]), _stream(stream)), "ds41_event_record")

    def elapsed(self, i, j):
        ms = ctypes.c_float(0)
        check(lib().ds41_event_elapsed_ms(ctypes.c_void_p(self.arr[i]), ctypes.c_void_p(self.arr[j]),
                                          ctypes.byref(ms)), "ds41_event_elapsed_ms")
        return ms.value

    def __del__(self):
        try:
            lib().ds41_events_destroy(self.arr, self.n)
        except Exception:
            pass


# ---- acceptance ------------------------------------------------------------------
def accept_workspace(drafts, vocab, device="cuda"):
    import torch
    return torch.zeros(lib().ds41_spark_accept_workspace_bytes(drafts, vocab), dtype=torch.uint8, device=device)


def verify_logits(target, draft, drafts_dev, temperature, top_p, seed, step, out, workspace, flags=0, stream=None):
    """target [k+1][V] fp32, draft [k][V] fp32 (None when greedy), drafts_dev int32 [k],
    out: device tensor of >= 40 bytes receiving ds41_spark_result."""
    k = target.shape[0] - 1
    V = target.shape[1]
    check(lib().ds41_spark_verify_logits_gpu_v2(
        target.data_ptr(), 0 if draft is None else draft.data_ptr(), 0 if k == 0 else drafts_dev.data_ptr(), k, V,
        float(temperature), float(top_p), seed, step, out.data_ptr(), workspace.data_ptr(), workspace.numel(),
        flags, _stream(stream).value), "ds41_spark_verify_logits_gpu_v2")


def sample_workspace(rows, vocab, device="cuda"):
    import torch
    return torch.zeros(lib().ds41_spark_sample_workspace_bytes(rows, vocab), dtype=torch.uint8, device=device)


def sample_logits_rc(logits, temperature, top_p, seed, step, first_slot, purpose, tokens, workspace, flags=0,
                     stream=None):
    """ds41_spark_sample_logits_gpu_v2 over logits [rows][V] fp32 -> tokens int32 [rows]; returns the rc."""
    rows, V = logits.shape
    return lib().ds41_spark_sample_logits_gpu_v2(
        logits.data_ptr(), rows, V, float(temperature), float(top_p), seed, step, first_slot, purpose,
        tokens.data_ptr(), workspace.data_ptr(), workspace.numel(), flags, _stream(stream).value)


def sample_logits(logits, temperature, top_p, seed, step, first_slot, purpose, tokens, workspace, flags=0,
                  stream=None):
    check(sample_logits_rc(logits, temperature, top_p, seed, step, first_slot, purpose, tokens, workspace, flags,
                           stream), "ds41_spark_sample_logits_gpu_v2")


# ---- host sampler C ABI (spark.h) -----------------------------------------------------
def spark_error():
    return lib().ds41_spark_error().decode()


def spark_probabilities(x, temperature, top_p):
    """Host fp64 probability row of fp32 logits x (numpy), or None on error."""
    import numpy as np
    x = np.ascontiguousarray(x, np.float32)
    p = np.empty(x.shape[0], np.float64)
    rc = lib().ds41_spark_probabilities(x.ctypes.data_as(ctypes.c_void_p), p.ctypes.data_as(ctypes.c_void_p),
                                        x.shape[0], ctypes.c_double(temperature), ctypes.c_double(top_p))
    return p if rc == 0 else None


def spark_sample_v2(p, seed, step, slot, purpose):
    """Host draw from the fp64 row p; None on error."""
    import numpy as np
    p = np.ascontiguousarray(p, np.float64)
    tok = ctypes.c_int32(-1)
    rc = lib().ds41_spark_sample_v2(p.ctypes.data_as(ctypes.c_void_p), p.shape[0], ctypes.c_uint64(seed),
                                    ctypes.c_uint64(step), ctypes.c_uint32(slot), ctypes.c_uint32(purpose),
                                    ctypes.byref(tok))
    return tok.value if rc == 0 else None


def spark_verify_v2(d, q, p, greedy, seed, step):
    """Host verify_v2 over fp64 rows; a result tuple, or None on error."""
    import numpy as np
    k, V = p.shape[0] - 1, p.shape[1]
    p = np.ascontiguousarray(p, np.float64)
    q = None if q is None else np.ascontiguousarray(q, np.float64)
    d = np.ascontiguousarray(np.asarray(d, np.int32)) if k else None
    res = SparkResult()
    vp = lambda a: ctypes.c_void_p(0) if a is None else a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = lib().ds41_spark_verify_v2(vp(d), vp(q), vp(p), k, V, greedy, ctypes.c_uint64(seed), ctypes.c_uint64(step),
                                    ctypes.byref(res))
    if rc:
        return None
    return (tuple(res.tokens[:res.emitted]), res.accepted_drafts, res.accepted_input_rows, res.rejected)


def spark_rng_word_v2(seed, step, slot, purpose, draw):
    return lib().ds41_spark_rng_word_v2(ctypes.c_uint64(seed), ctypes.c_uint64(step), ctypes.c_uint32(slot),
                                        ctypes.c_uint32(purpose), ctypes.c_uint64(draw))


def spark_uniform_v2(seed, step, slot, purpose, draw):
    return lib().ds41_spark_uniform_v2(ctypes.c_uint64(seed), ctypes.c_uint64(step), ctypes.c_uint32(slot),
                                       ctypes.c_uint32(purpose), ctypes.c_uint64(draw))


def result_tuple(buf):
    """Host view of a ds41_spark_result held in a device/host tensor."""
    import numpy as np
    raw = buf.cpu().numpy().view(np.int32)
    emitted = int(raw[6])
    return (tuple(int(v) for v in raw[:max(emitted, 0)]), int(raw[7]), int(raw[8]), int(raw[9])) if emitted >= 0 \
        else ((), -1, -1, -1)


def verify_gpu_v2(drafts_dev, q, p, greedy, seed, step, out, stream=None):
    """ds41_spark_verify_gpu_v2 over fp32 measures p [k+1][V], q [k][V] (None when greedy)."""
    k, V = p.shape[0] - 1, p.shape[1]
    check(lib().ds41_spark_verify_gpu_v2(_p(drafts_dev if k else None), _p(q), _p(p), k, V, greedy, seed, step,
                                         _p(out), _stream(stream)), "ds41_spark_verify_gpu_v2")


def sample_gpu_v2(p, seed, step, slot, purpose, out, stream=None):
    check(lib().ds41_spark_sample_gpu_v2(_p(p), p.shape[0], seed, step, slot, purpose, _p(out), _stream(stream)),
          "ds41_spark_sample_gpu_v2")


def result_raw(buf):
    """All fields of a ds41_spark_result held in a device tensor, including an invalid step's."""
    import numpy as np
    raw = buf.cpu().numpy().view(np.int32)
    return (tuple(int(v) for v in raw[:6]), int(raw[6]), int(raw[7]), int(raw[8]), int(raw[9]))


def accept_fallbacks(workspace, drafts, vocab):
    v = ctypes.c_uint32(0)
    check(lib().ds41_spark_accept_fallbacks(ctypes.c_void_p(workspace.data_ptr()), drafts, vocab, ctypes.byref(v)),
          "ds41_spark_accept_fallbacks")
    return v.value


def layer_plan(workspace, T, H, I, E, K):
    ids = (ctypes.c_int32 * (T * K + 1))()
    n = lib().ds41_moe_layer_plan(ctypes.c_void_p(workspace.data_ptr()), T, H, I, E, K, ids, T * K + 1)
    if n < 0:
        raise RuntimeError("ds41_moe_layer_plan failed")
    return list(ids[:n])


# ---- verify step through a layer stack with a host expert tier ----------------------
def slab_tile(src, dst, hidden, inter, count, stream=None):
    """ds41_expert_slab_tile: count canonical slabs (device uint8 tensors) with tiled weights."""
    check(lib().ds41_expert_slab_tile(_p(src), _p(dst), hidden, inter, count, _stream(stream)), "ds41_expert_slab_tile")


def slab_tile_host(src, dst, hidden, inter, count):
    """ds41_expert_slab_tile_host on host uint8 tensors or numpy arrays."""
    def ptr(a):
        return ctypes.c_void_p(a.data_ptr() if hasattr(a, "data_ptr") else a.ctypes.data)
    check(lib().ds41_expert_slab_tile_host(ptr(src), ptr(dst), hidden, inter, count), "ds41_expert_slab_tile_host")


def slab_layout(hidden, inter):
    """Canonical expert slab: ([gate, gate_scale, up, up_scale, down, down_scale] byte offsets, slab bytes)."""
    out = ExpertLayout()
    check(lib().ds41_expert_slab_layout(hidden, inter, ctypes.byref(out)), "ds41_expert_slab_layout")
    return list(out.offset), int(out.bytes)


SLAB_FIELDS = ("gate", "gate_scale", "up", "up_scale", "down", "down_scale")


def slab_entry(base_ptr, offsets, slot=-1):
    """DeviceExpert pointing into a canonical slab at base_ptr."""
    e = DeviceExpert()
    for f, o in zip(SLAB_FIELDS, offsets):
        setattr(e, f, base_ptr + o)
    e.ready, e.generation, e.slot = 0, 0, slot
    return e


class HostSlabs:
    """Pinned host memory from ds41_host_alloc (hipHostMalloc) viewed as a uint8 CPU tensor of
    [count][slab] bytes; freed with the object."""

    def __init__(self, count, slab):
        import numpy as np
        import torch
        self.ptr = ctypes.c_void_p(0)
        check(lib().ds41_host_alloc(ctypes.c_size_t(count * slab), ctypes.byref(self.ptr)), "ds41_host_alloc")
        buf = (ctypes.c_uint8 * (count * slab)).from_address(self.ptr.value)
        self.tensor = torch.from_numpy(np.ctypeslib.as_array(buf).reshape(count, slab))

    def __del__(self):
        try:
            if self.ptr.value:
                self.tensor = None
                lib().ds41_host_free(self.ptr)
                self.ptr = ctypes.c_void_p(0)
        except Exception:
            pass


class CacheStats(_Versioned):
    _fields_ = _ABI_FIELDS + [("requests", ctypes.c_uint64), ("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64),
                ("evictions", ctypes.c_uint64), ("h2d_bytes", ctypes.c_uint64), ("slots", ctypes.c_uint64),
                ("prefetch_requests", ctypes.c_uint64), ("prefetch_copies", ctypes.c_uint64)]


class VerifyStack:
    """ds41_verify_stack_*: layers is a list of dicts with router_w, router_bias, table (device tensors),
    expert_base, shared_index and optionally host_index (device int32 [E]) + host_slabs (pinned uint8
    tensor of host_slab_count slabs). The tensors must outlive the stack."""

    def __init__(self, layers, max_tokens, hidden, inter, n_experts, topk, score_mode=0, route_scale=1.5,
                 swiglu_limit=10.0, slab_bytes=None, weight_layout=0):
        arr = (StackLayer * len(layers))()
        for i, d in enumerate(layers):
            arr[i].router_w, arr[i].router_bias = d["router_w"].data_ptr(), d["router_bias"].data_ptr()
            arr[i].table = d["table"].data_ptr()
            arr[i].expert_base, arr[i].shared_index = d.get("expert_base", 0), d.get("shared_index", -1)
            hi, hs = d.get("host_index"), d.get("host_slabs")
            arr[i].host_index = 0 if hi is None else hi.data_ptr()
            arr[i].host_slabs = 0 if hs is None else hs.data_ptr()
            arr[i].host_slab_count = 0 if hs is None else hs.numel() // slab_bytes
        self._arr = arr
        desc = StackDesc(len(layers), max_tokens, hidden, inter, n_experts, topk, score_mode, route_scale,
                         swiglu_limit, arr, weight_layout)
        self.handle = ctypes.c_void_p(0)
        check(lib().ds41_verify_stack_create(ctypes.byref(desc), ctypes.byref(self.handle)),
              "ds41_verify_stack_create")
        self.L, self.H, self.K = len(layers), hidden, topk

    def step(self, x, y, route_ids=None, layer_out=None, ids_out=None, weights_out=None, stream=None):
        T = x.shape[0]
        check(lib().ds41_verify_stack_step(self.handle, _p(x), _p(y), T, _p(route_ids), _p(layer_out), _p(ids_out),
                                           _p(weights_out), _stream(stream)), "ds41_verify_stack_step")

    def layer(self, l, x, y, route_ids=None, ids_out=None, weights_out=None, stream=None):
        check(lib().ds41_verify_stack_layer(self.handle, l, _p(x), _p(y), x.shape[0], _p(route_ids), _p(ids_out),
                                            _p(weights_out), _stream(stream)), "ds41_verify_stack_layer")

    def cache(self, slots, placement=None):
        """ds41_verify_stack_cache: an HBM cache of `slots` expert slabs for the host-tier experts
        (slots <= 0: as many as the free HBM holds, less 2 GiB)."""
        check(lib().ds41_verify_stack_cache(self.handle, slots, None if placement is None else ctypes.byref(placement)),
              "ds41_verify_stack_cache")

    def prefetch_rc(self, layers, experts):
        """ds41_verify_stack_prefetch over (layer, expert) pairs; returns the HIP error code."""
        import numpy as np
        la = np.ascontiguousarray(np.asarray(layers, np.int32).ravel())
        ea = np.ascontiguousarray(np.asarray(experts, np.int32).ravel())
        return lib().ds41_verify_stack_prefetch(self.handle, la.ctypes.data_as(ctypes.c_void_p),
                                                ea.ctypes.data_as(ctypes.c_void_p), len(la))

    def prefetch(self, layers, experts):
        check(self.prefetch_rc(layers, experts), "ds41_verify_stack_prefetch")

    def prefetch_routes(self, route_ids):
        """Prefetches every (layer, expert) pair of a host int32 [L][T][K] route array."""
        import numpy as np
        r = np.asarray(route_ids, np.int32)
        L = r.shape[0]
        layers = np.repeat(np.arange(L, dtype=np.int32), r[0].size)
        self.prefetch(layers, r.reshape(-1))

    def cache_stats(self):
        st = CacheStats()
        check(lib().ds41_verify_stack_cache_stats(self.handle, ctypes.byref(st)), "ds41_verify_stack_cache_stats")
        return {f: int(getattr(st, f)) for f in CacheStats.data_fields()}

    def stats(self):
        st = StackStats()
        check(lib().ds41_verify_stack_stats(self.handle, ctypes.byref(st)), "ds41_verify_stack_stats")
        return {f: int(getattr(st, f)) for f in StackStats.data_fields()}

    def close(self):
        if self.handle:
            lib().ds41_verify_stack_destroy(self.handle)
            self.handle = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- expert slot pool (LFU residency) and placement files -------------------------------
POOL_MAX_LAYERS = 64
REFERENCE_LAYERS = [384] * 40 + [128] * 3  # components/moe/include/ds41/store.hpp:16


class Placement(ctypes.Structure):
    _fields_ = [("recent_window", ctypes.c_uint32), ("decay_interval", ctypes.c_uint32),
                ("distinct_lfu", ctypes.c_int32), ("hard_budgets", ctypes.c_int32),
                ("layers", ctypes.c_int32), ("n_vram", ctypes.c_int32), ("n_host", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("budget", ctypes.c_uint32 * POOL_MAX_LAYERS),
                ("host_budget", ctypes.c_uint32 * POOL_MAX_LAYERS), ("vram_pins", ctypes.c_void_p),
                ("host_residents", ctypes.c_void_p)]


class PoolAllocation(ctypes.Structure):
    _fields_ = [("id", ctypes.c_uint32), ("slot", ctypes.c_int32), ("hit", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("evicted", ctypes.c_int64)]


def _u32(ids):
    arr = (ctypes.c_uint32 * max(len(ids), 1))(*[int(i) & 0xFFFFFFFF for i in ids])
    return arr


def make_placement(layers, budget=None, hard=False, recent=6, decay=32, distinct=True, pins=()):
    p = Placement()
    p.recent_window, p.decay_interval, p.distinct_lfu, p.hard_budgets = recent, decay, int(distinct), int(hard)
    p.layers = layers
    for l, b in enumerate(budget or []):
        p.budget[l] = b
    p._pins = _u32(list(pins))
    p.n_vram = len(pins)
    p.vram_pins = ctypes.cast(p._pins, ctypes.c_void_p).value if pins else None
    return p


def load_placement(path, layer_experts=REFERENCE_LAYERS, cap=1 << 16):
    """ds41_placement_load -> (Placement, vram pins list, host residents list). Raises with the reason."""
    sizes = _u32(layer_experts)
    out = Placement()
    vram, host = (ctypes.c_uint32 * cap)(), (ctypes.c_uint32 * cap)()
    err = ctypes.create_string_buffer(256)
    rc = lib().ds41_placement_load(path.encode(), len(layer_experts), sizes, ctypes.byref(out), vram, cap, host, cap,
                                   err, 256)
    if rc != 0:
        raise ValueError(f"ds41_placement_load ({rc}): {err.value.decode()}")
    out._keep = (vram, host)
    return out, list(vram[:out.n_vram]), list(host[:out.n_host])


class ExpertPool:
    """ds41_pool_*: the library's expert slot pool. Methods return what the C calls return;
    acquire/borrow give (rc, [(id, slot, hit, evicted), ...])."""

    def __init__(self, slots, layer_experts=REFERENCE_LAYERS, recent=6, decay=32, distinct=True):
        self.h = ctypes.c_void_p(0)
        sizes = _u32(layer_experts)
        rc = lib().ds41_pool_create(slots, len(layer_experts), sizes, recent, decay, int(distinct),
                                    ctypes.byref(self.h))
        if rc != 0:
            raise ValueError(f"ds41_pool_create failed ({rc})")

    def _allocs(self, fn, ids, *extra):
        out = (PoolAllocation * max(len(ids), 1))()
        rc = fn(self.h, _u32(ids), len(ids), *extra, out)
        return rc, [(a.id, a.slot, bool(a.hit), a.evicted) for a in out[:max(rc, 0)]]

    def acquire(self, ids, prefetch=False):
        return self._allocs(lib().ds41_pool_acquire, ids, int(prefetch))

    def borrow(self, ids):
        return self._allocs(lib().ds41_pool_borrow, ids)

    def release(self, lease):
        arr = (PoolAllocation * max(len(lease), 1))()
        for i, (e, s, h, ev) in enumerate(lease):
            arr[i].id, arr[i].slot, arr[i].hit, arr[i].evicted = e, s, int(h), ev
        return lib().ds41_pool_release(self.h, arr, len(lease))

    def touch(self, ids):
        return lib().ds41_pool_touch(self.h, _u32(ids), len(ids))

    def policy(self, placement):
        return lib().ds41_pool_policy(self.h, ctypes.byref(placement))

    def pin(self, e):
        return lib().ds41_pool_pin(self.h, ctypes.c_uint32(e))

    def unpin(self, e):
        return lib().ds41_pool_unpin(self.h, ctypes.c_uint32(e))

    def residency(self, e):
        return lib().ds41_pool_residency(self.h, ctypes.c_uint32(e))

    def reset_history(self):
        return lib().ds41_pool_reset_history(self.h)

    def retain(self, e):
        """ds41_pool_retain -> (rc, token handle or None); drop it with token_release()."""
        t = ctypes.c_void_p(0)
        rc = lib().ds41_pool_retain(self.h, ctypes.c_uint32(e), ctypes.byref(t))
        return rc, (t.value if rc == 0 else None)

    @staticmethod
    def token_release(token):
        return lib().ds41_pool_token_release(ctypes.c_void_p(token))

    def reserve(self, target, wanted=()):
        out = (PoolAllocation * max(int(target), 1))()
        rc = lib().ds41_pool_reserve(self.h, int(target), _u32(list(wanted)), len(wanted), out)
        return rc, [(a.id, a.slot, bool(a.hit), a.evicted) for a in out[:max(rc, 0)]]

    def drained(self, slot):
        return lib().ds41_pool_drained(self.h, int(slot))

    def peer(self, other, host):
        return lib().ds41_pool_peer(self.h, other.h if other is not None else None, int(host))

    def exclusive(self, on):
        return lib().ds41_pool_exclusive(self.h, int(on))

    def decay_interval(self, d):
        return lib().ds41_pool_decay_interval(self.h, int(d))

    def fast_minima(self, on):
        return lib().ds41_pool_fast_minima(self.h, int(on))

    def switch_target_layer(self, placement, layer):
        return lib().ds41_pool_switch_target_layer(self.h, ctypes.byref(placement), int(layer))

    def late(self, layer):
        return lib().ds41_pool_late(self.h, int(layer))

    def error(self):
        return lib().ds41_pool_error(self.h).decode()

    def __del__(self):
        try:
            if self.h:
                lib().ds41_pool_destroy(self.h)
        except Exception:
            pass


class DriftControl:
    """ds41_drift_*: the width-one drift controller over a VRAM pool and its RAM pool (keeps both
    pools and the placement alive)."""

    def __init__(self, placement, vram, ram):
        self.h = ctypes.c_void_p(0)
        self._keep = (placement, vram, ram)
        err = ctypes.create_string_buffer(256)
        self.rc = lib().ds41_drift_create(ctypes.byref(placement), vram.h, ram.h, ctypes.byref(self.h), err, 256)
        self.msg = err.value.decode()

    def before(self, ids):
        return lib().ds41_drift_before(self.h, _u32(ids), len(ids))

    def after(self, ids):
        return lib().ds41_drift_after(self.h, _u32(ids), len(ids))

    def active(self):
        return lib().ds41_drift_active(self.h)

    def completed_tokens(self):
        return lib().ds41_drift_completed_tokens(self.h)

    def __del__(self):
        try:
            if self.h:
                lib().ds41_drift_destroy(self.h)
        except Exception:
            pass


# ---- on-disk expert format ----------------------------------------------------------------
class RecordInfo(ctypes.Structure):
    _fields_ = [("id", ctypes.c_uint32), ("n_extents", ctypes.c_int32), ("bytes", ctypes.c_uint64),
                ("view_offset", ctypes.c_uint64 * 6), ("view_bytes", ctypes.c_uint64 * 6)]


class RecordExtent(ctypes.Structure):
    _fields_ = [("path", ctypes.c_char * 4096), ("file_offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("dst_offset", ctypes.c_uint64), ("required_bytes", ctypes.c_uint64),
                ("expected_file_bytes", ctypes.c_uint64)]


class Records:
    """ds41_records_*: a records manifest (R/E lines) over safetensors shards. Methods raise
    ValueError with the library's reason."""

    def __init__(self, manifest):
        self.h = ctypes.c_void_p(0)
        err = ctypes.create_string_buffer(512)
        if lib().ds41_records_load(manifest.encode(), ctypes.byref(self.h), err, 512) != 0:
            raise ValueError(err.value.decode())

    def count(self):
        return lib().ds41_records_count(self.h)

    def find(self, expert_id):
        return lib().ds41_records_find(self.h, ctypes.c_uint32(expert_id))

    def info(self, i):
        o = RecordInfo()
        if lib().ds41_records_info(self.h, i, ctypes.byref(o)) != 0:
            raise ValueError("record index")
        return dict(id=o.id, bytes=o.bytes, n_extents=o.n_extents,
                    views=[(o.view_offset[k], o.view_bytes[k]) for k in range(6)])

    def extents(self, i):
        out = []
        for k in range(self.info(i)["n_extents"]):
            e = RecordExtent()
            if lib().ds41_records_extent(self.h, i, k, ctypes.byref(e)) != 0:
                raise ValueError("extent index")
            out.append((e.path.decode(), e.file_offset, e.bytes, e.dst_offset, e.required_bytes,
                        e.expected_file_bytes))
        return out

    def validate(self, root, complete=True):
        err = ctypes.create_string_buffer(512)
        if lib().ds41_records_validate(self.h, root.encode(), int(complete), err, 512) != 0:
            raise ValueError(err.value.decode())

    def read(self, i):
        import numpy as np
        buf = np.zeros(self.info(i)["bytes"], np.uint8)
        err = ctypes.create_string_buffer(512)
        if lib().ds41_record_read(self.h, i, ctypes.c_void_p(buf.ctypes.data), buf.size, err, 512) != 0:
            raise ValueError(err.value.decode())
        return buf

    def load_slab(self, i, hidden, inter, out=None):
        """Reads record i and repacks it into a canonical slab (numpy uint8, or `out`: any object
        with a data_ptr() / numpy array of at least the slab size)."""
        import numpy as np
        _, slab = slab_layout(hidden, inter)
        if out is None:
            out = np.zeros(slab, np.uint8)
        ptr = out.data_ptr() if hasattr(out, "data_ptr") else out.ctypes.data
        err = ctypes.create_string_buffer(512)
        if lib().ds41_record_load_slab(self.h, i, hidden, inter, ctypes.c_void_p(ptr), slab, err, 512) != 0:
            raise ValueError(err.value.decode())
        return out

    def __del__(self):
        try:
            if self.h:
                lib().ds41_records_free(self.h)
        except Exception:
            pass


# ---- MTP drafter: routed-expert service and router top-3 -------------------------------
class TargetExpertsDesc(_Versioned):
    _fields_ = _ABI_FIELDS + [("table", ctypes.c_void_p), ("expert_base", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("inter", ctypes.c_int32), ("swiglu_limit", ctypes.c_float), ("check_routes", ctypes.c_int32),
                ("stream", ctypes.c_void_p), ("stage_events", ctypes.c_void_p), ("weight_layout", ctypes.c_int32)]


class TargetExperts:
    """ds41_target_experts_*: the ds41_target_experts_fn service over a device table whose
    drafter experts of stage s, id e are table[expert_base + 128 * s + e]. Calls must use
    the stream given here. call() raises with the library's error text on failure."""

    def __init__(self, table, expert_base, hidden, inter, swiglu_limit=10.0, check_routes=False, stream=None,
                 events=None, weight_layout=0):
        self.stream = _stream(stream)
        self.desc = TargetExpertsDesc(table.data_ptr(), expert_base, hidden, inter, swiglu_limit,
                                      1 if check_routes else 0, self.stream, 0 if events is None else events,
                                      weight_layout)
        self.handle = ctypes.c_void_p(0)
        check(lib().ds41_target_experts_create(ctypes.byref(self.desc), ctypes.byref(self.handle)),
              "ds41_target_experts_create")
        self.H = hidden

    def call_rc(self, stage, x, ids, weights, out, rows=None, stream=None):
        rows = x.shape[0] if rows is None else rows
        return lib().ds41_target_experts(self.handle, stage, _p(x), _p(ids), _p(weights), _p(out), rows,
                                         self.stream if stream is None else _stream(stream))

    def error(self):
        return lib().ds41_target_experts_error(self.handle).decode()

    def __call__(self, stage, x, ids, weights, out=None):
        import torch
        if out is None:
            out = torch.empty((x.shape[0], 3, self.H), dtype=torch.bfloat16, device=x.device)
        if self.call_rc(stage, x, ids, weights, out) != 0:
            raise RuntimeError(f"ds41_target_experts: {self.error()}")
        return out

    def close(self):
        if self.handle:
            lib().ds41_target_experts_destroy(self.handle)
            self.handle = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def spark_topk3(scores, stream=None):
    import torch
    ids = torch.empty((scores.shape[0], 3), dtype=torch.int32, device=scores.device)
    check(lib().ds41_spark_topk3_gpu(_p(scores), _p(ids), scores.shape[0], _stream(stream)), "ds41_spark_topk3_gpu")
    return ids


# ---- chunked verify / prefill ---------------------------------------------------------
def prefill_raw(w, ws, xq, xs, m, n, k, out=None, stream=None):
    import torch
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=w.device)
    check(lib().ds41_mxfp4_prefill_raw(_p(w), _p(ws), _p(xq), _p(xs), _p(out), m, n, k, _stream(stream)),
          "ds41_mxfp4_prefill_raw")
    return out


def grouped_prefill(table, jobs, count, projection, n, k, max_tokens, stream=None):
    check(lib().ds41_grouped_mxfp4_prefill(_p(table), _p(jobs), count, projection, n, k, max_tokens,
                                           _stream(stream)), "ds41_grouped_mxfp4_prefill")


def prefill_workspace_bytes(T, H, I, E, K):
    return lib().ds41_moe_prefill_workspace_bytes(T, H, I, E, K)


def make_prefill_args(x, ids, weights, table, expert_base, shared_index, T, H, I, E, K, y, workspace,
                      swiglu_limit=10.0):
    a = MoePrefillArgs()
    a.x_bf16, a.ids, a.weights, a.table = x.data_ptr(), ids.data_ptr(), weights.data_ptr(), table.data_ptr()
    a.expert_base, a.shared_index = expert_base, shared_index
    a.tokens, a.hidden, a.inter, a.n_experts, a.topk = T, H, I, E, K
    a.swiglu_limit = swiglu_limit
    a.y_bf16, a.workspace, a.workspace_bytes = y.data_ptr(), workspace.data_ptr(), workspace.numel()
    return a


def moe_prefill(args, stream=None):
    check(lib().ds41_moe_prefill_layer(ctypes.byref(args), _stream(stream)), "ds41_moe_prefill_layer")


def prefill_plan_counts(workspace, T, H, I, E, K):
    """(tiles, GEMV jobs of experts with <= 4 rows, GEMV jobs of experts with 5..8 rows)."""
    v = (ctypes.c_int32 * 3)()
    check(lib().ds41_moe_prefill_plan_counts(ctypes.c_void_p(workspace.data_ptr()), T, H, I, E, K, v),
          "ds41_moe_prefill_plan_counts")
    return tuple(v)


def prefill_tiles(workspace, T, H, I, E, K):
    v = ctypes.c_int32(0)
    check(lib().ds41_moe_prefill_tiles(ctypes.c_void_p(workspace.data_ptr()), T, H, I, E, K, ctypes.byref(v)),
          "ds41_moe_prefill_tiles")
    return v.value
