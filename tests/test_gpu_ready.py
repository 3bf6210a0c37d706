"""The DeviceExpert residency flags (components/moe/include/ds41/store.hpp:110-117 `ready` /
`generation`; the kernels' acquire wait, components/moe/src/mxfp4.cu:36-43), through the C ABI.

Bars:
- flags that already hold each expert's generation give output bits identical to ready == NULL,
  for the verify layer (gate/up, fused down + reduce) and the grouped projection API;
- flags written by the host after the layer is queued: the kernels wait for them, the status word
  stays 0 and the output bits are again identical;
- a flag that the host never sets (the bounded wait's failure path, forced from the host): status
  bit 1 is raised, every output that needed the expert is NaN and the others are unchanged. The
  wait gives up after 2 s of the device's wall clock, so every kernel still exits."""
import ctypes
import time

import numpy as np
import pytest

from test_gpu_moe import dev, host, make_layer, rand_mx, rand_x, say

pytestmark = pytest.mark.gpu


def _flagged(experts, flags, gen):
    """Copies of the expert dicts whose table entries carry ready = &flags[i], generation gen[i]
    (flags: a tensor or the address of a uint32 array)."""
    base = flags if isinstance(flags, int) else flags.data_ptr()
    out = []
    for i, e in enumerate(experts):
        d = dict(e)
        d["ready"] = base + 4 * i
        d["generation"] = int(gen[i])
        out.append(d)
    return out


def _loaded_hip():
    """The HIP runtime this process already runs (torch's copy): a second copy of the runtime
    loaded beside it would own streams the first one cannot use."""
    with open("/proc/self/maps") as f:
        paths = {ln.split()[-1] for ln in f if "libamdhip64.so" in ln}
    assert len(paths) == 1, paths
    return ctypes.CDLL(paths.pop())


def _layer_inputs(gpu, T, H, E, seed):
    rng = np.random.default_rng(seed)
    x = dev(rand_x(rng, T, H), gpu)
    wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
    bias = dev(np.zeros(E, np.float32), gpu)
    return x, wg, bias


def _run_layer(gpu, table, x, wg, bias, T, H, I, E, K, stream=None):
    import torch
    import ds41_gfx950 as G
    y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    ids = torch.full((T, K), -1, dtype=torch.int32, device=gpu)
    a = G.make_layer_args(x, wg, bias, table, 0, E, T, H, I, E, K, y, ws, ids_out=ids)
    if stream is not None:  # the fills above run on the current stream
        stream.wait_stream(torch.cuda.current_stream())
    G.moe_layer(a, stream=stream)
    return y, ids, ws


def test_ready_flags_already_set_match_no_flags(gpu):
    import torch
    import ds41_gfx950 as G
    T, H, I, E, K = 4, 4096, 2880, 64, 6
    say(f"ready flags already set: layer T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 51, H, I, E, T)
    gen = np.arange(E + 1, dtype=np.uint32) * 7 + 3
    flags = torch.from_numpy(gen.astype(np.int32)).to(gpu)
    plain, _ = G.device_table(experts, gpu)
    flagged, _ = G.device_table(_flagged(experts, flags, gen), gpu)
    x, wg, bias = _layer_inputs(gpu, T, H, E, 52)
    y0, i0, _ = _run_layer(gpu, plain, x, wg, bias, T, H, I, E, K)
    y1, i1, _ = _run_layer(gpu, flagged, x, wg, bias, T, H, I, E, K)
    torch.cuda.synchronize()
    assert G.take_status() == 0
    assert np.array_equal(host(i0), host(i1))
    assert np.array_equal(host(y0), host(y1))
    assert not np.any((host(y1) & 0x7fff) > 0x7f80)
    # the grouped projection API reads the same flags
    rng = np.random.default_rng(53)
    n, k, m = 512, 1024, 3
    w, ws = rand_mx(rng, n, k)
    e = {"gate": dev(w, gpu), "gate_scale": dev(ws, gpu)}
    xq, xs = G.quantize_mxfp8(dev(rand_x(rng, m, k), gpu))
    outs = []
    for ready in (False, True):
        ee = dict(e)
        if ready:
            ee.update(ready=flags.data_ptr() + 8, generation=int(gen[2]))
        table, _ = G.device_table([ee], gpu)
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        jobs = G.device_jobs([(0, m, xq, xs, out)], gpu)
        G.grouped(table, jobs, 1, G.PROJ_GATE, n, k)
        outs.append(out)
    torch.cuda.synchronize()
    assert G.take_status() == 0
    assert np.array_equal(host(outs[0]), host(outs[1]))


def test_ready_flags_written_after_the_layer_is_queued(gpu):
    """The layer is queued first and its kernels wait; the host then writes the flags. The flags sit
    in coherent pinned host memory, which the kernels' polls read through to, so no copy has to get
    past the waiting kernels: HIP maps a process's streams onto a few hardware queues, and a copy on
    a stream that shares the waiting kernel's queue would run only after it."""
    import torch
    import ds41_gfx950 as G
    T, H, I, E, K = 4, 2048, 1024, 48, 6
    say(f"ready flags written after queueing: layer T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 54, H, I, E, T)
    gen = (np.arange(E + 1, dtype=np.uint32) + 1) * 5
    hip = _loaded_hip()
    hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    hip.hipHostFree.argtypes = [ctypes.c_void_p]
    raw = ctypes.c_void_p()
    assert hip.hipHostMalloc(ctypes.byref(raw), 4 * (E + 1), 0x40000000) == 0  # hipHostMallocCoherent
    try:
        flags = np.ctypeslib.as_array((ctypes.c_uint32 * (E + 1)).from_address(raw.value))
        flags[:] = 0
        plain, _ = G.device_table(experts, gpu)
        flagged, _ = G.device_table(_flagged(experts, raw.value, gen), gpu)
        x, wg, bias = _layer_inputs(gpu, T, H, E, 55)
        y0, _, _ = _run_layer(gpu, plain, x, wg, bias, T, H, I, E, K)
        torch.cuda.synchronize()
        t0 = time.time()
        y1, _, ws = _run_layer(gpu, flagged, x, wg, bias, T, H, I, E, K)
        time.sleep(0.05)  # the kernels are waiting by now
        flags[:] = gen
        torch.cuda.synchronize()
        dt = time.time() - t0
        say(f"  layer with flags set after queueing finished in {dt * 1e3:.1f} ms")
        assert G.take_status() == 0
        assert np.array_equal(host(y0), host(y1))
    finally:
        torch.cuda.synchronize()
        hip.hipHostFree(raw.value)


@pytest.mark.parametrize("H", [512, 1024])
def test_ready_flag_never_set_gives_nan_and_status(gpu, H):
    """A flag the host never sets on the shared expert (forced failure of the bounded wait): the
    wait gives up, status bit 1, and every token's output is NaN (the shared expert feeds every
    token). With H = 1024 the plan launch computes the shared expert's gate/up and marks the values
    it could not compute. Then the grouped API: only the job whose expert never became ready is NaN."""
    import torch
    import ds41_gfx950 as G
    T, I, E, K = 2, 256, 16, 2
    say(f"ready flag never set (bounded wait gives up after 2 s): layer T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 56, H, I, E, T)
    flags = torch.zeros(E + 1, dtype=torch.int32, device=gpu)
    ex = [dict(e) for e in experts]
    ex[E]["ready"], ex[E]["generation"] = flags.data_ptr() + 4 * E, 1  # never written
    table, _ = G.device_table(ex, gpu)
    x, wg, bias = _layer_inputs(gpu, T, H, E, 57)
    t0 = time.time()
    y, _, _ = _run_layer(gpu, table, x, wg, bias, T, H, I, E, K)
    torch.cuda.synchronize()
    say(f"  layer returned after {time.time() - t0:.2f} s")
    assert G.take_status() & 1
    assert np.all((host(y) & 0x7fff) > 0x7f80), "every output must be NaN"
    rng = np.random.default_rng(58)
    n, k, m = 128, 512, 2
    w, s = rand_mx(rng, n, k)
    good = {"gate": dev(w, gpu), "gate_scale": dev(s, gpu)}
    bad = dict(good, ready=flags.data_ptr(), generation=9)
    table, _ = G.device_table([good, bad], gpu)
    xq, xs = G.quantize_mxfp8(dev(rand_x(rng, m, k), gpu))
    o_good = torch.zeros((m, n), dtype=torch.bfloat16, device=gpu)
    o_bad = torch.zeros((m, n), dtype=torch.bfloat16, device=gpu)
    jobs = G.device_jobs([(0, m, xq, xs, o_good), (1, m, xq, xs, o_bad)], gpu)
    G.grouped(table, jobs, 2, G.PROJ_GATE, n, k)
    torch.cuda.synchronize()
    assert G.take_status() & 1
    assert np.all((host(o_bad) & 0x7fff) > 0x7f80)
    assert not np.any((host(o_good) & 0x7fff) > 0x7f80)
