"""Benchmark of the ds41 speculative-verify path on one MI355X.

Headline (the metric's own workload, configs[4] of the benchmark definition): the T=4 verify step
(1 committed + 3 MTP drafts) through 40 stacked MoE layers, hidden 4096, 384 routed experts
(intermediate 2880, MXFP4 e2m1 + e8m0/32) top-6 + 1 shared expert per layer, independent seeded
weights per layer. Per layer the Zipf(1.1)-hottest 320 experts and the shared expert sit in HBM
(241.7 GB) and the other 64 in pinned host RAM (48.1 GB), fetched by hipMemcpyAsync on a side stream
when routed. Routing: Zipf(1.1) ids drawn fresh for every step. The host-tier experts of each step's
routes are prefetched into an LFU HBM cache sized to the HBM left after the resident set (the
reference's VRAM slot pool in front of its RAM tier); the headline's W warmup + K timed steps run with
the cache as a preceding leg of the same run left it, and that leg, which starts from an empty cache,
is reported beside it, as are the legs without a cache and with router routing. A step is one
40-layer pass over one batch of T rows.

Prints ONE JSON line (the driver's contract) with a roofline object for the dominant kernel (the
fused gate/up/activation GEMV, timed live with HIP events on its launch stream over configs[1]
layers, the same kernel at the same shape), and a cpu_baseline object: the C oracle on the host
cores running the same layers (rank 0, N=1, a bounded sample). Sub-objects carry configs[0..3].
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "deepseek-v4.1-flash-pro6000_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, _p)

EXPERT_BYTES = 18_800_640          # gate + up + down weights and E8M0 scales (H=4096, I=2880)
GATE_UP_BYTES = 2 * (2880 * 2048 + 2880 * 128)
DOWN_BYTES = 4096 * 1440 + 4096 * 90
PEAK_HBM_GBPS = 8000.0
PEAK_FP4_TFLOPS = 10100.0
# HBM bytes per gate/up/act launch (tiled weights) from rocprofv3 FETCH_SIZE (x2.0) + WRITE_SIZE (x1.0),
# calibrated on a plain 1 GiB device copy, at mean U = 23.328 routed experts + shared
# (profiles/verify_layer_config1_traffic.md); the algorithmic figure at that U is 304,923,000 B.
GATE_UP_TRAFFIC_BYTES = 305_567_000
METRIC = "verify tokens/s per MTP step (T=1+k); MoE HBM GB/s as % of 8 TB/s peak"
# Expert weight layout of the configs[1] and configs[4] legs: 1 = tiled (ds41_expert_slab_tile, the MFMA
# operand order), 0 = the checkpoint's row-major layout. The synthetic weights are uniform random bytes,
# which read as uniform e2m1 codes in either layout.
LAYOUT = {"weights": 1}
DRAFT = 1


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_info():
    """The host the CPU baselines ran on: CPU model and the cores this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count()}


def bf16_bits_np(f):
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    import numpy as np
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def slab_expert(slab_np, off, H, I):
    """Views of one canonical slab (numpy uint8) as the six expert tensors."""
    shapes = [(I, H // 2), (I, H // 32), (I, H // 2), (I, H // 32), (H, I // 2), (H, I // 32)]
    names = ("gate", "gate_scale", "up", "up_scale", "down", "down_scale")
    return {n: slab_np[o:o + a * b].reshape(a, b) for n, o, (a, b) in zip(names, off, shapes)}


def cpu_layer_baseline(x_np, ids, w, experts_np, shared_np, H, I, seconds, layers=1, what=""):
    """The C oracle (a port of the reference arithmetic) on all host cores: one routed MoE layer
    (MXFP8 of x, every routed expert's FFN, the shared expert, the ordered reduce) per sample; the
    value is T tokens over `layers` such layers."""
    import oracle as O
    threads = len(os.sched_getaffinity(0))
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        O.moe_layer_routed(x_np, ids, w, experts_np, shared_np, H, I, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    T = x_np.shape[0]
    per = sum(times) / len(times)
    U = len(set(ids.ravel().tolist()))
    return dict({"value": T / (per * layers), "unit": "tokens/s", "cores": threads, "kind": "port",
                 "sample": f"{len(times)} passes of one layer (T={T}, {U} routed experts + shared{what}) of the "
                           f"C oracle, {per * 1e3:.1f} ms each" + (f", x {layers} layers" if layers > 1 else "")},
                **host_info())


def bench_layer(gpu, steps, warmup, cpu_seconds, no_cpu, fp8_legs=True):
    """one MoE layer decode verify, T=4 rows bf16 N(0,1) over a pool of 64 seeded activations
    (routing changes from step to step), router fp32 N(0, 0.02^2), 384 routed + 1 shared MXFP4 experts all
    HBM-resident. Carries the roofline object of the fused gate/up/activation kernel. Returns (result,
    state for the legs that reuse the layer's experts)."""
    import numpy as np
    import torch
    import ds41_gfx950 as G
    T, H, I, E, K = 4, 4096, 2880, 384, 6
    log(f"bench: configs[1] one MoE layer T={T} H={H} I={I} E={E}+1 shared, steps={steps} warmup={warmup}")
    g = torch.Generator(device=gpu).manual_seed(0)

    def rnd(shape, lo, hi):
        return torch.randint(lo, hi, shape, dtype=torch.uint8, device=gpu, generator=g)

    # e2m1 nibbles uniform over 16 codes (bytes uniform), e8m0 scales uniform over 2^-8..2^-4
    P = dict(gate=rnd((E + 1, I, H // 2), 0, 256), gate_scale=rnd((E + 1, I, H // 32), 119, 124),
             up=rnd((E + 1, I, H // 2), 0, 256), up_scale=rnd((E + 1, I, H // 32), 119, 124),
             down=rnd((E + 1, H, I // 2), 0, 256), down_scale=rnd((E + 1, H, I // 32), 119, 124))
    experts = [{k: v[e] for k, v in P.items()} for e in range(E + 1)]
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(0)
    pool = 64
    x_pool_np = [bf16_bits_np(rng.standard_normal((T, H)).astype(np.float32)) for _ in range(pool)]
    x_pool = torch.stack([torch.from_numpy(a.view(np.int16)) for a in x_pool_np]).to(gpu).view(torch.bfloat16)
    wg_np = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias_np = np.zeros(E, np.float32)
    wg, bias = torch.from_numpy(wg_np).to(gpu), torch.from_numpy(bias_np).to(gpu)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    ids_dev = torch.empty((pool, T, K), dtype=torch.int32, device=gpu)
    w_dev = torch.empty((pool, T, K), dtype=torch.float32, device=gpu)
    layer_args = [G.make_layer_args(x_pool[i], wg, bias, table, 0, E, T, H, I, E, K, y, ws) for i in range(pool)]
    for a in layer_args:
        a.weight_layout = LAYOUT["weights"]
    stream = torch.cuda.current_stream()

    # unique routed experts per pool entry (bytes actually streamed per step), and the routing
    uniq = []
    for i in range(pool):
        a = G.make_layer_args(x_pool[i], wg, bias, table, 0, E, T, H, I, E, K, y, ws, ids_out=ids_dev[i],
                              weights_out=w_dev[i])
        a.weight_layout = LAYOUT["weights"]
        G.moe_layer(a, stream)
        uniq.append(len(G.layer_plan(ws, T, H, I, E, K)))
    torch.cuda.synchronize()
    assert G.take_status() == 0

    for i in range(warmup):
        G.moe_layer(layer_args[i % pool], stream)
    torch.cuda.synchronize()

    ev = G.Events(2)
    torch.cuda.synchronize()
    ev.record(0, stream)
    for i in range(steps):
        G.moe_layer(layer_args[i % pool], stream)
    ev.record(1, stream)
    torch.cuda.synchronize()
    total_ms = ev.elapsed(0, 1)
    ms_per_step = total_ms / steps

    # per-kernel execution times from start/stop timestamps (a separate pass over the same steps)
    NS = 10
    stage = G.Events(NS * steps)
    for i in range(steps):
        a = layer_args[i % pool]
        a.stage_events = stage.ptr(NS * i)
        G.moe_layer(a, stream)
        a.stage_events = None
    torch.cuda.synchronize()
    # configs[1] runs the fused down + reduce kernel as stage 3; stage 4's events mark an empty interval
    names = ["router", "plan", "gate_up_act", "down_reduce"]
    stage_ms = {n: 0.0 for n in names}
    for i in range(steps):
        for j, n in enumerate(names):
            stage_ms[n] += stage.elapsed(NS * i + 2 * j, NS * i + 2 * j + 1)
    assert G.take_status() == 0
    avg = {n: stage_ms[n] / steps for n in names}

    # gate/up and down launched alone, back to back, over one prepared workspace per pool entry (each
    # launch streams its own step's experts); events around the whole batch give the average launch
    # duration of the kernel, the quantity the roofline divides by
    wss = [torch.zeros_like(ws) for _ in range(pool)]
    prep = [G.make_layer_args(x_pool[i], wg, bias, table, 0, E, T, H, I, E, K, y, wss[i]) for i in range(pool)]
    for a in prep:
        a.weight_layout = LAYOUT["weights"]
        G.moe_layer(a, stream)
    reps = max(steps // pool, 1)
    launch_us = {}
    # "down" is the fused down + reduce kernel; the separate pair (stage bit 5) is timed beside it
    for mask, n in ((4, "gate_up_act"), (8, "down"), (8 | 32, "down_separate"), (16 | 32, "reduce_separate")):
        for a in prep:
            a.stage_mask = mask
        G.moe_layer(prep[-1], stream)
        torch.cuda.synchronize()
        ev.record(0, stream)
        for _ in range(reps):
            for a in prep:
                G.moe_layer(a, stream)
        ev.record(1, stream)
        torch.cuda.synchronize()
        launch_us[n] = ev.elapsed(0, 1) * 1e3 / (reps * pool)
        for a in prep:
            a.stage_mask = 0
    assert G.take_status() == 0
    del wss, prep
    mean_u = float(np.mean(uniq))
    gate_gbps = (mean_u + 1) * GATE_UP_BYTES / (launch_us["gate_up_act"] * 1e-6) / 1e9
    down_gbps = (mean_u + 1) * DOWN_BYTES / (launch_us["down"] * 1e-6) / 1e9
    layer_bytes = sum((uniq[i % pool] + 1) * EXPERT_BYTES + E * H * 4 for i in range(steps))
    layer_gbps = layer_bytes / (total_ms * 1e-3) / 1e9
    log("stage avg us (start/stop timestamps, include dispatch): " +
        ", ".join(f"{n} {avg[n] * 1e3:.1f}" for n in names))
    log(f"launch avg us (back to back): gate_up_act {launch_us['gate_up_act']:.1f}, down+reduce (fused) "
        f"{launch_us['down']:.1f}; separate kernels: down {launch_us['down_separate']:.1f}, "
        f"reduce {launch_us['reduce_separate']:.1f}")
    log(f"configs[1]: {ms_per_step * 1e3:.1f} us/layer ({T / (ms_per_step * 1e-3):.0f} tok/s); gate_up_act "
        f"{gate_gbps:.0f} GB/s, down {down_gbps:.0f} GB/s, layer {layer_gbps:.0f} GB/s "
        f"({layer_gbps / PEAK_HBM_GBPS * 100:.1f}% of 8 TB/s), mean unique experts {mean_u:.2f}")

    ceiling, ceiling_sweep = read_ceiling(gpu, stream)
    best = max(ceiling_sweep, key=lambda r: r["gbps"])
    log(f"streaming-read ceiling (ds41_hbm_read_probe_ex, 1 GiB, best of {len(ceiling_sweep)}: "
        f"{best['blocks']} WGs, {best['loads_in_flight']} loads in flight, "
        f"{'non-temporal' if best['nontemporal'] else 'plain'}): {ceiling:.0f} GB/s; "
        f"gate_up_act at {gate_gbps / ceiling * 100:.1f}% of it")
    for r in ceiling_sweep:
        log(f"  read probe {r['blocks']:5d} WGs x {r['loads_in_flight']:2d} loads "
            f"{'nt   ' if r['nontemporal'] else 'plain'}: {r['gbps']:.0f} GB/s")

    fp8_shared = bench_fp8_shared(gpu, x_pool, wg, bias, table, steps, warmup) if fp8_legs else None

    cpu = None
    if not no_cpu:
        ids0, w0 = ids_dev[0].cpu().numpy(), w_dev[0].cpu().numpy()
        experts_np = [None] * E
        for e in sorted(set(ids0.ravel().tolist())):
            experts_np[e] = {k: v.cpu().numpy() for k, v in experts[e].items()}
        shared_np = {k: v.cpu().numpy() for k, v in experts[E].items()}
        cpu = cpu_layer_baseline(x_pool_np[0], ids0, w0, experts_np, shared_np, H, I, cpu_seconds,
                                 what=", router routing of pool entry 0")
        log(f"configs[1] cpu baseline: {cpu}")
    res = {
        "workload": "configs[1]: one MoE layer decode verify, T=4 (1+3 MTP drafts), hidden 4096, 384 routed "
                    "experts (I=2880, MXFP4) top-6 + 1 shared, all HBM-resident",
        "weight_layout": "tiled" if LAYOUT["weights"] else "row-major",
        "steps": steps, "warmup": warmup, "value": T / (ms_per_step * 1e-3), "unit": "tokens/s",
        "us_per_layer": ms_per_step * 1e3, "mean_unique_experts": mean_u,
        "hbm_gbps": layer_gbps, "hbm_frac": layer_gbps / PEAK_HBM_GBPS,
        "stage_us": {n: avg[n] * 1e3 for n in names},
        "launch_us": launch_us,
        "roofline": {"bound": "hbm", "kernel": "layer_gate_up_act_kernel", "achieved": gate_gbps,
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": gate_gbps / PEAK_HBM_GBPS,
                     "traffic": GATE_UP_TRAFFIC_BYTES,
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE/WRITE_SIZE, calibrated)",
                     "bytes_per_launch": (mean_u + 1) * GATE_UP_BYTES, "launch_us": launch_us["gate_up_act"],
                     "measured_read_ceiling": ceiling, "frac_of_measured_ceiling": gate_gbps / ceiling,
                     "read_ceiling_probe": {"best": best, "sweep": ceiling_sweep}},
        "cpu_baseline": cpu,
        "fp8_shared": fp8_shared,
    }
    return res, dict(table=table, P=P, E=E)


def bench_expert(gpu, reps, cpu_seconds, no_cpu, seed=0):
    """one MXFP4 expert SwiGLU FFN, 1 token, hidden 1024, intermediate 512. Inputs from numpy
    default_rng(0) in the order W_gate, S_gate, W_up, S_up, W_down, S_down, x: weight bytes uniform (two
    e2m1 nibbles uniform over the 16 codes), e8m0 scales uniform over 119..123 (2^-8..2^-4), x bf16 N(0,1).
    GPU: the reference kernel API's chain (quantize_mxfp8 -> grouped gate -> grouped up -> swiglu ->
    quantize_mxfp8 -> grouped down), six launches, timed eagerly and replayed from a HIP graph. CPU: the C
    oracle's expert FFN on the same inputs at 1 thread and at every host core."""
    import numpy as np
    import torch
    import ds41_gfx950 as G
    H, I = 1024, 512
    rng = np.random.default_rng(seed)
    W = {}
    W["gate"] = rng.integers(0, 256, (I, H // 2), dtype=np.uint8)
    W["gate_scale"] = rng.integers(119, 124, (I, H // 32), dtype=np.uint8)
    W["up"] = rng.integers(0, 256, (I, H // 2), dtype=np.uint8)
    W["up_scale"] = rng.integers(119, 124, (I, H // 32), dtype=np.uint8)
    W["down"] = rng.integers(0, 256, (H, I // 2), dtype=np.uint8)
    W["down_scale"] = rng.integers(119, 124, (H, I // 32), dtype=np.uint8)
    x_np = bf16_bits_np(rng.standard_normal((1, H)).astype(np.float32))
    dev = {k: torch.from_numpy(v).to(gpu) for k, v in W.items()}
    table, _ = G.device_table([dev], gpu)
    x = torch.from_numpy(x_np.view(np.int16)).to(gpu).view(torch.bfloat16)
    xq = torch.empty((1, H), dtype=torch.uint8, device=gpu)
    xs = torch.empty((1, H // 32), dtype=torch.uint8, device=gpu)
    gate = torch.empty((1, I), dtype=torch.bfloat16, device=gpu)
    up = torch.empty((1, I), dtype=torch.bfloat16, device=gpu)
    h = torch.empty((1, I), dtype=torch.bfloat16, device=gpu)
    hq = torch.empty((1, I), dtype=torch.uint8, device=gpu)
    hs = torch.empty((1, I // 32), dtype=torch.uint8, device=gpu)
    out = torch.empty((1, H), dtype=torch.bfloat16, device=gpu)
    jobs = {"gate": G.device_jobs([(0, 1, xq, xs, gate)], gpu), "up": G.device_jobs([(0, 1, xq, xs, up)], gpu),
            "down": G.device_jobs([(0, 1, hq, hs, out)], gpu)}
    L = G.lib()

    def chain(stream):
        s = G._stream(stream)
        G.check(L.ds41_quantize_mxfp8(G._p(x), G._p(xq), G._p(xs), 1, H, s), "quantize")
        G.check(L.ds41_grouped_mxfp4(G._p(table), G._p(jobs["gate"]), 1, G.PROJ_GATE, I, H, s), "gate")
        G.check(L.ds41_grouped_mxfp4(G._p(table), G._p(jobs["up"]), 1, G.PROJ_UP, I, H, s), "up")
        G.check(L.ds41_swiglu(G._p(gate), G._p(up), G._p(None), G._p(h), 1, I, ctypes.c_float(10.0), s), "swiglu")
        G.check(L.ds41_quantize_mxfp8(G._p(h), G._p(hq), G._p(hs), 1, I, s), "quantize h")
        G.check(L.ds41_grouped_mxfp4(G._p(table), G._p(jobs["down"]), 1, G.PROJ_DOWN, H, I, s), "down")

    stream = torch.cuda.current_stream()
    for _ in range(20):
        chain(stream)
    ev = G.Events(2)
    torch.cuda.synchronize()
    ev.record(0, stream)
    for _ in range(reps):
        chain(stream)
    ev.record(1, stream)
    torch.cuda.synchronize()
    us = ev.elapsed(0, 1) * 1e3 / reps
    eager_out = out.clone()
    gs = torch.cuda.Stream()
    gs.wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gs):
        chain(gs)
    torch.cuda.synchronize()
    for _ in range(5):
        graph.replay()
    torch.cuda.synchronize()
    ev.record(0, stream)
    for _ in range(reps):
        graph.replay()
    ev.record(1, stream)
    torch.cuda.synchronize()
    us_graph = ev.elapsed(0, 1) * 1e3 / reps
    if not torch.equal(out.view(torch.int16), eager_out.view(torch.int16)) or G.take_status():
        raise AssertionError("configs[0]: graph replay differs from the eager chain")
    nbytes = 3 * (I * H // 2 + I * H // 32)
    res = {"workload": "configs[0]: one MXFP4 expert SwiGLU FFN, 1 token, H=1024, I=512 (seed 0)",
           "us_per_call": us, "us_per_call_graph": us_graph, "launches": 6, "bytes": nbytes,
           "gbps": nbytes / (us * 1e-6) / 1e9, "flops": 2 * 3 * H * I,
           "bound": "latency (835,584 B of weights fit in the caches; roofline not meaningful)"}
    log(f"configs[0]: expert FFN {us:.1f} us/call eager, {us_graph:.1f} us graph-replayed")
    if not no_cpu:
        import oracle as O
        xq_np, xs_np = O.quantize_mxfp8(x_np)
        cpu = {}
        for threads in (1, len(os.sched_getaffinity(0))):
            O.set_threads(threads)
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < cpu_seconds / 2 or n < 3:
                q, s = O.quantize_mxfp8(x_np)
                O.expert_ffn(W, q, s, None, H, I)
                n += 1
            cpu[threads] = (time.perf_counter() - t0) / n
        O.set_threads(1)
        nt = max(cpu)
        res["cpu_baseline"] = dict({
            "value": cpu[1] * 1e6, "unit": "us/call", "cores": 1, "kind": "port",
            "value_all_cores": cpu[nt] * 1e6, "cores_all": nt,
            "sample": f"the C oracle's MXFP8 quantisation + expert FFN on the same inputs, about "
                      f"{cpu_seconds / 2:.0f} s at 1 thread and at {nt} threads"}, **host_info())
        log(f"configs[0] cpu baseline: {res['cpu_baseline']}")
    del table, dev
    return res


def bench_accept(gpu, steps, cpu_seconds, no_cpu, top_p=1.0):
    """the accept step alone, k=3 drafts + 1 bonus over V=129280, T=1.0, top-p 1.0 (and 0.95),
    Philox v2 seed 0, step = iteration. Logits from a pool of 16 resident sets (target N(0, 2.5^2),
    draft = target + N(0, 0.5^2)). A step is SpeculativeStep's sampling work: the three draft tokens drawn
    from q_k with (step, k, Draft) on the device (ds41_spark_sample_logits_gpu_v2), then the verify from
    logits (ds41_spark_verify_logits_gpu_v2) on those device tokens. The CPU baseline is the reference
    engine's own code for the same step (engine/src/sampling.cpp: probabilities + sample per draft,
    probabilities_rows over its 8-thread pool, reject_sample), compiled from its sources."""
    import numpy as np
    import torch
    import ds41_gfx950 as G
    import oracle as O
    k, V, pool, seed, T = 3, 129280, 16, 0, 1.0
    rng = np.random.default_rng(2)
    tgt, drf = [], []
    for i in range(pool):
        t = (rng.standard_normal((k + 1, V)) * 2.5).astype(np.float32)
        tgt.append(t)
        drf.append((t[:k] + rng.standard_normal((k, V)) * 0.5).astype(np.float32))
    T_dev = torch.from_numpy(np.stack(tgt)).to(gpu)
    D_dev = torch.from_numpy(np.stack(drf)).to(gpu)
    ws = G.accept_workspace(k, V, gpu)
    sws = G.sample_workspace(k, V, gpu)
    out = torch.zeros((steps, 16), dtype=torch.int32, device=gpu)
    toks = torch.zeros((steps, 8), dtype=torch.int32, device=gpu)
    stream = torch.cuda.current_stream()

    def step(s, o, tk, st=None):
        G.sample_logits(D_dev[s % pool], T, top_p, seed, s, 0, DRAFT, tk, sws, stream=st)
        G.verify_logits(T_dev[s % pool], D_dev[s % pool], tk, T, top_p, seed, s, o, ws, stream=st)

    for s in range(50):
        step(s, out[s], toks[s])
    ev = G.Events(2)
    torch.cuda.synchronize()
    ev.record(0, stream)
    for s in range(steps):
        step(s, out[s], toks[s])
    ev.record(1, stream)
    torch.cuda.synchronize()
    us = ev.elapsed(0, 1) * 1e3 / steps
    res_np = out.cpu().numpy()
    accepted = float(np.mean(res_np[:, 7]))
    # the sampling kernels alone, to split the step
    ev.record(0, stream)
    for s in range(min(steps, 2000)):
        G.sample_logits(D_dev[s % pool], T, top_p, seed, s, 0, DRAFT, toks[s], sws)
    ev.record(1, stream)
    torch.cuda.synchronize()
    us_sample = ev.elapsed(0, 1) * 1e3 / min(steps, 2000)
    # `pool` consecutive steps captured in one HIP graph (kernels only), replayed back to back; every
    # replay's results are checked against the eager ones
    gs = torch.cuda.Stream()
    out_g = torch.zeros((pool, 16), dtype=torch.int32, device=gpu)
    tok_g = torch.zeros((pool, 8), dtype=torch.int32, device=gpu)
    graph = torch.cuda.CUDAGraph()
    gs.wait_stream(stream)
    with torch.cuda.stream(gs):
        step(0, out_g[0], tok_g[0], gs)
    gs.synchronize()
    with torch.cuda.graph(graph, stream=gs):
        for s in range(pool):
            step(s, out_g[s], tok_g[s], gs)
    reps = max(steps // pool, 1)
    torch.cuda.synchronize()
    ev.record(0, stream)
    for _ in range(reps):
        graph.replay()
    ev.record(1, stream)
    torch.cuda.synchronize()
    us_graph = ev.elapsed(0, 1) * 1e3 / (reps * pool)
    for s in range(pool):
        if G.result_tuple(out_g[s]) != G.result_tuple(out[s]):
            raise AssertionError(f"accept graph replay differs from the eager step {s}")
    # parity spot checks against the oracle: every 500th step's drafts and decisions
    for s in range(0, steps, 500):
        d_ref = [O.sample_v2(O.probabilities(drf[s % pool][j], T, top_p), seed, s, j, DRAFT) for j in range(k)]
        if toks[s, :k].cpu().tolist() != d_ref:
            raise AssertionError(f"draft sampling parity failed at step {s}")
        ref = O.accept_logits(tgt[s % pool], drf[s % pool], np.array(d_ref, np.int32), T, top_p, seed, s)
        if G.result_tuple(out[s]) != ref.as_tuple():
            raise AssertionError(f"accept parity failed at step {s}")
    cpu = None
    if not no_cpu:
        n, t0 = 0, time.perf_counter()
        if O.refengine() is not None:  # the reference engine's own accept code
            while time.perf_counter() - t0 < cpu_seconds or n < 2:
                r = O.ref_accept_step(tgt[n % pool], drf[n % pool], k, T, top_p, seed, n)
                if r is None:
                    raise AssertionError("reference accept step failed")
                n += 1
            per = (time.perf_counter() - t0) / n
            cpu = {"value": per * 1e6, "unit": "us/step", "cores": 8, "kind": "reference",
                   "sample": f"{n} accept steps of the reference engine's sampler (engine/src/sampling.cpp: "
                             f"probabilities + sample for 3 drafts, probabilities_rows on its 8-thread pool for "
                             f"4 target rows, reject_sample; V={V}, top-p {top_p})"}
        else:
            while time.perf_counter() - t0 < cpu_seconds or n < 2:
                O.accept_logits(tgt[n % pool], drf[n % pool], np.array([0, 1, 2], np.int32), T, top_p, seed, n)
                n += 1
            per = (time.perf_counter() - t0) / n
            cpu = {"value": per * 1e6, "unit": "us/step", "cores": 1, "kind": "port",
                   "sample": f"{n} accept steps of the C oracle (7 fp64 probability rows + verify_v2)"}
        cpu.update(host_info())
    return {"workload": f"configs[2]: accept k=3 + bonus, V=129280, T=1.0, top-p {top_p}; drafts sampled on "
                        f"the device from q (step, k, Draft), then verify", "steps": steps,
            "us_per_step": us, "us_per_step_graph": us_graph, "us_draft_sampling": us_sample,
            "mean_accepted_drafts": accepted, "sequential_path_steps": G.accept_fallbacks(ws, k, V),
            "bytes_per_step": 7 * V * 4, "cpu_baseline": cpu}


def read_ceiling(gpu, stream, nbytes=1 << 30, reps=10):
    """The device's streaming-read ceiling: ds41_hbm_read_probe_ex streaming nbytes (4x the 256 MB
    last-level cache) once per launch, timed with events around reps launches, over a sweep of
    loads in flight per thread (4, 8, 16), plain and non-temporal loads, and 1k-8k workgroups.
    Returns (best GB/s, the sweep as a list of dicts)."""
    import torch
    import ds41_gfx950 as G
    buf = torch.ones(nbytes, dtype=torch.uint8, device=gpu)
    sweep = []
    for blocks in (1024, 2048, 4096, 8192):
        sink = torch.empty(blocks * 256, dtype=torch.int32, device=gpu)
        for u in (4, 8, 16):
            for nt in (0, 1):
                for _ in range(2):
                    G.hbm_read_probe_ex(buf, sink, blocks, u, nt, stream)
                ev = G.Events(2)
                torch.cuda.synchronize()
                ev.record(0, stream)
                for _ in range(reps):
                    G.hbm_read_probe_ex(buf, sink, blocks, u, nt, stream)
                ev.record(1, stream)
                torch.cuda.synchronize()
                gbps = nbytes * reps / (ev.elapsed(0, 1) * 1e-3) / 1e9
                sweep.append({"blocks": blocks, "loads_in_flight": u, "nontemporal": nt, "gbps": gbps})
        del sink
    del buf
    best = max(sweep, key=lambda r: r["gbps"])
    return best["gbps"], sweep


def bench_prefill(gpu, table, E, steps, warmup, seed=3, P=None, cpu_seconds=8.0, no_cpu=True):
    """one MoE layer chunked verify/prefill, T=512 rows bf16 N(0,1), each token routed to K=6
    distinct experts drawn from Zipf(1.1) over ranks (rank r -> expert perm[r-1], seeded permutation), route
    weights random positive normalised to 1.5 per token (labelled: the configs[3] text leaves them open),
    same 384+1 experts as configs[1]. A step is one prefill layer: MXFP8 quantisation, device route plan,
    gate/up + SwiGLU + MXFP8, down, ordered reduce."""
    import numpy as np
    import torch
    import ds41_gfx950 as G
    T, H, I, K = 512, 4096, 2880, 6
    rng = np.random.default_rng(seed)
    p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
    p /= p.sum()
    perm = rng.permutation(E)
    ids_np = np.stack([perm[rng.choice(E, size=K, replace=False, p=p)] for _ in range(T)]).astype(np.int32)
    w_np = (rng.random((T, K)) + 0.1).astype(np.float32)
    w_np = (w_np / w_np.sum(axis=1, keepdims=True) * 1.5).astype(np.float32)
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=gpu, dtype=torch.float32).to(torch.bfloat16)
    ids, w = torch.from_numpy(ids_np).to(gpu), torch.from_numpy(w_np).to(gpu)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.prefill_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    args = G.make_prefill_args(x, ids, w, table, 0, E, T, H, I, E, K, y, ws)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        G.moe_prefill(args, stream)
    torch.cuda.synchronize()
    tiles = G.prefill_tiles(ws, T, H, I, E, K)
    ev = G.Events(2)
    ev.record(0, stream)
    for _ in range(steps):
        G.moe_prefill(args, stream)
    ev.record(1, stream)
    torch.cuda.synchronize()
    us = ev.elapsed(0, 1) * 1e3 / steps
    kernels = ["quant", "plan", "gate_up_gemv4", "gate_up_gemv8", "gate_up_tiles", "down_gemv4", "down_gemv8",
               "down_tiles", "reduce"]
    NS = 2 * len(kernels)  # start/stop timestamps of each kernel
    st = G.Events(NS * steps)
    ktot = {n: 0.0 for n in kernels}
    for i in range(steps):
        args.stage_events = st.ptr(NS * i)
        G.moe_prefill(args, stream)
    args.stage_events = None
    torch.cuda.synchronize()
    for i in range(steps):
        for j, n in enumerate(kernels):
            ktot[n] += st.elapsed(NS * i + 2 * j, NS * i + 2 * j + 1) * 1e3 / steps
    names = ["quant", "plan", "gate_up_act", "down", "reduce"]
    tot = {"quant": ktot["quant"], "plan": ktot["plan"],
           "gate_up_act": ktot["gate_up_gemv4"] + ktot["gate_up_gemv8"] + ktot["gate_up_tiles"],
           "down": ktot["down_gemv4"] + ktot["down_gemv8"] + ktot["down_tiles"], "reduce": ktot["reduce"]}
    plan = G.prefill_plan_counts(ws, T, H, I, E, K)
    if G.take_status():
        raise AssertionError("prefill bench: kernel status bits set")
    U = int(np.unique(ids_np).size)
    rows = T * K + T
    weight_bytes = (U + 1) * EXPERT_BYTES
    act_bytes = T * H * 2 * 2 + rows * (I + I // 32) * 2 + rows * H * 2 * 2  # x in, y out, activation/down rows
    flops = 2.0 * rows * 3 * I * H
    gu_bytes = (U + 1) * GATE_UP_BYTES
    counts = np.bincount(ids_np.ravel(), minlength=E)
    out = {"workload": "configs[3]: one MoE layer chunked verify/prefill, T=512, hidden 4096, 384 experts "
                       "(I=2880, MXFP4) top-6 Zipf(1.1) + 1 shared; route weights random, normalised to 1.5",
           "steps": steps, "us_per_layer": us, "tokens_per_s": T / (us * 1e-6),
           "unique_experts": U, "max_rows_per_expert": int(counts.max()), "tiles": tiles,
           "hbm_bytes": weight_bytes + act_bytes, "hbm_gbps": (weight_bytes + act_bytes) / (us * 1e-6) / 1e9,
           "hbm_frac": (weight_bytes + act_bytes) / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS,
           "gflop": flops / 1e9, "tflops": flops / (us * 1e-6) / 1e12,
           "mfma_frac_fp4_peak": flops / (us * 1e-6) / 1e12 / PEAK_FP4_TFLOPS,
           "stage_us": tot, "kernel_us": ktot,
           "plan": {"tiles": plan[0], "gemv_jobs_le4_rows": plan[1], "gemv_jobs_5to8_rows": plan[2]},
           "gate_up_gbps": gu_bytes / (tot["gate_up_act"] * 1e-6) / 1e9,
           "down_gbps": (U + 1) * DOWN_BYTES / (tot["down"] * 1e-6) / 1e9}
    log(f"prefill: {us:.1f} us/layer ({T / (us * 1e-6):.0f} tok/s), U={U}, plan (tiles, gemv<=4, gemv5-8) {plan}, "
        f"HBM {out['hbm_gbps']:.0f} GB/s, {out['tflops']:.0f} TFLOP/s; kernels " +
        ", ".join(f"{n} {ktot[n]:.1f}" for n in kernels))
    out["cpu_baseline"] = None
    if not no_cpu and P is not None:
        out["cpu_baseline"] = prefill_cpu_baseline(x, ids_np, w_np, P, E, H, I, cpu_seconds)
        log(f"configs[3] cpu baseline: {out['cpu_baseline']}")
    return out


def bench_drafter(gpu, steps, warmup, seed=6):
    """The MTP drafter's routed-expert service (ds41_target_experts_fn, routed_spark): B=5 drafter rows,
    hidden 5120, 3 stages x 128 experts (I=2304, MXFP4, all HBM-resident, 7.2 GB), top-3 per row from the
    drafter's router top-3 (ds41_spark_topk3_gpu) over random scores; route weights random positive. A call
    is one stage: MXFP8 quantisation, plan from the caller's ids, gate/up + SwiGLU + MXFP8, down into slots."""
    import numpy as np
    import torch
    import ds41_gfx950 as G
    H, I, E, R = 5120, 2304, 3 * 128, 5
    g = torch.Generator(device=gpu).manual_seed(seed)
    # canonical slabs (e2m1 bytes uniform, e8m0 scales uniform over 2^-8..2^-4), tiled like the stack's
    off, slab = G.slab_layout(H, I)
    slabs = torch.randint(0, 256, (E, slab), dtype=torch.uint8, device=gpu, generator=g)
    for o, m in ((off[1], I * H // 32), (off[3], I * H // 32), (off[5], H * I // 32)):
        slabs[:, o:o + m].random_(119, 124, generator=g)
    if LAYOUT["weights"]:
        tiled = torch.empty_like(slabs)
        G.slab_tile(slabs, tiled, H, I, E)
        del slabs
        slabs = tiled
    entries = [G.slab_entry(slabs[e].data_ptr(), off, e) for e in range(E)]
    table = torch.frombuffer(bytearray(b"".join(bytes(x) for x in entries)), dtype=torch.uint8).to(gpu)
    pool = 64
    scores = torch.rand((pool, R, 128), generator=g, device=gpu)
    ids = torch.stack([G.spark_topk3(scores[i]) for i in range(pool)])
    w = torch.rand((pool, R, 3), generator=g, device=gpu) + 0.1
    x = torch.randn((pool, R, H), generator=g, device=gpu).to(torch.bfloat16)
    out = torch.empty((R, 3, H), dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.current_stream()
    svc = G.TargetExperts(table, 0, H, I, stream=stream, weight_layout=LAYOUT["weights"])
    for i in range(warmup):
        svc(i % 3, x[i % pool], ids[i % pool], w[i % pool], out)
    torch.cuda.synchronize()
    ev = G.Events(2)
    ev.record(0, stream)
    for i in range(steps):
        svc(i % 3, x[i % pool], ids[i % pool], w[i % pool], out)
    ev.record(1, stream)
    torch.cuda.synchronize()
    us = ev.elapsed(0, 1) * 1e3 / steps
    ev.record(0, stream)
    for i in range(steps):
        G.spark_topk3(scores[i % pool], stream)
    ev.record(1, stream)
    torch.cuda.synchronize()
    top3_us = ev.elapsed(0, 1) * 1e3 / steps
    names = ["quant_plan", "", "gate_up_act", "down"]  # one launch quantises and plans; pair 1 spans nothing
    NS = 2 * len(names)
    st = G.Events(NS)
    svc_t = G.TargetExperts(table, 0, H, I, stream=stream, events=st.ptr(0), weight_layout=LAYOUT["weights"])
    ktot = {n: 0.0 for n in names}
    for i in range(steps):  # the handle's one event set is read back after every call
        svc_t(i % 3, x[i % pool], ids[i % pool], w[i % pool], out)
        torch.cuda.synchronize()
        for j, n in enumerate(names):
            ktot[n] += st.elapsed(2 * j, 2 * j + 1) * 1e3 / steps
    ktot.pop("")
    svc_t.close()
    svc.close()
    if G.take_status():
        raise AssertionError("drafter bench: kernel status bits set")
    ids_np = ids.cpu().numpy()
    U = float(np.mean([np.unique(ids_np[i % pool]).size for i in range(steps)]))
    ebytes = 3 * (I * H // 2) + 3 * (I * H // 32)
    gu_bytes = 2 * (I * H // 2 + I * H // 32)
    res = {"workload": "MTP drafter routed experts: 5 rows, hidden 5120, 3 stages x 128 experts (I=2304, MXFP4) "
                       "top-3 (drafter router top-3 over random scores), route weights random",
           "weight_layout": "tiled" if LAYOUT["weights"] else "row-major",
           "steps": steps, "us_per_call": us, "mean_unique_experts": U,
           "hbm_gbps": U * ebytes / (us * 1e-6) / 1e9, "hbm_frac": U * ebytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS,
           "kernel_us": ktot, "gate_up_gbps": U * gu_bytes / (ktot["gate_up_act"] * 1e-6) / 1e9,
           "top3_us_per_call": top3_us}
    log(f"drafter experts: {us:.1f} us/call, U={U:.2f}, HBM {res['hbm_gbps']:.0f} GB/s; kernels " +
        ", ".join(f"{n} {v:.1f}" for n, v in ktot.items()) + f"; top-3 {top3_us:.1f} us")
    del slabs, table
    torch.cuda.empty_cache()
    return res


def zipf_route_ids(rng, perms, pool, T, K, s=1.1):
    """[pool][L][T][K] int32: per token K distinct Zipf(s) ranks over 1..E (sequential draws without
    replacement), rank r -> expert perms[l][r-1]."""
    import numpy as np
    L, E = len(perms), len(perms[0])
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    out = np.empty((pool, L, T, K), np.int32)
    for i in range(pool):
        for l in range(L):
            for t in range(T):
                out[i, l, t] = perms[l][rng.choice(E, size=K, replace=False, p=p)]
    return out


def bench_fp8_shared(gpu, x_pool, wg, bias, table, steps, warmup, T=4, H=4096, I=2880, E=384, K=6, seed=5):
    """configs[1] with the shared expert as the checkpoint stores it: FP8 E4M3 gate/up/down with one
    E8M0 scale per 32 x 32 block (W8A8, MXFP8 activations), routed experts unchanged. Also the
    standalone ds41_dense_fp8 at the shared expert's gate shape (M=4, N=2880, K=4096)."""
    import ctypes
    import torch
    import ds41_gfx950 as G
    g = torch.Generator(device=gpu).manual_seed(seed)

    def fp8(n, k):  # N(0, 1) quantised per 32 x 32 block (amax -> 448), scaled to ~0.01
        v = torch.randn((n, k), generator=g, device=gpu, dtype=torch.float32)
        e = torch.ceil(torch.log2(v.abs().reshape(n // 32, 32, k // 32, 32).amax(dim=(1, 3)) / 448.0))
        sc = torch.exp2(e).repeat_interleave(32, 0).repeat_interleave(32, 1)
        w = (v / sc).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        return torch.where((w & 0x7F) == 0x7F, torch.full_like(w, 0x7E), w), (e + 121).to(torch.uint8)

    gw_, gs_ = fp8(I, H)
    uw_, us_ = fp8(I, H)
    dw_, ds_ = fp8(H, I)
    f8 = G.fp8_expert(dict(gate=gw_, gate_scale=gs_, up=uw_, up_scale=us_, down=dw_, down_scale=ds_))
    pool = x_pool.shape[0]
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
    args = [G.make_layer_args(x_pool[i], wg, bias, table, 0, -1, T, H, I, E, K, y, ws) for i in range(pool)]
    for a in args:
        a.shared_fp8 = ctypes.addressof(f8)
        a.weight_layout = LAYOUT["weights"]  # the routed experts are configs[1]'s table, in its layout
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        G.moe_layer(args[i % pool], stream)
    torch.cuda.synchronize()
    ev = G.Events(2)
    ev.record(0, stream)
    for i in range(steps):
        G.moe_layer(args[i % pool], stream)
    ev.record(1, stream)
    torch.cuda.synchronize()
    layer_us = ev.elapsed(0, 1) * 1e3 / steps
    xq, xs = G.dense_quant(x_pool[0])
    yd = torch.empty((T, I), dtype=torch.bfloat16, device=gpu)
    reps = max(steps, 50)
    for _ in range(5):
        G.lib().ds41_dense_fp8(G._p(xq), G._p(xs), G._p(gw_), G._p(gs_), G._p(yd), T, I, H, -1, G._stream(stream))
    ev.record(0, stream)
    for _ in range(reps):
        G.lib().ds41_dense_fp8(G._p(xq), G._p(xs), G._p(gw_), G._p(gs_), G._p(yd), T, I, H, -1, G._stream(stream))
    ev.record(1, stream)
    torch.cuda.synchronize()
    fp8_us = ev.elapsed(0, 1) * 1e3 / reps
    if G.take_status():
        raise AssertionError("fp8 shared bench: kernel status bits set")
    wbytes = I * H + (I // 32) * (H // 32)
    res = {"workload": "configs[1] layer with an FP8 W8A8 shared expert (32x32 block scales), routed MXFP4 unchanged",
           "us_per_layer": layer_us, "tokens_per_s": T / (layer_us * 1e-6),
           "shared_fp8_bytes": 3 * wbytes, "dense_fp8_us": fp8_us,
           "dense_fp8_gbps": wbytes / (fp8_us * 1e-6) / 1e9, "dense_fp8_shape": [T, I, H]}
    log(f"fp8 shared: layer {layer_us:.1f} us/step; ds41_dense_fp8 M={T} N={I} K={H}: {fp8_us:.1f} us, "
        f"{res['dense_fp8_gbps']:.0f} GB/s")
    return res


def zipf_route_ids_fast(rng, perms, n, T, K, s=1.1):
    """As zipf_route_ids for n fresh step sets, vectorised: the top-K of log p + Gumbel noise is a
    sample of K distinct ranks drawn one after another with probability proportional to p."""
    import numpy as np
    L, E = len(perms), len(perms[0])
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    out = np.empty((n, L, T, K), np.int32)
    for l in range(L):
        g = logp + rng.gumbel(size=(n, T, E))
        ranks = np.argpartition(-g, K - 1, axis=-1)[..., :K]
        out[:, l] = np.asarray(perms[l])[ranks]
    return out


def prefill_cpu_baseline(x, ids_np, w_np, P, E, H, I, seconds, tokens=32):
    """The C oracle on a bounded sample of configs[3]: the first `tokens` tokens of the step with their
    routing (every routed expert's FFN, the shared expert, the ordered reduce), on all host cores."""
    import numpy as np
    import torch
    import oracle as O
    threads = len(os.sched_getaffinity(0))
    x_np = x[:tokens].view(torch.int16).cpu().numpy().view(np.uint16)
    ids, w = ids_np[:tokens], w_np[:tokens]
    experts_np = [None] * E
    for e in sorted(set(ids.ravel().tolist())):
        experts_np[e] = {k: v[e].cpu().numpy() for k, v in P.items()}
    shared_np = {k: v[E].cpu().numpy() for k, v in P.items()}
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        O.moe_layer_routed(x_np, ids, w, experts_np, shared_np, H, I, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    per = sum(times) / len(times)
    U = len(set(ids.ravel().tolist()))
    return dict({"value": tokens / per, "unit": "tokens/s", "cores": threads, "kind": "port",
                 "sample": f"{len(times)} passes of the C oracle over the first {tokens} of the 512 tokens with their "
                           f"routing ({U} routed experts + shared), {per * 1e3:.1f} ms each"}, **host_info())


def bench_stack(gpu, steps, warmup, fill_steps, side_steps, cpu_seconds, no_cpu, seed=4):
    """the T=4 verify step through 40 stacked MoE layers (H=4096, I=2880, 384 routed experts
    top-6 + 1 shared, independent seeded weights per layer). Per layer the Zipf(1.1)-hottest 320 experts
    (ranks 1..320 of a seeded per-layer permutation) and the shared expert are HBM-resident; the other 64
    sit in pinned host memory and are copied in with hipMemcpyAsync on the stack's copy stream when
    routed. Inputs bf16 N(0,1) from a pool of 16. Legs, in order:
      zipf          Zipf(1.1) ids (6 distinct per token) drawn fresh every step, no cache
      router        the router on the chained activations (layer l+1 reads layer l's output), no cache
      zipf_cache_fill  from an EMPTY HBM cache sized to the free HBM (the reference's VRAM slot pool over
                    its RAM tier): fresh Zipf ids, each step's host-tier experts prefetched before it
      zipf_cache    the headline: W warmup + K timed steps as zipf_cache_fill, on the cache it left
      router_cache  router routing on the same cache (demand misses, no prefetch)
    Returns (legs, headline cpu baseline)."""
    import numpy as np
    import torch
    import ds41_gfx950 as G
    L, T, H, I, E, K, RES = 40, 4, 4096, 2880, 384, 6, 320
    NH = E - RES
    off, slab = G.slab_layout(H, I)
    spans = [(off[1], I * H // 32), (off[3], I * H // 32), (off[5], H * I // 32)]
    g = torch.Generator(device=gpu).manual_seed(seed)

    def fill(n):  # e2m1 bytes uniform, e8m0 scales uniform over 2^-8..2^-4
        t = torch.randint(0, 256, (n, slab), dtype=torch.uint8, device=gpu, generator=g)
        for o, m in spans:
            t[:, o:o + m].random_(119, 124, generator=g)
        return t

    t0 = time.perf_counter()
    layers, keep, perms = [], [], []
    for l in range(L):
        perm = np.random.default_rng([seed, l]).permutation(E)  # Zipf rank r+1 -> expert perm[r]
        perms.append(perm)
        dev = fill(RES + 1)  # resident experts by rank, then the shared expert
        host = G.HostSlabs(NH, slab)  # pinned host tier of this layer
        tmp = fill(NH)
        host.tensor.copy_(tmp)
        del tmp
        entries = [G.DeviceExpert() for _ in range(E + 1)]  # host-tier entries stay null: never read
        hidx = np.full(E, -1, np.int32)
        for r, e in enumerate(perm):
            if r < RES:
                entries[e] = G.slab_entry(dev[r].data_ptr(), off, int(e))
            else:
                hidx[e] = r - RES
        entries[E] = G.slab_entry(dev[RES].data_ptr(), off, E)
        table = torch.frombuffer(bytearray(b"".join(bytes(e) for e in entries)), dtype=torch.uint8).to(gpu)
        wg = torch.randn((E, H), generator=g, device=gpu, dtype=torch.float32) * 0.02
        layers.append(dict(router_w=wg, router_bias=torch.zeros(E, dtype=torch.float32, device=gpu), table=table,
                           expert_base=0, shared_index=E, host_index=torch.from_numpy(hidx).to(gpu),
                           host_slabs=host.tensor))
        keep.append((dev, host, hidx))
        if l % 10 == 9:
            log(f"stack: {l + 1} layers built, {time.perf_counter() - t0:.1f} s")
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    resident_gb = torch.cuda.memory_allocated() / 1e9
    log(f"stack: {L} layers x ({RES}+1 resident, {NH} host) experts ready in {time.perf_counter() - t0:.1f} s, "
        f"HBM in use {resident_gb:.1f} GB")
    stack = G.VerifyStack(layers, T, H, I, E, K, slab_bytes=slab, weight_layout=LAYOUT["weights"])
    rng = np.random.default_rng(seed)
    pool = 16
    xs = torch.randn((pool, T, H), generator=g, device=gpu, dtype=torch.float32).to(torch.bfloat16)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.current_stream()
    n_fresh = 2 * warmup + side_steps + fill_steps + warmup + steps + 8
    fresh_np = zipf_route_ids_fast(rng, perms, n_fresh, T, K)  # fresh ids: no leg repeats another's routes
    fresh = torch.from_numpy(fresh_np).to(gpu)
    cursor = [0]
    results = {}
    plan = [("zipf", warmup, side_steps, False), ("router", warmup, max(side_steps // 4, 1), False),
            ("zipf_cache_fill", 0, fill_steps, True), ("zipf_cache", warmup, steps, True),
            ("router_cache", warmup, max(side_steps // 4, 1), True)]
    for mode, nwarm, nsteps, cached in plan:
        if cached and mode == "zipf_cache_fill":
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            stack.cache(0)  # as many slabs as the free HBM holds, less 2 GiB
            cs = stack.cache_stats()
            log(f"stack: HBM cache of {cs['slots']} slots ({cs['slots'] * slab / 1e9:.1f} GB) beside "
                f"{resident_gb:.1f} GB of resident experts; {L * NH} host-tier experts in all")
        zipf = mode.startswith("zipf")
        prefetch = cached and zipf

        def step(i):
            if zipf:
                j = cursor[0]
                cursor[0] += 1
                if prefetch:
                    stack.prefetch_routes(fresh_np[j])
                stack.step(xs[i % pool], y, route_ids=fresh[j], stream=stream)
            else:
                stack.step(xs[i % pool], y, stream=stream)
        for i in range(nwarm):
            step(i)
        torch.cuda.synchronize()
        s0 = stack.stats()
        c0 = stack.cache_stats() if cached else None
        ev = G.Events(2)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        ev.record(0, stream)
        for i in range(nsteps):
            step(nwarm + i)
        ev.record(1, stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        ms = ev.elapsed(0, 1) / nsteps
        s1 = stack.stats()
        d = {k: s1[k] - s0[k] for k in s1}
        if d["invalid_layers"] or G.take_status():
            raise AssertionError(f"stack {mode}: invalid routes or kernel status during the timed steps")
        served = d["resident_routed"] + d["cached_routed"]
        # router rows read: with caller route ids a layer scores only its routed experts (a token's
        # weights normalise over its own routed experts); router routing scores all E of them
        router_rows = served + d["host_fetched"] if mode.startswith("zipf") else d["layers"] * E
        hbm = (served + d["layers"]) * EXPERT_BYTES + router_rows * H * 4
        sec = ms * 1e-3 * nsteps
        routing = {"zipf": "Zipf(1.1) ids drawn fresh every step (4b), no cache",
                   "router": "router on chained activations (4a), no cache",
                   "zipf_cache_fill": "Zipf(1.1) ids drawn fresh every step, prefetched into the HBM LFU cache, "
                                      "from an empty cache",
                   "zipf_cache": "Zipf(1.1) ids drawn fresh every step, prefetched into the HBM LFU cache, "
                                 "cache as the fill leg left it",
                   "router_cache": "router on chained activations, HBM LFU cache (demand misses)"}[mode]
        r = {"routing": routing, "warmup": nwarm,
             "steps": nsteps, "ms_per_step": ms, "wall_ms_per_step": wall * 1e3 / nsteps,
             "tokens_per_s": T / (ms * 1e-3),
             "hbm_bytes_per_step": hbm / nsteps, "hbm_gbps": hbm / sec / 1e9,
             "router_rows_per_layer": router_rows / d["layers"],
             "hbm_frac": hbm / sec / 1e9 / PEAK_HBM_GBPS,
             "h2d_bytes_per_step": d["h2d_bytes"] / nsteps, "h2d_gbps": d["h2d_bytes"] / sec / 1e9,
             "resident_routed_per_layer": d["resident_routed"] / d["layers"],
             "cached_routed_per_layer": d["cached_routed"] / d["layers"],
             "host_fetched_per_layer": d["host_fetched"] / d["layers"]}
        if c0 is not None:
            c1 = stack.cache_stats()
            cd = {k: c1[k] - c0[k] for k in c1 if k != "slots"}
            r["cache"] = {"slots": c1["slots"], "bytes": c1["slots"] * slab, "requests": cd["requests"],
                          "hits": cd["hits"], "misses": cd["misses"], "evictions": cd["evictions"],
                          "prefetch_requests": cd["prefetch_requests"], "prefetch_copies": cd["prefetch_copies"],
                          "hit_rate": cd["hits"] / max(cd["requests"], 1)}
            log(f"stack {mode}: cache {r['cache']}")
        results[mode] = r
        log(f"stack {mode}: {ms:.3f} ms/step ({T / (ms * 1e-3):.0f} tok/s), HBM {hbm / sec / 1e9:.0f} GB/s "
            f"({hbm / sec / 1e9 / PEAK_HBM_GBPS * 100:.1f}%), H2D {d['h2d_bytes'] / sec / 1e9:.1f} GB/s, per layer: "
            f"resident {r['resident_routed_per_layer']:.2f} cached {r['cached_routed_per_layer']:.2f} "
            f"copied {r['host_fetched_per_layer']:.2f}")
    stack.close()
    cpu = None
    if not no_cpu:  # layer 0 of the headline workload with one of its Zipf routings, scaled to 40 layers
        j = fresh_np.shape[0] - 1
        ids0 = fresh_np[j, 0]
        wts = np.full((T, K), 1.5 / K, np.float32)  # the step's router weights: the oracle's cost is alike
        dev0, host0, hidx0 = keep[0]
        experts_np = [None] * E
        rank = {int(e): r for r, e in enumerate(perms[0])}
        for e in sorted(set(ids0.ravel().tolist())):
            r = rank[e]
            src = dev0[r].cpu().numpy() if r < RES else host0.tensor[hidx0[e]].numpy()
            experts_np[e] = slab_expert(src, off, H, I)
        shared_np = slab_expert(dev0[RES].cpu().numpy(), off, H, I)
        x_np = xs[0].view(torch.int16).cpu().numpy().view(np.uint16)
        cpu = cpu_layer_baseline(x_np, ids0, wts, experts_np, shared_np, H, I, cpu_seconds, layers=L,
                                 what=", Zipf(1.1) routing of layer 0")
        log(f"configs[4] cpu baseline: {cpu}")
    del layers, keep
    torch.cuda.empty_cache()
    return results, cpu


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed 40-layer steps of the headline leg")
    ap.add_argument("--warmup", type=int, default=5, help="untimed warmup steps before every stack leg")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--layer-steps", type=int, default=200, help="configs[1] layer steps")
    ap.add_argument("--accept-steps", type=int, default=10000)
    ap.add_argument("--prefill-steps", type=int, default=50)
    ap.add_argument("--drafter-steps", type=int, default=300)
    ap.add_argument("--expert-reps", type=int, default=2000)
    ap.add_argument("--stack-fill-steps", type=int, default=1000, help="steps of the cache fill leg")
    ap.add_argument("--stack-side-steps", type=int, default=200, help="steps of the no-cache Zipf leg")
    ap.add_argument("--fp8-shared", type=int, default=1, help="0 skips the FP8 shared-expert leg")
    ap.add_argument("--legs", default="all", help="comma list of expert,layer,accept,prefill,drafter,stack")
    ap.add_argument("--weight-layout", type=int, default=1, help="1 tiled expert weights, 0 row-major")
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="only run 5 plain device copies of this many bytes (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        src = torch.ones(args.copy_probe, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 5 x {args.copy_probe} B device-to-device copies done")
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the verify path "
              "is a single-GPU workload here and multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)
    legs = set(("expert,layer,accept,prefill,drafter,stack" if args.legs == "all" else args.legs).split(","))
    LAYOUT["weights"] = args.weight_layout

    import torch
    gpu = torch.device("cuda:0")
    cs = min(args.cpu_seconds, 8.0)
    expert = bench_expert(gpu, args.expert_reps, cs, args.no_cpu) if "expert" in legs else None
    layer = state = None
    if "layer" in legs or "prefill" in legs:
        layer, state = bench_layer(gpu, args.layer_steps, 20, cs, args.no_cpu or "layer" not in legs,
                                   bool(args.fp8_shared) and "layer" in legs)
        if "layer" not in legs:
            layer = None
    accept = accept_tp = None
    if "accept" in legs and args.accept_steps > 0:
        accept = bench_accept(gpu, args.accept_steps, cs, args.no_cpu)
        log(f"accept: {accept['us_per_step']:.1f} us/step ({accept['us_per_step_graph']:.1f} graph-replayed; "
            f"draft sampling {accept['us_draft_sampling']:.1f}), mean accepted drafts "
            f"{accept['mean_accepted_drafts']:.2f}, cpu {accept['cpu_baseline']}")
        accept_tp = bench_accept(gpu, max(args.accept_steps // 4, 1), cs, args.no_cpu, 0.95)
        log(f"accept top-p 0.95: {accept_tp['us_per_step']:.1f} us/step ({accept_tp['us_per_step_graph']:.1f} "
            f"graph-replayed; draft sampling {accept_tp['us_draft_sampling']:.1f}), sequential-path steps "
            f"{accept_tp['sequential_path_steps']}, cpu {accept_tp['cpu_baseline']}")
    prefill = None
    if "prefill" in legs and args.prefill_steps > 0:
        prefill = bench_prefill(gpu, state["table"], state["E"], args.prefill_steps, 5, P=state["P"],
                                cpu_seconds=cs, no_cpu=args.no_cpu)
    state = None
    torch.cuda.empty_cache()
    drafter = bench_drafter(gpu, args.drafter_steps, 10) if "drafter" in legs and args.drafter_steps > 0 else None
    stack = cpu4 = None
    if "stack" in legs:
        stack, cpu4 = bench_stack(gpu, args.steps, args.warmup, args.stack_fill_steps, args.stack_side_steps, cs,
                                  args.no_cpu)
    head = stack["zipf_cache"] if stack else None
    out = {
        "metric": METRIC, "value": head["tokens_per_s"] if head else None, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"] if head else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4 weights x mxfp8 activations, fp32 accumulate",
        "data": "synthetic (seeded uniform e2m1/e8m0 weights, N(0,1) bf16 rows, random-init routers, Zipf(1.1) ids)",
        "config": {"workload": "configs[4]: T=4 verify step through 40 MoE layers (hidden 4096, 384 routed experts "
                               "I=2880 MXFP4 top-6 + 1 shared); per layer the Zipf(1.1)-hottest 320 experts + shared "
                               "HBM-resident and 64 in pinned host RAM copied in by hipMemcpyAsync on a side stream; "
                               "routing: Zipf(1.1) ids drawn fresh every step, each step's host-tier experts "
                               "prefetched into an HBM LFU cache sized to the HBM left after the resident set, "
                               "warm from the zipf_cache_fill leg of this run (reported in step40)",
                   "tokens": 4, "layers": 40, "hidden": 4096, "inter": 2880, "experts": 384, "topk": 6,
                   "resident_per_layer": 320, "host_tier_per_layer": 64,
                   "weight_layout": "tiled" if LAYOUT["weights"] else "row-major",
                   "cache_slots": head["cache"]["slots"] if head else None},
        "hbm_gbps": head["hbm_gbps"] if head else None, "hbm_frac": head["hbm_frac"] if head else None,
        "roofline": dict(layer["roofline"], measured_on="configs[1] layer launches of this run (the gate/up/act "
                         "kernel every stack layer runs, same shape)") if layer else None,
        "cpu_baseline": cpu4,
        "step40": stack,
        "layer": layer,
        "expert": expert,
        "accept": accept,
        "accept_top_p": accept_tp,
        "prefill": prefill,
        "drafter_experts": drafter,
    }
    if stack and accept:  # acceptance time as a fraction of the 40-layer step (target < 3 %)
        for a in (accept, accept_tp):
            a["frac_of_step40"] = {m: a["us_per_step"] * 1e-3 / r["ms_per_step"] for m, r in stack.items()}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
