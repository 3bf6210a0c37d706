"""The verify layer captured in a HIP graph and replayed (the reference captures each per-layer
body once and replays it: engine/src/forward.cu:1098-1120; engine/src/hotpath/batch.inc:336-344),
through the C ABI: ds41_moe_verify_layer and ds41_moe_verify_layer_noalloc.

The captured launches read their inputs from the same device buffers at every replay (the
reference kernel API re-reads its tables and jobs at each replay), so writing new inputs into the
buffers and replaying must give the bits an eager call gives on those inputs. Each replay is
followed by eager work (the copies of the next inputs and an eager reference call on other
buffers) and a synchronisation, and every replay is checked."""
import numpy as np
import pytest

from test_gpu_moe import dev, host, make_layer, rand_x, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("noalloc", [False, True])
def test_layer_graph_replays_match_eager(gpu, noalloc):
    import torch
    import ds41_gfx950 as G
    T, H, I, E, K = 4, 1024, 512, 32, 6
    say(f"graph-captured verify layer (noalloc={noalloc}) T={T} H={H} I={I} E={E}")
    P, experts = make_layer(gpu, 91, H, I, E, T)
    table, _ = G.device_table(experts, gpu)
    rng = np.random.default_rng(92)
    wg = dev((rng.standard_normal((E, H)) * 0.02).astype(np.float32), gpu)
    bias = dev(np.zeros(E, np.float32), gpu)
    inputs = [dev(rand_x(rng, T, H), gpu) for _ in range(4)]

    def buffers():
        x = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
        y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
        ids = torch.empty((T, K), dtype=torch.int32, device=gpu)
        wts = torch.empty((T, K), dtype=torch.float32, device=gpu)
        ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
        args = G.make_layer_args(x, wg, bias, table, 0, E, T, H, I, E, K, y, ws, ids_out=ids, weights_out=wts)
        return dict(x=x, y=y, ids=ids, wts=wts, ws=ws, args=args)

    def call(b, use_noalloc, stream=None):
        if use_noalloc:
            b["args"].workspace, b["args"].workspace_bytes = 0, 0
            G.check(G.moe_layer_noalloc_rc(b["args"], stream), "ds41_moe_verify_layer_noalloc")
        else:
            G.moe_layer(b["args"], stream)

    cap, ref = buffers(), buffers()
    # eager first: one-time set-up (LDS limits, the no-alloc array's address) happens outside capture
    cap["x"].copy_(inputs[0])
    call(cap, noalloc)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(cap, noalloc, stream=s)
    torch.cuda.synchronize()
    for r, x in enumerate(inputs):
        cap["x"].copy_(x)
        cap["y"].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = [host(cap[k]).copy() for k in ("y", "ids", "wts")]
        # the eager reference on its own buffers (the workspace path for both entries: the
        # no-alloc array is the graph's own)
        ref["x"].copy_(x)
        call(ref, False)
        torch.cuda.synchronize()
        want = [host(ref[k]) for k in ("y", "ids", "wts")]
        assert G.take_status() == 0
        for a, b in zip(got, want):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"replay {r}"
        say(f"  replay {r}: y, ids and weights equal the eager call's bits")
