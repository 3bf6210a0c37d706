"""one MXFP4 expert SwiGLU FFN at hidden 1024, intermediate 512, 1 token, through the
reference kernel API's chain on the device (quantize_mxfp8 -> grouped gate and up -> swiglu ->
quantize_mxfp8 -> grouped down), against the oracle's expert FFN, through the C ABI.

Inputs: numpy default_rng(0) in the order W_gate, S_gate, W_up, S_up, W_down, S_down, x (weight
bytes uniform, e8m0 scales uniform over 119..123, x bf16 N(0,1)), as bench.py's configs[0] leg.
Bars:
- MXFP8 quantisation of x and of the SwiGLU row: bit-exact;
- SwiGLU given the device's gate/up rows: bit-exact;
- gate and up projections (their activations are read magnitude-split): every bf16 output within one
  bf16 ulp of the oracle's fp32 accumulation (rounding is half an ulp; the scaled MFMA's own fp32
  rounding may move a value across a rounding boundary), and rel-L2 <= 1e-3 against its bf16 outputs;
- the down projection and the whole chain: rel-L2 <= 1e-3 against the oracle's bf16 outputs, and
  rel-L2 <= 2.2e-3 against its fp32 accumulations: the 1e-3 bar plus what rounding the output to bf16
  alone adds (a relative rounding error of at most 2^-9, about 1.1e-3 RMS). Unsplit, the scaled MFMA
  drops a block's products more than ~14 bits below its largest, so an output that nearly cancels can
  sit many of its own ulps from the exact sum while the vector stays within the bar."""
import numpy as np
import pytest

import oracle as O
from test_gpu_moe import dev, host, rel_l2, say

pytestmark = pytest.mark.gpu
H, I = 1024, 512


def config0_inputs(seed=0):
    rng = np.random.default_rng(seed)
    W = {}
    W["gate"] = rng.integers(0, 256, (I, H // 2), dtype=np.uint8)
    W["gate_scale"] = rng.integers(119, 124, (I, H // 32), dtype=np.uint8)
    W["up"] = rng.integers(0, 256, (I, H // 2), dtype=np.uint8)
    W["up_scale"] = rng.integers(119, 124, (I, H // 32), dtype=np.uint8)
    W["down"] = rng.integers(0, 256, (H, I // 2), dtype=np.uint8)
    W["down_scale"] = rng.integers(119, 124, (H, I // 32), dtype=np.uint8)
    x = O.bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    return W, x


def within_bf16_ulp(got_bits, acc):
    """|bf16 output - fp32 accumulation| <= one bf16 ulp of the accumulation, for every element."""
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    a = np.asarray(acc, np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(a), 1e-30))) - 7)
    return float(np.max(np.abs(got - a) / ulp))


def test_config0_expert_chain_vs_oracle(gpu):
    import torch
    import ds41_gfx950 as G
    W, x_np = config0_inputs(0)
    say(f"configs[0] expert FFN chain H={H} I={I}, 1 token, seed 0")
    W_dev = {k: dev(v, gpu) for k, v in W.items()}  # the table points into these: keep them alive
    table, _ = G.device_table([W_dev], gpu)
    x = dev(x_np, gpu)
    xq, xs = G.quantize_mxfp8(x)
    gate = torch.empty((1, I), dtype=torch.bfloat16, device=gpu)
    up = torch.empty((1, I), dtype=torch.bfloat16, device=gpu)
    G.grouped(table, G.device_jobs([(0, 1, xq, xs, gate)], gpu), 1, G.PROJ_GATE, I, H, entry="ds41_grouped_mxfp4")
    G.grouped(table, G.device_jobs([(0, 1, xq, xs, up)], gpu), 1, G.PROJ_UP, I, H, entry="ds41_grouped_mxfp4")
    h = G.swiglu(gate, up, None, 10.0)
    hq, hs = G.quantize_mxfp8(h)
    out = torch.empty((1, H), dtype=torch.bfloat16, device=gpu)
    G.grouped(table, G.device_jobs([(0, 1, hq, hs, out)], gpu), 1, G.PROJ_DOWN, H, I, entry="ds41_grouped_mxfp4")
    torch.cuda.synchronize()
    assert G.take_status() == 0
    oxq, oxs = O.quantize_mxfp8(x_np)
    assert np.array_equal(host(xq), oxq) and np.array_equal(host(xs), oxs)
    g_acc, g_bf = O.mxfp4_gemm(W["gate"], W["gate_scale"], oxq, oxs, 1, I, H)
    u_acc, u_bf = O.mxfp4_gemm(W["up"], W["up_scale"], oxq, oxs, 1, I, H)
    gg, uu = host(gate), host(up)
    for name, got, acc, bf in (("gate", gg, g_acc, g_bf), ("up", uu, u_acc, u_bf)):
        u_acc_, e_bf = within_bf16_ulp(got, acc), rel_l2(O.bf16_to_f32(got), O.bf16_to_f32(bf))
        say(f"  {name}: max distance to the fp32 accumulations {u_acc_:.2f} bf16 ulp, rel-L2 vs bf16 {e_bf:.2e}, "
            f"bf16 equal {np.mean(got == bf):.4f}")
        assert u_acc_ <= 1.0 and e_bf <= 1e-3
    assert np.array_equal(host(h), O.swiglu(gg, uu, None, 10.0))
    ohq, ohs = O.quantize_mxfp8(host(h))
    assert np.array_equal(host(hq), ohq) and np.array_equal(host(hs), ohs)
    d_acc, d_bf = O.mxfp4_gemm(W["down"], W["down_scale"], ohq, ohs, 1, H, I)
    ob = host(out)
    got = O.bf16_to_f32(ob)
    e_d32, e_d = rel_l2(got, d_acc), rel_l2(got, O.bf16_to_f32(d_bf))
    say(f"  down (device SwiGLU row): rel-L2 vs fp32 {e_d32:.2e}, vs bf16 {e_d:.2e}; max distance to fp32 "
        f"{within_bf16_ulp(ob, d_acc):.1f} bf16 ulp, max |error| / max |output| "
        f"{np.max(np.abs(got - d_acc)) / np.max(np.abs(d_acc)):.2e}")
    assert e_d32 <= 2.2e-3 and e_d <= 1e-3
    ref_bf, ref_acc = O.expert_ffn(W, oxq, oxs, None, H, I, return_acc=True)
    e_f32, e_f = rel_l2(got, ref_acc), rel_l2(got, O.bf16_to_f32(ref_bf))
    say(f"  expert FFN: rel-L2 vs the oracle's fp32 down accumulations {e_f32:.2e}, vs its bf16 output {e_f:.2e}, "
        f"bf16 equal {np.mean(ob == ref_bf):.4f}")
    assert e_f32 <= 2.2e-3 and e_f <= 1e-3
