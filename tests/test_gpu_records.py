"""Experts loaded from a safetensors checkpoint through the records manifest (ds41_records_*)
feed the decode MoE layer unchanged: the layer over slabs read from disk gives the same output,
bit for bit, as the layer over the same tensors uploaded from memory."""
import os
import sys

import numpy as np
import pytest

import oracle as O
import test_expert_records as R

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_layer_over_file_loaded_experts_bitexact(gpu, tmp_path):
    import torch
    import ds41_gfx950 as G
    H, I, T, K = 512, 256, 4, 3
    root = str(tmp_path / "ckpt")
    os.makedirs(root)
    data = R.make_checkpoint(root, seed=3, h=H, i=I)
    manifest = str(tmp_path / "records.tsv")
    R.write_manifest(root, manifest)
    rs = G.Records(manifest)
    rs.validate(root)
    experts = R.EXPERTS
    E = len(experts)
    say(f"records layer: {E} experts from disk, T={T} H={H} I={I} top-{K}")
    off, slab = G.slab_layout(H, I)
    slabs = torch.empty((E, slab), dtype=torch.uint8, pin_memory=True)
    for j, ex in enumerate(experts):
        rs.load_slab(rs.find(R.expert_id(*ex)), H, I, out=slabs[j])
    dev = slabs.to(gpu)
    table_file = torch.frombuffer(bytearray(b"".join(bytes(G.slab_entry(dev[j].data_ptr(), off, j))
                                                      for j in range(E))), dtype=torch.uint8).to(gpu)
    names = ["w1.weight", "w1.scale", "w3.weight", "w3.scale", "w2.weight", "w2.scale"]
    mem = [{f: torch.from_numpy(data[ex][n]).to(gpu) for f, n in zip(G.SLAB_FIELDS, names)} for ex in experts]
    table_mem, _ = G.device_table(mem, gpu)
    rng = np.random.default_rng(4)
    x = torch.from_numpy(O.bf16_bits(rng.standard_normal((T, H)).astype(np.float32)).view(np.int16)).to(gpu)
    x = x.view(torch.bfloat16)
    wg = torch.from_numpy((rng.standard_normal((E, H)) * 0.05).astype(np.float32)).to(gpu)
    bias = torch.zeros(E, dtype=torch.float32, device=gpu)
    outs = []
    for table in (table_file, table_mem):
        y = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
        ws = torch.zeros(G.layer_workspace_bytes(T, H, I, E, K), dtype=torch.uint8, device=gpu)
        G.moe_layer(G.make_layer_args(x, wg, bias, table, 0, -1, T, H, I, E, K, y, ws))
        torch.cuda.synchronize()
        outs.append(y.view(torch.int16).cpu().numpy())
    assert G.take_status() == 0
    assert np.array_equal(outs[0], outs[1]) and np.any(outs[0] != 0)
