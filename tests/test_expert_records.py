"""The on-disk expert format (ds41_records_*, host code: runs without a GPU).

A synthetic safetensors checkpoint is written with the `safetensors` package; a records
manifest is made from the shard headers (read here with Python's json, independently of the
library's JSON reader) in the documented R/E format. Checks:
- the library parses the manifest exactly as the reference's own load_records
  (components/moe/src/manifest.cpp, compiled from its sources into oracle/_ref);
- the engine's validation (engine/src/forward.cu:1781-1832) accepts it and rejects each kind
  of mismatch it guards against;
- every expert read from disk and repacked equals its tensors from numpy, byte for byte, in
  the canonical slab layout the kernels read."""
import json
import os
import struct

import numpy as np
import pytest

import ds41_gfx950 as G
import oracle as O

H, I = 64, 32
ALIGN = 4096
FIELDS = ["w1.weight", "w1.scale", "w3.weight", "w3.scale", "w2.weight", "w2.scale"]
def shapes(h, i):
    return {"w1.weight": (i, h // 2), "w1.scale": (i, h // 32), "w3.weight": (i, h // 2), "w3.scale": (i, h // 32),
            "w2.weight": (h, i // 2), "w2.scale": (h, i // 32)}
# (layer, expert): layer >= 40 is drafter stage layer - 40
EXPERTS = [(0, 0), (0, 1), (0, 383), (3, 7), (41, 5)]


def expert_id(layer, e):
    return layer * 384 + e if layer < 40 else 15360 + (layer - 40) * 128 + e


def prefix(layer, e):
    return (f"layers.{layer}" if layer < 40 else f"mtp.{layer - 40}") + f".ffn.experts.{e}"


def make_checkpoint(root, seed=0, h=H, i=I):
    """Two shards; expert tensors interleaved with other tensors, one expert split across shards.
    Returns {expert (layer, e): {field: uint8 array}}."""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(seed)
    shp = shapes(h, i)
    data = {ex: {f: rng.integers(0, 256, shp[f], dtype=np.uint8) for f in FIELDS} for ex in EXPERTS}
    shards = [{}, {}]
    for k, ex in enumerate(EXPERTS):
        for j, f in enumerate(FIELDS):
            shard = 1 if (k == 3 and j >= 4) or k == 4 else 0  # expert 3's w2 lives in the second shard
            shards[shard][f"{prefix(*ex)}.{f}"] = data[ex][f]
    shards[0]["model.layers.0.self_attn.q.weight_scale_inv"] = rng.integers(0, 9, (3, 5)).astype(np.float32)
    shards[1]["model.layers.0.mlp.gate.weight"] = rng.standard_normal((7, 11)).astype(np.float32)
    weight_map = {}
    for i, sh in enumerate(shards):
        name = f"model-{i + 1:05d}-of-00002.safetensors"
        save_file(sh, os.path.join(root, name))
        for k in sh:
            weight_map[k] = name
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)
    return data


def shard_tensors(root):
    """name -> (abs path, absolute offset, bytes, file bytes) from the shard headers."""
    idx = json.load(open(os.path.join(root, "model.safetensors.index.json")))["weight_map"]
    out = {}
    for name, shard in idx.items():
        path = os.path.realpath(os.path.join(root, shard))
        with open(path, "rb") as f:
            n, = struct.unpack("<Q", f.read(8))
            hdr = json.loads(f.read(n))
        lo, hi = hdr[name]["data_offsets"]
        out[name] = (path, 8 + n + lo, hi - lo, os.path.getsize(path))
    return out


def write_manifest(root, path, mutate=None):
    """The R/E lines for every expert: adjacent tensors of one file coalesce into one span, each
    span is read from the 4096-aligned offset below it for an aligned length (which may run past
    EOF: `required` is what must arrive)."""
    t = shard_tensors(root)
    lines = ["# R id bytes (offset bytes)x6; E id path file_offset bytes dst required expected_file_bytes"]
    recs = []
    for ex in EXPERTS:
        ts = {f: t[f"{prefix(*ex)}.{f}"] for f in FIELDS}
        spans = []
        for f, (p, off, n, fb) in sorted(ts.items(), key=lambda kv: (kv[1][0], kv[1][1])):
            if spans and spans[-1]["path"] == p and spans[-1]["off"] + spans[-1]["n"] == off:
                spans[-1]["n"] += n
            else:
                spans.append(dict(path=p, off=off, n=n, fb=fb))
        size, views, extents = 0, {}, []
        for sp in spans:
            ro = sp["off"] // ALIGN * ALIGN
            pre = sp["off"] - ro
            rs = (pre + sp["n"] + ALIGN - 1) // ALIGN * ALIGN
            extents.append([sp["path"], ro, rs, size, pre + sp["n"], sp["fb"]])
            for f, (p, off, n, fb) in ts.items():
                if p == sp["path"] and sp["off"] <= off and off + n <= sp["off"] + sp["n"]:
                    views[f] = [size + off - ro, n]
            size += rs
        recs.append(dict(id=expert_id(*ex), bytes=size, views=[views[f] for f in FIELDS], extents=extents))
    if mutate:
        mutate(recs)
    for r in recs:
        lines.append("R " + " ".join(str(v) for v in [r["id"], r["bytes"]] + [x for v in r["views"] for x in v]))
        for e in r["extents"]:
            lines.append(f"E {r['id']} {json.dumps(e[0])} " + " ".join(str(v) for v in e[1:]))
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    return recs


@pytest.fixture()
def ckpt(tmp_path):
    root = str(tmp_path / "ckpt")
    os.makedirs(root)
    data = make_checkpoint(root)
    manifest = str(tmp_path / "records.tsv")
    recs = write_manifest(root, manifest)
    return root, manifest, data, recs


def ref_records(path):
    R = O.refpool()
    rec = np.zeros((64, 15), np.uint64)
    ext = np.zeros((256, 6), np.uint64)
    paths = np.zeros((256, 4096), np.uint8)
    n_ext = np.zeros(1, np.int32)
    n = R.refrecords_load(path.encode(), 64, rec.ctypes.data, 256, ext.ctypes.data, paths.ctypes.data,
                          n_ext.ctypes.data)
    if n < 0:
        return None
    out = []
    for i in range(n):
        r = rec[i]
        exts = [(bytes(paths[k]).split(b"\0")[0].decode(), *[int(v) for v in ext[k][1:]])
                for k in range(n_ext[0]) if int(ext[k][0]) == i]
        out.append(dict(id=int(r[0]), bytes=int(r[1]), views=[(int(r[2 + 2 * j]), int(r[3 + 2 * j])) for j in range(6)],
                        extents=exts))
    return out


def ours(path):
    rs = G.Records(path)
    return [dict(id=rs.info(i)["id"], bytes=rs.info(i)["bytes"], views=rs.info(i)["views"], extents=rs.extents(i))
            for i in range(rs.count())]


@pytest.mark.skipif(O.refpool() is None, reason="oracle/_ref not built (needs the reference sources)")
def test_manifest_parse_matches_reference(ckpt):
    root, manifest, data, recs = ckpt
    a, b = ours(manifest), ref_records(manifest)
    assert a == b and len(a) == len(EXPERTS)
    assert any(len(r["extents"]) == 2 for r in a)  # the expert split across shards


BAD_MANIFESTS = ["R 1 10 0 1 1 1 2 1 3 1 4 1 5 1\nR 1 10 0 1 1 1 2 1 3 1 4 1 5 1\n",  # duplicate id
                 "E 1 \"/x\" 0 1 0 1 1\n",  # extent before its record
                 "R 15744 10 0 1 1 1 2 1 3 1 4 1 5 1\n",  # id out of range
                 "R 1 10 0 1 1 1 2 1 3 1 4 1\n",  # short record line
                 "X 1\n",
                 "R 1 10 0 1 1 1 2 1 3 1 4 1 5 1\nE 1 \"/x\" 0 1 0\n"]  # short extent line


@pytest.mark.skipif(O.refpool() is None, reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("k", range(len(BAD_MANIFESTS)))
def test_manifest_rejects_like_reference(tmp_path, k):
    p = str(tmp_path / "bad.tsv")
    open(p, "w").write(BAD_MANIFESTS[k])
    assert ref_records(p) is None
    with pytest.raises(ValueError):
        G.Records(p)


def canonical_slab(tensors):
    off, size = G.slab_layout(H, I)
    s = np.zeros(size, np.uint8)
    for o, f in zip(off, FIELDS):
        a = tensors[f].ravel()
        s[o:o + a.size] = a
    return s


def test_validate_and_load_slabs_exact(ckpt):
    root, manifest, data, recs = ckpt
    rs = G.Records(manifest)
    rs.validate(root)
    paths_sizes = {e[0]: e[5] for r in recs for e in r["extents"]}
    assert any(e[1] + e[2] > e[5] for r in recs for e in r["extents"]), "no extent reads past EOF"
    assert all(os.path.getsize(p) == n for p, n in paths_sizes.items())
    for ex in EXPERTS:
        i = rs.find(expert_id(*ex))
        assert i >= 0
        slab = rs.load_slab(i, H, I)
        assert np.array_equal(slab, canonical_slab(data[ex])), ex
        buf = rs.read(i)
        for (o, n), f in zip(rs.info(i)["views"], FIELDS):
            assert np.array_equal(buf[o:o + n], data[ex][f].ravel())
    assert rs.find(12345) == -1


MUTATIONS = {
    "view_offset": lambda recs: recs[0]["views"][2].__setitem__(0, recs[0]["views"][2][0] + 1),
    "view_bytes": lambda recs: recs[1]["views"][0].__setitem__(1, recs[1]["views"][0][1] - 16),
    "wrong_file": lambda recs: recs[3]["extents"][1].__setitem__(0, recs[0]["extents"][0][0]),
    "expected_size": lambda recs: recs[0]["extents"][0].__setitem__(5, recs[0]["extents"][0][5] + 1),
    "extra_extent": lambda recs: recs[2]["extents"].append(
        [recs[2]["extents"][0][0], 0, ALIGN, recs[2]["bytes"], ALIGN, recs[2]["extents"][0][5]])
    or recs[2].__setitem__("bytes", recs[2]["bytes"] + ALIGN),
    "required_over_bytes": lambda recs: recs[0]["extents"][0].__setitem__(4, recs[0]["extents"][0][2] + 1),
    "overlap": lambda recs: recs[3]["extents"][1].__setitem__(3, 0),
    "duplicate_id": lambda recs: recs[1].__setitem__("id", recs[0]["id"]),
    "absent_expert": lambda recs: recs[0].__setitem__("id", expert_id(5, 5)),
    "span_past_record": lambda recs: recs[0].__setitem__("bytes", recs[0]["extents"][-1][3] + 8),
    "empty_extent": lambda recs: recs[1]["extents"].append(
        [recs[1]["extents"][0][0], 0, 0, recs[1]["bytes"], 0, recs[1]["extents"][0][5]]),
    "required_past_file": lambda recs: recs[4]["extents"][0].__setitem__(4, recs[4]["extents"][0][5] + 1),
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_validate_rejects(tmp_path, name):
    root = str(tmp_path / "ckpt")
    os.makedirs(root)
    make_checkpoint(root)
    manifest = str(tmp_path / "records.tsv")
    write_manifest(root, manifest, MUTATIONS[name])
    try:
        rs = G.Records(manifest)
    except ValueError:
        assert name == "duplicate_id"  # the parser already refuses a repeated id
        return
    with pytest.raises(ValueError):
        rs.validate(root)


def test_checkpoint_checks(tmp_path):
    root = str(tmp_path / "ckpt")
    os.makedirs(root)
    make_checkpoint(root)
    manifest = str(tmp_path / "records.tsv")
    write_manifest(root, manifest)
    rs = G.Records(manifest)
    shard = os.path.join(root, "model-00002-of-00002.safetensors")
    raw = open(shard, "rb").read()
    open(shard, "wb").write(raw[:-3])  # truncated shard
    with pytest.raises(ValueError, match="incomplete"):
        rs.validate(root)
    rs.validate(root, complete=False)  # complete=0 skips only the shard-size check
    n, = struct.unpack("<Q", raw[:8])
    hdr = json.loads(raw[8:8 + n])
    for key, bad in (("dtype", "Q7"), ("data_offsets", None)):
        h = json.loads(json.dumps(hdr))
        name = next(k for k in h if k != "__metadata__")
        if key == "dtype":
            h[name]["dtype"] = bad
        else:
            lo, hi = h[name]["data_offsets"]
            h[name]["data_offsets"] = [lo + 1, hi + 1]  # a gap before it
        body = json.dumps(h).encode()
        open(shard, "wb").write(struct.pack("<Q", len(body)) + body + raw[8 + n:])
        with pytest.raises(ValueError):
            rs.validate(root, complete=False)


def _rewrite_index(root, fn):
    p = os.path.join(root, "model.safetensors.index.json")
    idx = json.load(open(p))
    fn(idx["weight_map"])
    json.dump(idx, open(p, "w"))


@pytest.mark.parametrize("case", ["unsafe_path", "absolute_path", "duplicate_engine_name", "header_too_long"])
def test_checkpoint_rejects(tmp_path, case):
    """The checkpoint index and shard checks of engine/src/store.cpp:140-217 (as rules, not text): shard
    names stay inside the checkpoint directory, two source names may not map to one engine name, and a
    header length must be 1 .. 128 MiB."""
    root = str(tmp_path / "ckpt")
    os.makedirs(root)
    make_checkpoint(root)
    manifest = str(tmp_path / "records.tsv")
    write_manifest(root, manifest)
    rs = G.Records(manifest)
    rs.validate(root)
    if case == "unsafe_path":
        _rewrite_index(root, lambda m: m.__setitem__(next(iter(m)), "../" + m[next(iter(m))]))
    elif case == "absolute_path":
        _rewrite_index(root, lambda m: m.__setitem__(next(iter(m)), os.path.join(root, m[next(iter(m))])))
    elif case == "duplicate_engine_name":
        # "model.layers.0.mlp.gate.weight" normalises to "layers.0.ffn.gate.weight": add the second spelling
        shard = os.path.join(root, "model-00002-of-00002.safetensors")
        raw = open(shard, "rb").read()
        n, = struct.unpack("<Q", raw[:8])
        hdr = json.loads(raw[8:8 + n])
        hdr["layers.0.ffn.gate.weight"] = dict(hdr["model.layers.0.mlp.gate.weight"])
        hdr["layers.0.ffn.gate.weight"]["data_offsets"] = [0, 0]
        hdr["layers.0.ffn.gate.weight"]["shape"] = [0]
        body = json.dumps(hdr).encode()
        open(shard, "wb").write(struct.pack("<Q", len(body)) + body + raw[8 + n:])
        _rewrite_index(root, lambda m: m.__setitem__("layers.0.ffn.gate.weight", "model-00002-of-00002.safetensors"))
    else:
        shard = os.path.join(root, "model-00001-of-00002.safetensors")
        raw = bytearray(open(shard, "rb").read())
        raw[:8] = struct.pack("<Q", (128 << 20) + 1)
        open(shard, "wb").write(bytes(raw))
    with pytest.raises(ValueError):
        rs.validate(root)
