"""The C-ABI library loads without a GPU and exports every entry point the
public headers declare (no compute calls here)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "deepseek-v4.1-flash-pro6000_amd", "libds41_gfx950.so")


def declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(ds41_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_headers_declare_entry_points():
    names = declared()
    assert "ds41_moe_verify_layer" in names and "ds41_xk_grouped_v1" in names
    assert len(names) >= 25


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail("libds41_gfx950.so not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB)
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_struct_sizes():
    import sys
    sys.path.insert(0, os.path.join(ROOT, "deepseek-v4.1-flash-pro6000_amd"))
    import ds41_gfx950 as G
    assert ctypes.sizeof(G.DeviceExpert) == 64 and ctypes.sizeof(G.GemmJob) == 32
    lib = ctypes.CDLL(LIB)
    assert lib.ds41_xk_projection_abi_version() == 1
    lib.ds41_moe_layer_workspace_bytes.restype = ctypes.c_size_t
    assert lib.ds41_moe_layer_workspace_bytes(4, 4096, 2880, 384, 6) > 0
    # argument validation happens on the host, before any device call
    assert lib.ds41_quantize_mxfp8(None, None, None, 1, 32, None) == 1
    assert lib.ds41_grouped_mxfp4(None, None, 1, 0, 8, 32, None) == 1


def test_stack_abi_host_checks():
    """Layout of the expert slab and the stack descriptors; argument checks that run before any device call."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "deepseek-v4.1-flash-pro6000_amd"))
    import ds41_gfx950 as G
    assert ctypes.sizeof(G.StackLayer) == 56 and ctypes.sizeof(G.StackStats) == 64
    off, slab = G.slab_layout(4096, 2880)
    # the reference's offload slot: 18,800,640 B per expert (gate/up/down weights + e8m0 scales)
    assert slab == 18800640 and off == [0, 5898240, 6266880, 12165120, 12533760, 18432000]
    assert all(o % 256 == 0 for o in off) and slab % 4096 == 0
    with pytest.raises(RuntimeError):
        G.slab_layout(4096, 2881)
    lib = ctypes.CDLL(LIB)
    h = ctypes.c_void_p(0)
    layers = (G.StackLayer * 1)()
    desc = G.StackDesc(1, 4, 4096, 2880, 384, 6, 0, 1.5, 10.0, layers)  # null router/table pointers
    assert lib.ds41_verify_stack_create(ctypes.byref(desc), ctypes.byref(h)) == 1 and not h.value
    desc = G.StackDesc(1, 9, 4096, 2880, 384, 6, 0, 1.5, 10.0, layers)  # 9 tokens > 8
    assert lib.ds41_verify_stack_create(ctypes.byref(desc), ctypes.byref(h)) == 1
    desc = G.StackDesc(1, 4, 4096, 2880, 513, 6, 0, 1.5, 10.0, layers)  # > 512 experts
    assert lib.ds41_verify_stack_create(ctypes.byref(desc), ctypes.byref(h)) == 1
    assert lib.ds41_verify_stack_step(None, None, None, 1, None, None, None, None, None) == 1
    assert lib.ds41_verify_stack_destroy(None) == 1


def test_target_experts_abi_host_checks():
    """Drafter service descriptor layout and the checks that run before any device call."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "deepseek-v4.1-flash-pro6000_amd"))
    import ds41_gfx950 as G
    assert ctypes.sizeof(G.TargetExpertsDesc) == 64
    assert G.TargetExpertsDesc.weight_layout.offset == 56
    lib = ctypes.CDLL(LIB)
    h = ctypes.c_void_p(0)
    d = G.TargetExpertsDesc(0, 0, 5120, 2304, 10.0, 0, None, None, 0)  # null table
    assert lib.ds41_target_experts_create(ctypes.byref(d), ctypes.byref(h)) == 1 and not h.value
    d = G.TargetExpertsDesc(64, 0, 5000, 2304, 10.0, 0, None, None, 0)  # hidden not a multiple of 256
    assert lib.ds41_target_experts_create(ctypes.byref(d), ctypes.byref(h)) == 1 and not h.value
    d = G.TargetExpertsDesc(64, 0, 5120, 2304, 10.0, 0, None, None, 2)  # no such weight layout
    assert lib.ds41_target_experts_create(ctypes.byref(d), ctypes.byref(h)) == 1 and not h.value
    lib.ds41_target_experts_error.restype = ctypes.c_char_p
    assert lib.ds41_target_experts_error(None) == b"null target experts handle"
    assert lib.ds41_target_experts(None, 0, None, None, None, None, 1, None) == -1
    assert lib.ds41_target_experts_destroy(None) == 1
    assert lib.ds41_spark_topk3_gpu(None, None, 1, None) == 1


def test_read_probe_host_checks():
    """ds41_hbm_read_probe rejects bad sizes and pointers before any launch (no GPU needed)."""
    lib = ctypes.CDLL(LIB)
    f = lib.ds41_hbm_read_probe
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    assert f(None, 1024, ctypes.c_void_p(256), 4, None) != 0
    assert f(ctypes.c_void_p(256), 1000, ctypes.c_void_p(256), 4, None) != 0   # not a multiple of 16
    assert f(ctypes.c_void_p(264), 1024, ctypes.c_void_p(256), 4, None) != 0   # misaligned
    assert f(ctypes.c_void_p(256), 1024, ctypes.c_void_p(256), 0, None) != 0   # no workgroups


def test_versioned_structs_lead_with_abi_pair():
    """The structs that grow between builds begin with (abi_version, struct_bytes), the pair the
    reference's C structs carry (engine/include/ds41/target_shared.h:11-13). The Python mirrors fill
    it in; the header's layout puts it at offsets 0 and 4; a caller built against another layout is
    rejected before any field past the pair is read (the device-side half of this check runs in
    tests/test_gpu_moe.py::test_layer_args_abi_pair_checked)."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "deepseek-v4.1-flash-pro6000_amd"))
    import ds41_gfx950 as G
    for cls in (G.MoeLayerArgs, G.StackDesc, G.StackStats, G.CacheStats, G.TargetExpertsDesc):
        assert cls.abi_version.offset == 0 and cls.struct_bytes.offset == 4, cls
        v = cls()
        assert v.abi_version == G.ABI_VERSION == 1 and v.struct_bytes == ctypes.sizeof(cls), cls
        assert "abi_version" not in cls.data_fields() and "struct_bytes" not in cls.data_fields()
    hdr = open(os.path.join(ROOT, "include", "ds41_moe_gfx950.h")).read()
    assert "#define DS41_GFX950_ABI_VERSION 1u" in hdr
    for name in ("ds41_moe_layer_args", "ds41_stack_desc", "ds41_stack_stats", "ds41_cache_stats",
                 "ds41_target_experts_desc"):
        body = hdr.split("typedef struct %s {" % name, 1)[1]
        first = [ln.split(";")[0].split()[-1] for ln in body.splitlines()[1:3]]
        assert first == ["abi_version", "struct_bytes"], (name, first)
    # a descriptor from another build (other size or version) is rejected by the host checks
    lib = ctypes.CDLL(LIB)
    h = ctypes.c_void_p(0)
    layers = (G.StackLayer * 1)()
    for version, size in ((G.ABI_VERSION + 1, ctypes.sizeof(G.StackDesc)),
                          (G.ABI_VERSION, ctypes.sizeof(G.StackDesc) - 8)):
        desc = G.StackDesc(1, 4, 4096, 2880, 384, 6, 0, 1.5, 10.0, layers)
        desc.abi_version, desc.struct_bytes = version, size
        assert lib.ds41_verify_stack_create(ctypes.byref(desc), ctypes.byref(h)) == 1 and not h.value
    st = G.StackStats()
    st.abi_version = 0
    assert lib.ds41_verify_stack_stats(ctypes.c_void_p(1), ctypes.byref(st)) == 1  # rejected before the handle is used
