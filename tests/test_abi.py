"""The C-ABI library loads and exports every entry point include/smoe_hip.h
declares; argument validation happens before any device call.  Runs without a
GPU (no compute calls)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smoe_hip.h")


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(smoe_(?:metal|hip)_\w+)\s*\(", text)))


def test_header_declares_reference_surface():
    names = declared_functions()
    for n in ("smoe_metal_init", "smoe_metal_destroy", "smoe_metal_fused_ffn", "smoe_metal_wait",
              "smoe_metal_fused_ffn_group", "smoe_metal_fused_ffn_batch", "smoe_metal_wait_ffn_batch",
              "smoe_metal_register_buffer", "smoe_metal_kernel_dispatches"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import smoe_amd
    L = smoe_amd.lib()
    for n in declared_functions():
        assert hasattr(L, n), n
    assert sorted(s[0] for s in smoe_amd.SIGNATURES) == declared_functions()


def test_null_context_is_rejected():
    import smoe_amd
    L = smoe_amd.lib()
    shape = smoe_amd.make_shape(2048, 128, 8, 768)
    assert L.smoe_hip_moe_decode(None, C.byref(shape), None, None, 1, None, None) == smoe_amd.SMOE_ERR_ARG
    assert L.smoe_hip_reserve(None, C.byref(shape), 1) == smoe_amd.SMOE_ERR_ARG
    assert L.smoe_hip_compute_top_k(None, None, 1, 128, 8, None, None, 1) == smoe_amd.SMOE_ERR_ARG
    assert L.smoe_hip_set_stream(None, None) == smoe_amd.SMOE_ERR_ARG
    assert L.smoe_metal_kernel_dispatches(None) == 0
    assert L.smoe_metal_fused_ffn_group(None, None, 1, None, 768, 2048, 2048, 768, 64, 4) is None
    L.smoe_metal_destroy(None)
    L.smoe_metal_wait(None, None, None, 0, 0)
    L.smoe_metal_wait_ffn_batch(None, None, None, 0, 0)
    L.smoe_metal_register_buffer(None, None, 0)


def test_init_without_gpu_returns_null():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import smoe_amd
    assert smoe_amd.lib().smoe_metal_init(1 << 20) is None


def test_blob_layout_matches_oracle(oracle):
    import smoe_amd
    for D, I in ((2048, 768), (4096, 1536), (64, 64)):
        off, raw, stride = smoe_amd.blob_layout(D, I)
        o2, nb = oracle.blob_layout(D, I)
        assert off == o2 and raw == nb and stride % 16384 == 0 and stride >= raw
    assert smoe_amd.blob_layout(2048, 768)[1] == 2506752       # 153 pages, no padding
    assert smoe_amd.blob_layout(4096, 1536)[1] == 10027008     # 612 pages
