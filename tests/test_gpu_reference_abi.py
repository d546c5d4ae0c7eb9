"""The reference surface (smoe_metal_fused_ffn / _group / _batch + waits,
metal_bridge.h:74-154) against the oracle expert FFN, expert by expert."""
import ctypes as C

import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import Layer, rel_err

pytestmark = pytest.mark.gpu


def blob_ptrs(layer, e):
    base = layer.pool.data_ptr() + e * layer.stride
    return [base + o for o in layer.off]


@pytest.mark.parametrize("D,I,E", [(2048, 768, 16), (4096, 1536, 16)])
def test_group_dispatch_per_slot(ctx, oracle, D, I, E):
    """smoe_metal_fused_ffn_group (the decode dispatch, decode.cpp:386-392)
    with 5 experts in scattered slots, then all 16 slots at once, and the
    single-expert smoe_metal_fused_ffn: every slot's output against the
    oracle's decode-path FFN (qrow_dot2 / qrow_dot, kernels.metal:159-365)."""
    layer = Layer(ctx, D, E, 8, I, layer_id=9 + D // 1024)
    L = smoe_amd.lib()
    x = np.random.default_rng(0).standard_normal(D).astype(np.float32)
    worst = 0.0
    for experts, slots in (([3, 0, 15, 7, 8], [4, 0, 9, 15, 1]), (list(range(16))[::-1], list(range(16)))):
        blobs = [smoe_amd.SmoeExpertBlob(*blob_ptrs(layer, e), s) for e, s in zip(experts, slots)]
        before = ctx.dispatches()
        h = ctx.fused_ffn_group(blobs, x.ctypes.data, I, D)
        assert h
        assert ctx.dispatches() - before == len(experts)
        for e, s in zip(experts, slots):
            out = np.zeros(D, np.float32)
            ctx.wait(h, out.ctypes.data, s, D)
            _, y = oracle.expert_ffn(layer.h_pool[e * layer.stride:(e + 1) * layer.stride], layer.off, D, I, x,
                                     decode=True)
            worst = max(worst, rel_err(out, y)[0])
    # single-expert entry point
    hv = np.zeros(I, np.float32)
    ov = np.zeros(D, np.float32)
    h1 = L.smoe_metal_fused_ffn(ctx.ptr, *blob_ptrs(layer, 5), x.ctypes.data, hv.ctypes.data, ov.ctypes.data,
                                I, D, D, I, 64, 4, 2)
    assert h1
    out = np.zeros(D, np.float32)
    L.smoe_metal_wait(ctx.ptr, h1, out.ctypes.data, 2, D)
    _, y = oracle.expert_ffn(layer.h_pool[5 * layer.stride:6 * layer.stride], layer.off, D, I, x, decode=True)
    worst = max(worst, rel_err(out, y)[0])
    print(f"fused_ffn_group D={D}: worst slot rel_err {worst:.2e}")
    assert worst <= 1e-3


@pytest.mark.parametrize("D,I,B", [(2048, 768, 37), (4096, 1536, 64)])
def test_batch_dispatch(ctx, oracle, D, I, B):
    """smoe_metal_fused_ffn_batch (the prefill dispatch, prefill.cpp:371-381)
    on B token rows (64 = its maximum): every row against the oracle's
    token-batch FFN (kernels.metal:672-769)."""
    layer = Layer(ctx, D, 4, 2, I, layer_id=11 + D // 1024)
    L = smoe_amd.lib()
    X = np.random.default_rng(1).standard_normal((B, D)).astype(np.float32)
    h = L.smoe_metal_fused_ffn_batch(ctx.ptr, *blob_ptrs(layer, 2), X.ctypes.data, B, I, D, D, I, 64, 4)
    assert h
    out = np.zeros((B, D), np.float32)
    L.smoe_metal_wait_ffn_batch(ctx.ptr, h, out.ctypes.data, B, D)
    blob = layer.h_pool[2 * layer.stride:3 * layer.stride]
    worst = 0.0
    with oracle.threads(oracle.usable_cores()):
        for b in range(B):
            _, y = oracle.expert_ffn(blob, layer.off, D, I, X[b])
            worst = max(worst, rel_err(out[b], y)[0])
    print(f"fused_ffn_batch D={D} B={B}: worst row rel_err {worst:.2e}")
    assert worst <= 1e-3


def test_reference_surface_rejections(ctx):
    L = smoe_amd.lib()
    x = np.zeros(2048, np.float32)
    dummy = [1 << 20] * 6
    # batch above SMOE_MAX_FFN_BATCH -> NULL (caller falls back, prefill.cpp:386-405)
    assert L.smoe_metal_fused_ffn_batch(ctx.ptr, *dummy, x.ctypes.data, 65, 768, 2048, 2048, 768, 64, 4) is None
    # bits != 4, group not a multiple of 32, mismatched dims -> NULL
    blob = smoe_amd.SmoeExpertBlob(*dummy, 0)
    arr = (smoe_amd.SmoeExpertBlob * 1)(blob)
    assert L.smoe_metal_fused_ffn_group(ctx.ptr, arr, 1, x.ctypes.data, 768, 2048, 2048, 768, 64, 2) is None
    assert L.smoe_metal_fused_ffn_group(ctx.ptr, arr, 1, x.ctypes.data, 768, 2048, 2048, 768, 48, 4) is None
    assert L.smoe_metal_fused_ffn_group(ctx.ptr, arr, 1, x.ctypes.data, 768, 2048, 2048, 512, 64, 4) is None
    assert L.smoe_metal_fused_ffn_group(ctx.ptr, arr, 17, x.ctypes.data, 768, 2048, 2048, 768, 64, 4) is None
    # slot out of range
    bad = (smoe_amd.SmoeExpertBlob * 1)(smoe_amd.SmoeExpertBlob(*dummy, 16))
    assert L.smoe_metal_fused_ffn_group(ctx.ptr, bad, 1, x.ctypes.data, 768, 2048, 2048, 768, 64, 4) is None
    # device-resident entry: bits / shape errors are status codes
    shape = smoe_amd.make_shape(2048, 128, 8, 768, bits=2)
    lay = smoe_amd.make_layer(1 << 20, 1 << 20, 1 << 20, 1 << 22, [0] * 6)
    assert L.smoe_hip_moe_decode(ctx.ptr, C.byref(shape), C.byref(lay), 1 << 20, 1, None, None) == smoe_amd.SMOE_ERR_BITS
    shape = smoe_amd.make_shape(2048, 128, 17, 768)
    assert L.smoe_hip_moe_decode(ctx.ptr, C.byref(shape), C.byref(lay), 1 << 20, 1, None, None) == smoe_amd.SMOE_ERR_SHAPE
    shape = smoe_amd.make_shape(2000, 128, 8, 768)
    assert L.smoe_hip_moe_decode(ctx.ptr, C.byref(shape), C.byref(lay), 1 << 20, 1, None, None) == smoe_amd.SMOE_ERR_SHAPE


def test_scout_matvec_bf16(ctx, oracle):
    """metal_bridge.h:157-161: dense bf16 GEMV with host vectors, and the
    batch form (metal_bridge.h:198-204), against the compiled-reference-pinned
    oracle matvec (rtol 1e-5: only the fp32 summation order differs)."""
    L = smoe_amd.lib()
    rng = np.random.default_rng(3)
    for rows, cols in ((128, 2048), (37, 100), (512, 4096)):
        w = torch.empty(rows * cols, dtype=torch.int16, device="cuda")
        ctx.synth_bf16(w.data_ptr(), rows * cols, 5, rows, 0.02)
        x = rng.standard_normal(cols).astype(np.float32)
        out = np.zeros(rows, np.float32)
        L.smoe_metal_scout_matvec_bf16(ctx.ptr, w.data_ptr(), x.ctypes.data, out.ctypes.data, rows, cols)
        ref = oracle.matvec_bf16(w.cpu().numpy().view(np.uint16).reshape(rows, cols), x)
        assert np.allclose(out, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
    # batch of two
    ws = [torch.empty(64 * 256, dtype=torch.int16, device="cuda") for _ in range(2)]
    for i, w in enumerate(ws):
        ctx.synth_bf16(w.data_ptr(), 64 * 256, 6, i, 0.02)
    xs = [rng.standard_normal(256).astype(np.float32) for _ in range(2)]
    outs = [np.zeros(64, np.float32) for _ in range(2)]
    VP = C.c_void_p
    L.smoe_metal_scout_matvec_batch_bf16(
        ctx.ptr, (VP * 2)(*[w.data_ptr() for w in ws]), (VP * 2)(*[x.ctypes.data for x in xs]),
        (VP * 2)(*[o.ctypes.data for o in outs]), (C.c_uint32 * 2)(64, 64), (C.c_uint32 * 2)(256, 256), 2)
    for w, x, o in zip(ws, xs, outs):
        ref = oracle.matvec_bf16(w.cpu().numpy().view(np.uint16).reshape(64, 256), x)
        assert np.allclose(o, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
