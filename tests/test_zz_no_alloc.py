"""smoe_hip_moe_decode_static (the allocation-free single-token decode) against
smoe_hip_moe_decode with n_tokens = 1, called through the C ABI: the same
kernels, so ids, weights and the updated hidden state must be bit-identical.
Two calls in a row per form, the second on a smaller shape; shapes above the
static scratch's limits are rejected with SMOE_ERR_CAPACITY."""
import ctypes as C

import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import Layer, hidden_states

pytestmark = pytest.mark.gpu


def static_decode(layer, hidden, ids, w, err):
    stream = torch.cuda.current_stream().cuda_stream
    return smoe_amd.lib().smoe_hip_moe_decode_static(C.byref(layer.shape), C.byref(layer.layer), hidden.data_ptr(),
                                                     ids.data_ptr(), w.data_ptr(), err.data_ptr(), stream)


@pytest.mark.parametrize("shapes", [
    # one-launch layer kernel (k = 8), then a smaller shape
    ((2048, 128, 8, 768), (1024, 64, 8, 512)),
    # the two-launch form (k != 8), then a smaller shape
    ((1024, 64, 4, 512), (512, 32, 2, 256)),
    # the 235B shape, then the 30B shape
    ((4096, 128, 8, 1536), (2048, 128, 8, 768)),
])
def test_static_decode_matches_decode(ctx, shapes):
    for i, (D, E, K, I) in enumerate(shapes):
        layer = Layer(ctx, D, E, K, I, layer_id=300 + 7 * i + D // 64, host=False)
        for index0 in (11, 12):
            x = hidden_states(ctx, 1, D, index0=index0 + i)[0]
            a, b = x.clone(), x.clone()
            ia = torch.zeros(K, dtype=torch.int32, device="cuda")
            wa = torch.zeros(K, dtype=torch.float32, device="cuda")
            ib, wb = torch.full_like(ia, -1), torch.full_like(wa, -1.0)
            err = torch.zeros(1, dtype=torch.int32, device="cuda")
            ctx.moe_decode(layer.shape, layer.layer, a.data_ptr(), 1, ia.data_ptr(), wa.data_ptr())
            assert static_decode(layer, b, ib, wb, err) == smoe_amd.SMOE_OK
            ctx.synchronize()
            torch.cuda.synchronize()
            assert int(err.item()) == 0
            assert torch.equal(ia, ib), (ia, ib)
            assert torch.equal(wa, wb)
            assert torch.equal(a, b), float((a - b).abs().max())
            assert not torch.equal(a, x)


def test_static_decode_rejects_large_shapes(ctx):
    lib = smoe_amd.lib()
    stream = torch.cuda.current_stream().cuda_stream
    h = torch.zeros(8192, dtype=torch.float32, device="cuda")
    lay = smoe_amd.make_layer(h.data_ptr(), h.data_ptr(), h.data_ptr(), 1 << 20, [0] * 6)
    for D, E, K, I in ((8192, 128, 8, 768), (2048, 128, 8, 4096)):
        shape = smoe_amd.make_shape(D, E, K, I)
        rc = lib.smoe_hip_moe_decode_static(C.byref(shape), C.byref(lay), h.data_ptr(), None, None, None, stream)
        assert rc == smoe_amd.SMOE_ERR_CAPACITY
    assert lib.smoe_hip_moe_decode_static(None, C.byref(lay), h.data_ptr(), None, None, None, stream) == \
        smoe_amd.SMOE_ERR_ARG


@pytest.mark.parametrize("D,E,K,I", [
    (2048, 128, 8, 768),     # one launch (k = 8)
    (1024, 64, 4, 512),      # two launches (k != 8)
])
def test_static_decode_graph_replay(ctx, D, E, K, I):
    """The static call captured into a graph (its scratch already set up by
    smoe_metal_init): replays with eager static calls between them, each
    replay bit-identical to smoe_hip_moe_decode on the same input."""
    layer = Layer(ctx, D, E, K, I, layer_id=400 + K, host=False)
    x0 = hidden_states(ctx, 1, D, index0=21)[0]
    ref = x0.clone()
    rid = torch.zeros(K, dtype=torch.int32, device="cuda")
    rw = torch.zeros(K, dtype=torch.float32, device="cuda")
    ctx.moe_decode(layer.shape, layer.layer, ref.data_ptr(), 1, rid.data_ptr(), rw.data_ptr())
    ctx.synchronize()
    buf = x0.clone()
    ids = torch.full((K,), -1, dtype=torch.int32, device="cuda")
    w = torch.full((K,), -1.0, dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = smoe_amd.lib().smoe_hip_moe_decode_static(C.byref(layer.shape), C.byref(layer.layer),
                                                           buf.data_ptr(), ids.data_ptr(), w.data_ptr(),
                                                           err.data_ptr(), s.cuda_stream)
    assert rc == smoe_amd.SMOE_OK
    for rep in range(4):
        buf.copy_(x0)
        ids.fill_(-1)
        w.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        assert torch.equal(ids, rid) and torch.equal(w, rw), rep
        assert torch.equal(buf, ref), (rep, float((buf - ref).abs().max()))
        # eager work on the same scratch between replays
        junk = hidden_states(ctx, 1, D, index0=40 + rep)[0]
        ji, jw = torch.zeros_like(ids), torch.zeros_like(w)
        assert static_decode(layer, junk, ji, jw, err) == smoe_amd.SMOE_OK
        torch.cuda.synchronize()
        assert int(err.item()) == 0
