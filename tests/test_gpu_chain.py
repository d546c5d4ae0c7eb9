"""The chained decode engine (SMOE_DECODE_CHAIN: the decode.cpp:121 layer loop
over decode.cpp:236-509 in one launch, the single-launch layer kernel's wave
schedule per layer) against the per-layer launches and the CPU oracle.

The chain computes every layer exactly as the single-launch layer kernel
does (same waves, same exchanges, same summation order; only where the
layer's input comes from differs), so a chained stack must equal the same
layers run one call at a time bit for bit.  Four layers are also checked
against the oracle (ids bit-exact, MoE delta and hidden within 1e-3)."""
import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import Layer, hidden_states, moe_delta_err, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture
def chain(ctx):
    ctx.set_decode_engine(smoe_amd.DECODE_CHAIN)
    yield
    ctx.set_decode_engine(smoe_amd.DECODE_CHAIN)


def run_stack(ctx, layers, hid, ids=True):
    K = layers[0].K
    n = len(layers)
    i = torch.zeros((n, K), dtype=torch.int32, device="cuda")
    w = torch.zeros((n, K), dtype=torch.float32, device="cuda")
    ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], hid.data_ptr(),
                         i.data_ptr() if ids else None, w.data_ptr() if ids else None)
    ctx.synchronize()
    return i.cpu().numpy().view(np.uint32), w.cpu().numpy()


def test_chain_engine_is_used(ctx, chain):
    """The 30B shape runs as one chained launch (not a fallback)."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=200 + i, host=False) for i in range(3)]
    hid = hidden_states(ctx, 1, 2048, 1)[0]
    ctx.profile_enable(True)
    run_stack(ctx, layers, hid)
    n, _ = ctx.profile_read(smoe_amd.KERNEL_CHAIN)
    m, _ = ctx.profile_read(smoe_amd.KERNEL_MOE_LAYER)
    ctx.profile_enable(False)
    assert (n, m) == (1, 0)


@pytest.mark.parametrize("n", [1, 2, 7, 12])
def test_chain_equals_layer_calls(ctx, oracle, chain, n):
    """n layers in one chained launch equal n single-layer calls bit for bit
    (hidden, ids, weights); the first two and last two layers agree with the
    oracle on the GPU's own input of that layer."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=210 + i, host=False) for i in range(n)]
    x0 = hidden_states(ctx, 1, 2048, 31)[0]
    full = x0.clone()
    fids, fw = run_stack(ctx, layers, full)
    step = x0.clone()
    worst = 0.0
    for i, layer in enumerate(layers):
        h_in = step.cpu().numpy()
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        w = torch.zeros(8, dtype=torch.float32, device="cuda")
        ctx.moe_decode(layer.shape, layer.layer, step.data_ptr(), 1, ids.data_ptr(), w.data_ptr())
        ctx.synchronize()
        gids, gw = ids.cpu().numpy().view(np.uint32), w.cpu().numpy()
        assert (gids == fids[i]).all() and (gw == fw[i]).all(), i
        if i in (0, 1, n - 2, n - 1):
            layer.host_copies()
            out, oid, ow, logits, normed, yo = layer.oracle_decode(oracle, h_in)
            assert (gids == oid).all()
            assert np.allclose(gw, ow, rtol=1e-5, atol=1e-7)
            e1, _ = moe_delta_err(step.cpu().numpy(), h_in, yo, ow)
            e2, _ = rel_err(step.cpu().numpy(), out)
            worst = max(worst, e1, e2)
            del layer.h_pool
    assert torch.equal(full, step)
    print(f"chain x{n}: worst layer rel_err {worst:.2e}")
    assert worst <= TOL


def test_chain_repeated_calls_shape_change_and_graph_replay(ctx, chain):
    """Calls in a row (with and without routing outputs), a shorter chain in
    between, and replays of a captured graph with eager chains between them
    all reproduce the first call."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=230 + i, host=False) for i in range(6)]
    x0 = hidden_states(ctx, 1, 2048, 33)[0]
    ref = x0.clone()
    rids, _ = run_stack(ctx, layers, ref)
    for k in range(3):
        buf = x0.clone()
        ids, _ = run_stack(ctx, layers, buf, ids=k != 1)
        assert torch.equal(buf, ref)
        if k != 1:
            assert (ids == rids).all()
    tmp = x0.clone()
    run_stack(ctx, layers[:3], tmp)
    buf = x0.clone()
    ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], buf.data_ptr())   # table upload, eager
    ctx.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        ctx.set_stream(s.cuda_stream)
        with torch.cuda.graph(g, stream=s):
            ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], buf.data_ptr())
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    for _ in range(4):
        buf.copy_(x0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(buf, ref)
        junk = x0.clone()
        ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], junk.data_ptr())
        ctx.synchronize()
        assert torch.equal(junk, ref)


@pytest.mark.parametrize("D,I", [(4096, 1536), (2048, 768)])
@pytest.mark.parametrize("ties", [False, True])
def test_chain_shapes_equal_layer_calls(ctx, chain, D, I, ties):
    """At both Qwen3 shapes the chain engine runs one chained launch and equals
    the per-layer launches bit for bit; also with router rows duplicated in
    pairs (exact logit ties at every rank boundary, where the proposed ranks
    give way to the exact selection and rows requested for an overturned
    proposal, down rows first in the 30B chain, are requested again)."""
    layers = [Layer(ctx, D, 128, 8, I, layer_id=240 + i + I, host=False) for i in range(3)]
    if ties:
        for l in layers:
            rows = l.router.view(128, D)
            rows[1::2] = rows[0::2]
        torch.cuda.synchronize()
    x0 = hidden_states(ctx, 1, D, 34)[0]
    a = x0.clone()
    ctx.profile_enable(True)
    aids, aw = run_stack(ctx, layers, a)
    n, _ = ctx.profile_read(smoe_amd.KERNEL_CHAIN)
    ctx.profile_enable(False)
    assert n == 1
    ctx.set_decode_engine(smoe_amd.DECODE_LAUNCHES)
    b = x0.clone()
    bids, bw = run_stack(ctx, layers, b)
    assert torch.equal(a, b) and (aids == bids).all() and (aw == bw).all()


def test_chain_other_shapes_take_the_launches(ctx, chain):
    """A shape the chained kernel does not take (d_model 4096 with 32 down
    rows a wave: it would spill registers) runs as one-launch layer kernels
    under the chain engine, with the same results as the launches engine."""
    layers = [Layer(ctx, 4096, 128, 8, 1280, layer_id=250 + i, host=False) for i in range(2)]
    x0 = hidden_states(ctx, 1, 4096, 35)[0]
    a = x0.clone()
    ctx.profile_enable(True)
    run_stack(ctx, layers, a)
    n, _ = ctx.profile_read(smoe_amd.KERNEL_CHAIN)
    m, _ = ctx.profile_read(smoe_amd.KERNEL_MOE_LAYER)
    ctx.profile_enable(False)
    assert (n, m) == (0, 2)
    ctx.set_decode_engine(smoe_amd.DECODE_LAUNCHES)
    b = x0.clone()
    run_stack(ctx, layers, b)
    assert torch.equal(a, b)
