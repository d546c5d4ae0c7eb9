"""The prefetching persistent decode engine (SMOE_DECODE_PREFETCH: the
decode.cpp:121 layer loop in one launch, each CU copying its slice of the next
layer's predicted experts into LDS) against the CPU oracle of
decode.cpp:236-509.

A prediction only decides where a layer's weights come from (a slice already
in LDS, or one fetched after the layer's top-k), never what is computed, so a
multi-layer call must equal the same layers run one call at a time bit for bit
(a one-layer call predicts nothing: every slice is fetched after its top-k),
whatever mix of hits and misses the multi-layer call had.  Ids bit-exact;
MoE delta and hidden within 1e-3 per element (rel_err)."""
import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import Layer, hidden_states, moe_delta_err, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture
def prefetch(ctx):
    ctx.set_decode_engine(smoe_amd.DECODE_PREFETCH)
    yield
    ctx.set_decode_engine(smoe_amd.DECODE_CHAIN)


def run_stack(ctx, layers, hid):
    K = layers[0].K
    ids = torch.zeros((len(layers), K), dtype=torch.int32, device="cuda")
    w = torch.zeros((len(layers), K), dtype=torch.float32, device="cuda")
    ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], hid.data_ptr(), ids.data_ptr(), w.data_ptr())
    ctx.synchronize()
    return ids.cpu().numpy().view(np.uint32), w.cpu().numpy()


def check_layer(oracle, layer, h_in, h_out, gids, gw):
    out, oid, ow, logits, normed, yo = layer.oracle_decode(oracle, h_in)
    assert (gids == oid).all(), (gids, oid)
    assert np.allclose(gw, ow, rtol=1e-5, atol=1e-7)
    e1, _ = moe_delta_err(h_out, h_in, yo, ow)
    e2, _ = rel_err(h_out, out)
    return max(e1, e2)


def test_prefetch_engine_is_used(ctx, prefetch):
    """The shapes below run on the prefetching kernel (not a fallback)."""
    layer = Layer(ctx, 2048, 128, 8, 768, layer_id=60, host=False)
    hid = hidden_states(ctx, 1, 2048, 1)[0]
    ctx.profile_enable(True)
    run_stack(ctx, [layer, layer], hid)
    n, _ = ctx.profile_read(smoe_amd.KERNEL_STACK_PREFETCH)
    ctx.profile_enable(False)
    assert n == 1


@pytest.mark.parametrize("E,I", [(128, 768), (64, 384), (16, 576), (8, 192)])
def test_prefetch_single_layer_vs_oracle(ctx, oracle, prefetch, E, I):
    layer = Layer(ctx, 2048, E, 8, I, layer_id=61 + E + I)
    worst = 0.0
    for index0 in (0, 5):
        hid = hidden_states(ctx, 1, 2048, index0)[0]
        h0 = hid.cpu().numpy()
        gids, gw = run_stack(ctx, [layer], hid)
        worst = max(worst, check_layer(oracle, layer, h0, hid.cpu().numpy(), gids[0], gw[0]))
    print(f"prefetch single layer E={E} I={I}: rel_err {worst:.2e}")
    assert worst <= TOL


@pytest.mark.parametrize("E,I,n", [(128, 768, 12), (16, 384, 9)])
def test_prefetch_stack_equals_layer_calls(ctx, oracle, prefetch, E, I, n):
    """n layers in one call (predictions hit and miss) equal n one-layer calls
    bit for bit; four of the layers are checked against the oracle on the
    GPU's own input of that layer."""
    layers = [Layer(ctx, 2048, E, 8, I, layer_id=70 + i, host=False) for i in range(n)]
    x0 = hidden_states(ctx, 1, 2048, 21)[0]
    full = x0.clone()
    fids, fw = run_stack(ctx, layers, full)
    step = x0.clone()
    worst = 0.0
    for i, layer in enumerate(layers):
        h_in = step.cpu().numpy()
        gids, gw = run_stack(ctx, [layer], step)
        assert (gids[0] == fids[i]).all() and (gw[0] == fw[i]).all(), i
        if i in (0, 1, n // 2, n - 1):
            layer.host_copies()
            worst = max(worst, check_layer(oracle, layer, h_in, step.cpu().numpy(), gids[0], gw[0]))
            del layer.h_pool
    assert torch.equal(full, step)
    print(f"prefetch stack E={E} I={I} x{n}: worst layer rel_err {worst:.2e}")
    assert worst <= TOL


def test_prefetch_matches_per_layer_engine(ctx, prefetch):
    """Against the per-layer launch engine on the same 6 layers: same ids,
    hidden states within the tolerance of each other."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=90 + i, host=False) for i in range(6)]
    x0 = hidden_states(ctx, 1, 2048, 22)[0]
    ctx.set_decode_engine(smoe_amd.DECODE_PREFETCH)
    a = x0.clone()
    aids, _ = run_stack(ctx, layers, a)
    ctx.set_decode_engine(smoe_amd.DECODE_LAUNCHES)
    b = x0.clone()
    bids, _ = run_stack(ctx, layers, b)
    assert (aids == bids).all()
    x = x0.cpu().numpy().astype(np.float64)
    da, db = a.cpu().numpy() - x, b.cpu().numpy() - x
    slack = np.spacing(np.abs(a.cpu().numpy())) + np.spacing(np.abs(b.cpu().numpy()))
    assert rel_err(da, db, slack=slack)[0] <= 6 * 2 * TOL


def test_prefetch_repeated_calls_and_graph_replay(ctx, prefetch):
    """Calls in a row, a shorter call in between, and replays of a captured
    graph with eager calls between them all reproduce the first call."""
    layers = [Layer(ctx, 2048, 128, 8, 384, layer_id=100 + i, host=False) for i in range(5)]
    x0 = hidden_states(ctx, 1, 2048, 23)[0]
    ref = x0.clone()
    rids, _ = run_stack(ctx, layers, ref)
    for _ in range(3):
        buf = x0.clone()
        ids, _ = run_stack(ctx, layers, buf)
        assert torch.equal(buf, ref) and (ids == rids).all()
    tmp = x0.clone()
    run_stack(ctx, layers[:2], tmp)
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
