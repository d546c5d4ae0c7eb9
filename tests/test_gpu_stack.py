"""The whole-stack decode step (smoe_hip_moe_decode_stack: the decode.cpp:121
layer loop) against the CPU oracle of decode.cpp:236-509, layer by layer, for
both engines: the chained launch (one per step) and per-layer calls.  Top-k ids must be bit-exact; the MoE
delta and the post-residual hidden state within 1e-3 per element (rel_err
metric).  A multi-layer call must equal the same layers run one call at a time
bit for bit (each layer's input is the previous layer's fp32 output either
way), across repeated calls and graph replays."""
import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import Layer, hidden_states, moe_delta_err, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
ENGINES = [smoe_amd.DECODE_LAUNCHES, smoe_amd.DECODE_CHAIN]


@pytest.fixture(params=ENGINES, ids=["launches", "chain"])
def engine(ctx, request):
    ctx.set_decode_engine(request.param)
    yield request.param
    ctx.set_decode_engine(smoe_amd.DECODE_CHAIN)


def run_stack(ctx, layers, hid):
    """One stack call over `layers` on hid [D] (in place); returns ids, w [L x K]."""
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
    print(f"stack layer rel_err delta={e1:.2e} hidden={e2:.2e}")
    return max(e1, e2)


@pytest.mark.parametrize("D,E,K,I,norm", [
    (2048, 128, 8, 768, True),     # Qwen3-30B-A3B
    (64, 8, 2, 64, True),
    (128, 16, 4, 192, True),
    (256, 64, 8, 128, True),
    (512, 200, 6, 256, True),
    (512, 128, 16, 256, False),    # two ranks per XCD, no renormalisation
    (1024, 512, 8, 1024, True),
])
def test_stack_single_layer_vs_oracle(ctx, oracle, engine, D, E, K, I, norm):
    layer = Layer(ctx, D, E, K, I, layer_id=D + E + K, norm_topk=norm)
    for index0 in (0, 5):
        hid = hidden_states(ctx, 1, D, index0)[0]
        h0 = hid.cpu().numpy()
        gids, gw = run_stack(ctx, [layer], hid)
        assert check_layer(oracle, layer, h0, hid.cpu().numpy(), gids[0], gw[0]) <= TOL


def test_stack_235b_shape_per_layer_path(ctx, oracle, engine):
    """Config 3 shape through smoe_hip_moe_decode_stack, two layers, each
    checked against the oracle on the GPU's own input of that layer, and the
    stack call bit-identical to one-layer calls."""
    layers = [Layer(ctx, 4096, 128, 8, 1536, layer_id=7 + i) for i in range(2)]
    x0 = hidden_states(ctx, 1, 4096, 3)[0]
    full = x0.clone()
    fids, fw = run_stack(ctx, layers, full)
    step = x0.clone()
    for i, layer in enumerate(layers):
        h_in = step.cpu().numpy()
        gids, gw = run_stack(ctx, [layer], step)
        assert (gids[0] == fids[i]).all()
        assert check_layer(oracle, layer, h_in, step.cpu().numpy(), gids[0], gw[0]) <= TOL
    assert torch.equal(full, step)


def test_stack_multi_layer_teacher_forced(ctx, oracle, engine):
    """Four 30B-shaped layers in one call: bit-identical to four one-layer
    calls, and every layer within the tolerance of the oracle applied to the
    GPU's own input of that layer."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=20 + i) for i in range(4)]
    x0 = hidden_states(ctx, 1, 2048, 11)[0]
    full = x0.clone()
    fids, fw = run_stack(ctx, layers, full)
    step = x0.clone()
    worst = 0.0
    for i, layer in enumerate(layers):
        h_in = step.cpu().numpy()
        gids, gw = run_stack(ctx, [layer], step)
        assert (gids[0] == fids[i]).all() and (gw[0] == fw[i]).all()
        worst = max(worst, check_layer(oracle, layer, h_in, step.cpu().numpy(), gids[0], gw[0]))
    assert torch.equal(full, step)
    assert worst <= TOL


def test_stack_matches_per_layer_decode(ctx, engine):
    """The stack call and per-layer smoe_hip_moe_decode calls implement one
    MoE block: same ids, hidden states within the tolerance of each other
    (bit-identical: both engines run the one-launch layer's schedule)."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=30 + i, host=False) for i in range(3)]
    x0 = hidden_states(ctx, 1, 2048, 12)[0]
    a = x0.clone()
    fids, _ = run_stack(ctx, layers, a)
    b = x0.clone()
    ids = torch.zeros((3, 8), dtype=torch.int32, device="cuda")
    for i, l in enumerate(layers):
        ctx.moe_decode(l.shape, l.layer, b.data_ptr(), 1, ids[i].data_ptr())
    ctx.synchronize()
    assert (ids.cpu().numpy().view(np.uint32) == fids).all()
    assert torch.equal(a, b)
    x = x0.cpu().numpy().astype(np.float64)
    da, db = a.cpu().numpy() - x, b.cpu().numpy() - x
    slack = np.spacing(np.abs(a.cpu().numpy())) + np.spacing(np.abs(b.cpu().numpy()))
    assert rel_err(da, db, slack=slack)[0] <= 3 * 2 * TOL


def test_stack_repeated_calls_and_graph_replay(ctx, engine):
    """Calls in a row (the exchange flags advance per call and are never
    re-armed) and replays of a captured graph with eager work in between all
    reproduce the first call exactly."""
    layers = [Layer(ctx, 1024, 128, 8, 512, layer_id=40 + i, host=False) for i in range(3)]
    x0 = hidden_states(ctx, 1, 1024, 13)[0]
    ref = x0.clone()
    rids, _ = run_stack(ctx, layers, ref)
    for _ in range(3):
        buf = x0.clone()
        ids, _ = run_stack(ctx, layers, buf)
        assert torch.equal(buf, ref) and (ids == rids).all()
    # a shorter call in between uses a different layer table
    tmp = x0.clone()
    run_stack(ctx, layers[:1], tmp)
    buf = x0.clone()
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], buf.data_ptr())   # table upload, eager
    ctx.synchronize()
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
