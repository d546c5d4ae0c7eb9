"""The scale+min 4-bit format (bf16 scale and min per group of 64, the format
the benchmark configurations name; no counterpart in the reference) on the
GPU: its quantizer and pool generator bit-exact against the oracle's, the
one-launch decode layer and the chained stack against the oracle (ids
bit-exact, MoE delta within 1e-3) and fp64 (within 5e-4), the chain equal to
per-layer launches bit for bit, and SMOE_ERR_BITS wherever the format does
not run."""
import ctypes as C

import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import Layer, hidden_states, moe_block_f64, moe_delta_err, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
QM = smoe_amd.QUANT_Q4_SCALE_MIN


def test_quantize_min_bit_exact(ctx, oracle):
    """16M generated weights plus edge groups (constant, exact ties, far from
    zero, tiny and large spans) against orc_quantize_q4_min."""
    w = oracle.gen_normal(1 << 24, 3, 777, 0.02)
    g = w.reshape(-1, 64)
    g[0] = 0.375                                    # constant group: s = 1, codes 0
    g[1] = 0
    g[1, 1] = 15.0
    g[1, 2:9] = [0.5, 1.5, 2.5, 3.5, 6.5, 13.5, 14.5]   # ties on a unit grid
    g[2] += 0.5                                     # far from zero
    g[3] *= 1e-30                                   # tiny span
    g[4] *= 1e6                                     # large span
    dw = torch.from_numpy(w).cuda()
    dp = torch.zeros(w.size // 2, dtype=torch.uint8, device="cuda")
    ds = torch.zeros(w.size // 64, dtype=torch.int16, device="cuda")
    dm = torch.zeros(w.size // 64, dtype=torch.int16, device="cuda")
    ctx.quantize_q4_scale_min(dw.data_ptr(), w.size, 64, dp.data_ptr(), ds.data_ptr(), dm.data_ptr())
    p, s, m = oracle.quantize_q4_min(w)
    assert (ds.cpu().numpy().view(np.uint16) == s).all()
    assert (dm.cpu().numpy().view(np.uint16) == m).all()
    bad = np.nonzero(dp.cpu().numpy() != p)[0]
    assert bad.size == 0, (bad.size, bad[:4])


def test_expert_pool_min_bit_exact(ctx, oracle):
    """The generator's pool in the scale+min format: every matrix of three
    (layer, expert) pairs equals the oracle quantizer applied to the same
    draws, mins right after the scales."""
    D, I = 2048, 768
    shape = smoe_amd.make_shape(D, 4, 2, I, quant=QM)
    off, raw, stride = smoe_amd.blob_layout(D, I, quant=QM)
    assert raw == 3 * (D * I // 2 + D * I // 16)
    pool = torch.zeros(3 * 4 * stride, dtype=torch.uint8, device="cuda")
    ctx.synth_expert_pool(pool.data_ptr(), 5, 3, 4, stride, shape, 42, 0.02)
    host = pool.cpu().numpy()
    ng = D * I // 64
    for (l, e) in ((0, 0), (2, 3), (1, 2)):
        blob = host[(l * 4 + e) * stride:(l * 4 + e) * stride + raw]
        for k in range(3):
            w = oracle.gen_normal(D * I, 42, smoe_amd.expert_stream(5 + l, e, k), 0.02)
            p, s, m = oracle.quantize_q4_min(w)
            so = off[2 * k + 1]
            assert (blob[off[2 * k]:off[2 * k] + p.size] == p).all(), (l, e, k)
            assert (blob[so:so + 2 * ng].view(np.uint16) == s).all()
            assert (blob[so + 2 * ng:so + 4 * ng].view(np.uint16) == m).all()


def test_decode_layer_min_vs_oracle_and_fp64(ctx, oracle):
    """One 30B-shaped layer in the scale+min format through the one-launch
    kernel: ids bit-exact against the oracle's router + top-k, the MoE delta
    within 1e-3 of the oracle and 5e-4 of fp64, for 4 hidden states."""
    layer = Layer(ctx, 2048, 128, 8, 768, layer_id=61, quant=QM)
    worst = w64 = 0.0
    mats = {}
    for index0 in range(4):
        hid = hidden_states(ctx, 1, 2048, 70 + index0)[0]
        h0 = hid.cpu().numpy()
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        w = torch.zeros(8, dtype=torch.float32, device="cuda")
        ctx.profile_enable(True)
        ctx.moe_decode(layer.shape, layer.layer, hid.data_ptr(), 1, ids.data_ptr(), w.data_ptr())
        ctx.synchronize()
        n_layer, _ = ctx.profile_read(smoe_amd.KERNEL_MOE_LAYER)
        ctx.profile_enable(False)
        assert n_layer == 1
        gids, gw = ids.cpu().numpy().view(np.uint32), w.cpu().numpy()
        out, oid, ow, _lg, _nr, yo = layer.oracle_decode(oracle, h0)
        assert (gids == oid).all(), (gids, oid)
        assert np.allclose(gw, ow, rtol=1e-5, atol=1e-7)
        got = hid.cpu().numpy()
        worst = max(worst, moe_delta_err(got, h0, yo, ow)[0], rel_err(got, out)[0])
        ref = moe_block_f64(layer, h0, gids, gw, mats)
        w64 = max(w64, rel_err(got.astype(np.float64) - h0, ref, slack=np.spacing(np.abs(got)))[0])
    print(f"scale+min layer: rel_err {worst:.2e} (oracle), {w64:.2e} (fp64)")
    assert worst <= TOL
    assert w64 <= 5e-4


def test_chain_min_equals_layer_calls(ctx, oracle):
    """Six 30B-shaped scale+min layers in one chained launch equal six
    one-launch layer calls bit for bit; the first and last layer agree with
    the oracle on the GPU's own input."""
    layers = [Layer(ctx, 2048, 128, 8, 768, layer_id=80 + i, host=False, quant=QM) for i in range(6)]
    x0 = hidden_states(ctx, 1, 2048, 90)[0]
    a = x0.clone()
    ia = torch.zeros((6, 8), dtype=torch.int32, device="cuda")
    wa = torch.zeros((6, 8), dtype=torch.float32, device="cuda")
    ctx.set_decode_engine(smoe_amd.DECODE_CHAIN)
    ctx.profile_enable(True)
    ctx.moe_decode_stack(layers[0].shape, [l.layer for l in layers], a.data_ptr(), ia.data_ptr(), wa.data_ptr())
    ctx.synchronize()
    n, _ = ctx.profile_read(smoe_amd.KERNEL_CHAIN)
    ctx.profile_enable(False)
    assert n == 1
    b = x0.clone()
    worst = 0.0
    for i, l in enumerate(layers):
        h_in = b.cpu().numpy()
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        w = torch.zeros(8, dtype=torch.float32, device="cuda")
        ctx.moe_decode(l.shape, l.layer, b.data_ptr(), 1, ids.data_ptr(), w.data_ptr())
        ctx.synchronize()
        assert torch.equal(ids, ia[i]) and torch.equal(w, wa[i]), i
        if i in (0, 5):
            l.host_copies()
            out, oid, ow, _lg, _nr, yo = l.oracle_decode(oracle, h_in)
            assert (ids.cpu().numpy().view(np.uint32) == oid).all()
            got = b.cpu().numpy()
            worst = max(worst, moe_delta_err(got, h_in, yo, ow)[0])
            del l.h_pool
    assert torch.equal(a, b)
    assert worst <= TOL


def test_min_format_rejected_where_it_does_not_run(ctx):
    """SMOE_ERR_BITS for the scale+min format on prefill, on two tokens, under
    SMOE_DECODE_SPLIT, on a 235B-shaped (d_model 4096) layer, and on the
    allocation-free decode of such a layer; an unknown format is refused by
    every shape check."""
    lay = Layer(ctx, 2048, 128, 8, 768, layer_id=95, host=False, quant=QM)
    h = hidden_states(ctx, 2, 2048, 99)
    with pytest.raises(smoe_amd.SmoeError) as e:
        ctx.moe_prefill(lay.shape, lay.layer, h.data_ptr(), 2)
    assert e.value.code == smoe_amd.SMOE_ERR_BITS
    with pytest.raises(smoe_amd.SmoeError) as e:
        ctx.moe_decode(lay.shape, lay.layer, h.data_ptr(), 2)
    assert e.value.code == smoe_amd.SMOE_ERR_BITS
    ctx.set_decode_engine(smoe_amd.DECODE_SPLIT)
    try:
        with pytest.raises(smoe_amd.SmoeError) as e:
            ctx.moe_decode(lay.shape, lay.layer, h.data_ptr(), 1)
        assert e.value.code == smoe_amd.SMOE_ERR_BITS
    finally:
        ctx.set_decode_engine(smoe_amd.DECODE_CHAIN)
    wide = Layer(ctx, 4096, 16, 8, 1536, layer_id=96, host=False, quant=QM)
    h4 = hidden_states(ctx, 1, 4096, 98)[0]
    with pytest.raises(smoe_amd.SmoeError) as e:
        ctx.moe_decode(wide.shape, wide.layer, h4.data_ptr(), 1)
    assert e.value.code == smoe_amd.SMOE_ERR_BITS
    stream = torch.cuda.current_stream().cuda_stream
    rc = smoe_amd.lib().smoe_hip_moe_decode_static(C.byref(wide.shape), C.byref(wide.layer), h4.data_ptr(),
                                                   None, None, None, stream)
    assert rc == smoe_amd.SMOE_ERR_BITS
    bad = smoe_amd.make_shape(2048, 128, 8, 768, quant=7)
    with pytest.raises(smoe_amd.SmoeError) as e:
        ctx.moe_decode(bad, lay.layer, h.data_ptr(), 1)
    assert e.value.code == smoe_amd.SMOE_ERR_BITS
    torch.cuda.synchronize()
