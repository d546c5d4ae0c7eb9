"""Dense-trunk kernels against the CPU oracle: the grouped bf16 GEMV
(smoe_hip_matvec_*, common.hpp:293-306) and the single-token decode attention
layer (smoe_hip_attention_layer / smoe_metal_attention_layer,
decode.cpp:150-229) at Qwen3 head layouts, with and without QK norm, over a
ring that wraps.  GEMV: every output within 4 sqrt(n) eps sum_j |w_j x_j| of
the exact (float64) dot product -- the bound fp32 summation in any order
meets -- and the oracle's sequential sum meets it too.  Attention output and
the KV rows written for the token within 1e-3 (rel_err metric, 1 % floor);
every other ring row untouched."""
import numpy as np
import pytest
import torch

import smoe_amd
from gpu_helpers import SEED, rel_err

pytestmark = pytest.mark.gpu
TOL_ATTN = 1e-3
EPS32 = np.finfo(np.float32).eps


def dot_bound_err(got, W, x):
    """max_r |got_r - (W x)_r| / (4 sqrt(n) eps sum_j |W_rj x_j|)  (<= 1 passes)."""
    W64, x64 = W.astype(np.float64), x.astype(np.float64)
    exact = W64 @ x64
    scale = 4 * np.sqrt(W.shape[1]) * EPS32 * (np.abs(W64) @ np.abs(x64)) + 1e-30
    return float(np.max(np.abs(got.astype(np.float64) - exact) / scale))


def bf16_weights(ctx, rows, cols, stream, std=0.02):
    w = torch.empty(rows * cols, dtype=torch.int16, device="cuda")
    ctx.synth_bf16(w.data_ptr(), rows * cols, SEED, stream, std)
    return w


def randn(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g, dtype=torch.float32)


@pytest.mark.parametrize("rows,cols", [(4096, 2048), (512, 2048), (2048, 4096), (1000, 136), (20000, 2048)])
def test_gemv_vs_oracle(ctx, oracle, rows, cols):
    w = bf16_weights(ctx, rows, cols, 7000 + rows)
    x = randn(cols, rows).cuda()
    y = torch.zeros(rows, dtype=torch.float32, device="cuda")
    ctx.matvec_bf16(w.data_ptr(), x.data_ptr(), y.data_ptr(), rows, cols)
    ctx.synchronize()
    ref = np.zeros(rows, np.float32)
    wh, xh = w.cpu().numpy().view(np.uint16), x.cpu().numpy()
    oracle.lib().orc_matvec_bf16(ref, wh, xh, rows, cols)
    Wf = (wh.astype(np.uint32) << 16).view(np.float32).reshape(rows, cols)
    e_gpu, e_orc = dot_bound_err(y.cpu().numpy(), Wf, xh), dot_bound_err(ref, Wf, xh)
    e, _ = rel_err(y.cpu().numpy(), ref)
    print(f"gemv {rows}x{cols}: error/bound gpu {e_gpu:.2f} oracle {e_orc:.2f}; rel_err vs oracle {e:.2e}")
    assert e_gpu <= 1.0 and e_orc <= 1.0


def test_gemv_group_vs_separate(ctx):
    shapes = [(4096, 2048), (512, 2048), (512, 2048), (2048, 4096)]
    ws = [bf16_weights(ctx, r, c, 7100 + i) for i, (r, c) in enumerate(shapes)]
    xs = [randn(c, 20 + i).cuda() for i, (r, c) in enumerate(shapes)]
    ys = [torch.zeros(r, dtype=torch.float32, device="cuda") for r, c in shapes]
    ctx.matvec_group_bf16([w.data_ptr() for w in ws], [x.data_ptr() for x in xs], [y.data_ptr() for y in ys],
                          [r for r, c in shapes], [c for r, c in shapes])
    for (r, c), w, x, y in zip(shapes, ws, xs, ys):
        one = torch.zeros(r, dtype=torch.float32, device="cuda")
        ctx.matvec_bf16(w.data_ptr(), x.data_ptr(), one.data_ptr(), r, c)
        ctx.synchronize()
        assert torch.equal(one, y)


def test_gemv_rejects_bad_layouts(ctx):
    w = bf16_weights(ctx, 16, 64, 7200)
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    y = torch.zeros(16, dtype=torch.float32, device="cuda")
    for rows, cols, xp in ((16, 60, x.data_ptr()), (16, 64, x.data_ptr() + 4), (0, 64, x.data_ptr())):
        with pytest.raises(smoe_amd.SmoeError):
            ctx.matvec_bf16(w.data_ptr(), xp, y.data_ptr(), rows, cols)


def rope(pos, head_dim, theta=1e6):
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    ang = pos * inv
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("d_model,nh,nkv,hd,ctx_len,slot,valid,qk", [
    (2048, 32, 4, 128, 4096, 0, 1, True),        # Qwen3-30B-A3B layout, first token
    (2048, 32, 4, 128, 4096, 299, 300, True),
    (2048, 32, 4, 128, 4096, 17, 4096, True),    # full ring, wrapped
    (2048, 32, 4, 128, 1024, 700, 513, False),   # no QK norm
    (4096, 64, 4, 128, 2048, 1999, 1000, True),  # Qwen3-235B-A22B layout (16 query heads per KV head)
    (512, 8, 8, 64, 64, 5, 40, True),            # MHA, head_dim 64
    (1024, 16, 16, 64, 2048, 100, 1500, True),   # MHA, several context splits
    (2048, 8, 2, 256, 512, 300, 400, True),      # head_dim 256
    (1280, 10, 2, 128, 1024, 50, 800, False),    # 5 query heads per KV head (padded group)
])
def test_attention_layer_vs_oracle(ctx, oracle, d_model, nh, nkv, hd, ctx_len, slot, valid, qk):
    run_attention_case(ctx, oracle, d_model, nh, nkv, hd, ctx_len, slot, valid, qk)


def test_attention_scratch_reuse(ctx, oracle):
    """Shapes that grow, shrink and grow the context's split scratch in turn:
    the split counters must survive every reuse."""
    for case in ((4096, 64, 4, 128, 2048, 1999, 1000, True), (2048, 8, 2, 256, 512, 300, 400, True),
                 (512, 8, 8, 64, 1024, 5, 900, False), (4096, 64, 4, 128, 2048, 7, 2048, True)):
        run_attention_case(ctx, oracle, *case)


def run_attention_case(ctx, oracle, d_model, nh, nkv, hd, ctx_len, slot, valid, qk):
    print(f"case attention d={d_model} heads={nh}/{nkv}x{hd} ctx={ctx_len} slot={slot} valid={valid}", flush=True)
    q_dim, kv_dim = nh * hd, nkv * hd
    W = {n: bf16_weights(ctx, r, c, 7300 + i) for i, (n, (r, c)) in enumerate(
        dict(q=(q_dim, d_model), k=(kv_dim, d_model), v=(kv_dim, d_model), o=(d_model, q_dim)).items())}
    qn = bf16_weights(ctx, 1, hd, 7310, std=0.3) if qk else None
    kn = bf16_weights(ctx, 1, hd, 7311, std=0.3) if qk else None
    if qk:   # norm weights around 1
        for t in (qn, kn):
            t.copy_(((t.view(torch.bfloat16).float() + 1.0).to(torch.bfloat16)).view(torch.int16))
    cos, sin = rope(12345 + slot, hd)
    x = randn(d_model, 1).cuda()
    kc = randn(ctx_len * kv_dim, 2).reshape(ctx_len, kv_dim).cuda()
    vc = randn(ctx_len * kv_dim, 3).reshape(ctx_len, kv_dim).cuda()
    kc0, vc0 = kc.cpu().numpy(), vc.cpu().numpy()
    dev = dict(cos=torch.from_numpy(cos).cuda(), sin=torch.from_numpy(sin).cuda(),
               q=torch.zeros(q_dim, device="cuda"), k=torch.zeros(kv_dim, device="cuda"),
               v=torch.zeros(kv_dim, device="cuda"), att=torch.zeros(q_dim, device="cuda"),
               o=torch.zeros(d_model, device="cuda"))
    a = smoe_amd.SmoeAttnLayerArgs()
    a.w_q, a.w_k, a.w_v, a.w_o = (W[n].data_ptr() for n in "qkvo")
    a.q_norm_w = qn.data_ptr() if qk else None
    a.k_norm_w = kn.data_ptr() if qk else None
    a.rope_cos, a.rope_sin, a.normed_in = dev["cos"].data_ptr(), dev["sin"].data_ptr(), x.data_ptr()
    a.qbuf, a.kbuf, a.vbuf = dev["q"].data_ptr(), dev["k"].data_ptr(), dev["v"].data_ptr()
    a.k_cache, a.v_cache, a.attn_out, a.o_out = kc.data_ptr(), vc.data_ptr(), dev["att"].data_ptr(), dev["o"].data_ptr()
    a.d_model, a.q_dim, a.kv_dim, a.head_dim, a.num_heads, a.num_kv_heads = d_model, q_dim, kv_dim, hd, nh, nkv
    a.slot, a.valid, a.attn_ctx, a.attn_scale = slot, valid, ctx_len, 1.0 / np.sqrt(hd)
    ctx.attention_layer(a)
    ctx.synchronize()
    h16 = lambda t: t.cpu().numpy().view(np.uint16)
    o_ref, kc_ref, vc_ref = oracle.attention_layer(h16(W["q"]), h16(W["k"]), h16(W["v"]), h16(W["o"]),
                                                   h16(qn) if qk else None, h16(kn) if qk else None, cos, sin,
                                                   x.cpu().numpy(), kc0, vc0, hd, nh, nkv, slot, valid,
                                                   1.0 / np.sqrt(hd))
    got_k, got_v = kc.cpu().numpy(), vc.cpu().numpy()
    e_k, _ = rel_err(got_k[slot], kc_ref[slot])
    e_v, _ = rel_err(got_v[slot], vc_ref[slot])
    others = np.arange(ctx_len) != slot
    assert np.array_equal(got_k[others], kc0[others]) and np.array_equal(got_v[others], vc0[others])
    e_o, _ = rel_err(dev["o"].cpu().numpy(), o_ref)
    print(f"attention {nh}/{nkv}x{hd} valid={valid}: rel_err o={e_o:.2e} k={e_k:.2e} v={e_v:.2e}")
    assert e_k <= TOL_ATTN and e_v <= TOL_ATTN and e_o <= TOL_ATTN
    # the synchronous reference-surface entry point gives the same result
    kc.copy_(torch.from_numpy(kc0))
    vc.copy_(torch.from_numpy(vc0))
    o_async = dev["o"].clone()
    dev["o"].zero_()
    ctx.attention_layer(a, sync=True)
    assert torch.equal(dev["o"], o_async)


def test_attention_decode_steps(ctx, oracle):
    """Five consecutive tokens through one ring (the split counters and the KV
    append carry from call to call), each output against the oracle run on
    the oracle's own ring."""
    d_model, nh, nkv, hd, ctx_len = 2048, 32, 4, 128, 1024
    q_dim, kv_dim = nh * hd, nkv * hd
    W = {n: bf16_weights(ctx, r, c, 7400 + i) for i, (n, (r, c)) in enumerate(
        dict(q=(q_dim, d_model), k=(kv_dim, d_model), v=(kv_dim, d_model), o=(d_model, q_dim)).items())}
    kc = randn(ctx_len * kv_dim, 12).reshape(ctx_len, kv_dim).cuda()
    vc = randn(ctx_len * kv_dim, 13).reshape(ctx_len, kv_dim).cuda()
    kc_ref, vc_ref = kc.cpu().numpy(), vc.cpu().numpy()
    h16 = lambda t: t.cpu().numpy().view(np.uint16)
    dev = dict(q=torch.zeros(q_dim, device="cuda"), k=torch.zeros(kv_dim, device="cuda"),
               v=torch.zeros(kv_dim, device="cuda"), att=torch.zeros(q_dim, device="cuda"),
               o=torch.zeros(d_model, device="cuda"))
    for step, (slot, valid) in enumerate(((1020, 700), (1021, 701), (1022, 702), (1023, 703), (0, 704))):
        print(f"case decode step {step} slot={slot} valid={valid}", flush=True)
        cos, sin = rope(5000 + step, hd)
        x = randn(d_model, 40 + step).cuda()
        cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        a = smoe_amd.SmoeAttnLayerArgs()
        a.w_q, a.w_k, a.w_v, a.w_o = (W[n].data_ptr() for n in "qkvo")
        a.q_norm_w = a.k_norm_w = None
        a.rope_cos, a.rope_sin, a.normed_in = cos_d.data_ptr(), sin_d.data_ptr(), x.data_ptr()
        a.qbuf, a.kbuf, a.vbuf = dev["q"].data_ptr(), dev["k"].data_ptr(), dev["v"].data_ptr()
        a.k_cache, a.v_cache, a.attn_out, a.o_out = kc.data_ptr(), vc.data_ptr(), dev["att"].data_ptr(), dev["o"].data_ptr()
        a.d_model, a.q_dim, a.kv_dim, a.head_dim, a.num_heads, a.num_kv_heads = d_model, q_dim, kv_dim, hd, nh, nkv
        a.slot, a.valid, a.attn_ctx, a.attn_scale = slot, valid, ctx_len, 1.0 / np.sqrt(hd)
        ctx.attention_layer(a)
        ctx.synchronize()
        o_ref, kc_ref, vc_ref = oracle.attention_layer(h16(W["q"]), h16(W["k"]), h16(W["v"]), h16(W["o"]), None, None,
                                                       cos, sin, x.cpu().numpy(), kc_ref, vc_ref, hd, nh, nkv, slot,
                                                       valid, 1.0 / np.sqrt(hd))
        e_o, _ = rel_err(dev["o"].cpu().numpy(), o_ref)
        e_k, _ = rel_err(kc.cpu().numpy()[slot], kc_ref[slot])
        print(f"  rel_err o={e_o:.2e} k={e_k:.2e}")
        assert e_o <= TOL_ATTN and e_k <= TOL_ATTN
        # keep the two rings identical so the next step compares like with like
        kc.copy_(torch.from_numpy(kc_ref))
        vc.copy_(torch.from_numpy(vc_ref))
