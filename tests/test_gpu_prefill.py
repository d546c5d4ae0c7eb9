"""GPU parity of the prefill path (prefill.cpp:308-453) against the CPU oracle:
the token-by-expert permute bit-exact (orc_permute, prefill.cpp:38-68), the
router top-k ids bit-exact, the hidden update within 1e-3 (relative error per
element with a floor of 1% of the delta's RMS)."""
import numpy as np
import pytest
import torch

from gpu_helpers import Layer, hidden_states, moe_block_f64, moe_delta_f64_batch, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def gpu_permute(ctx, ids, w, E):
    T, K = ids.shape
    d_ids = torch.from_numpy(ids.astype(np.int32)).cuda()
    d_w = torch.from_numpy(w.astype(np.float32)).cuda()
    offs = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
    tok = torch.full((T * K,), -1, dtype=torch.int32, device="cuda")
    wo = torch.zeros(T * K, dtype=torch.float32, device="cuda")
    uni = torch.full((E,), -1, dtype=torch.int32, device="cuda")
    nu = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.permute(d_ids.data_ptr(), d_w.data_ptr(), T, K, E, offs.data_ptr(), tok.data_ptr(), wo.data_ptr(),
                uni.data_ptr(), nu.data_ptr())
    ctx.synchronize()
    n = int(nu.item())
    return (offs.cpu().numpy().view(np.uint32), tok.cpu().numpy().view(np.uint32), wo.cpu().numpy(),
            uni.cpu().numpy().view(np.uint32)[:n])


@pytest.mark.parametrize("T,K,E,kind", [
    (512, 8, 128, "random"), (1, 8, 128, "random"), (37, 4, 16, "random"), (64, 8, 128, "one_expert"),
    (200, 6, 7, "random"), (736, 8, 128, "zipf"), (60, 16, 512, "random"),
])
def test_permute_bit_exact(ctx, oracle, T, K, E, kind):
    rng = np.random.default_rng(T * 7 + K)
    if kind == "one_expert":
        ids = np.full((T, K), 5, np.uint32)
    elif kind == "zipf":
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        ids = rng.choice(E, size=(T, K), p=p / p.sum()).astype(np.uint32)
    else:
        ids = np.stack([rng.choice(E, size=K, replace=K > E) for _ in range(T)]).astype(np.uint32)
    w = rng.random((T, K), dtype=np.float32)
    go, gt, gw, gu = gpu_permute(ctx, ids, w, E)
    ro, rt, rw, ru = oracle.permute(ids, w, E)
    assert (go == ro).all()
    assert (gt == rt).all()
    assert (gw == rw).all()
    assert (gu == ru).all()


def test_permute_rejects_bad_ids(ctx):
    ids = np.array([[1, 2], [3, 9]], np.uint32)     # 9 >= E
    w = np.ones((2, 2), np.float32)
    d_ids = torch.from_numpy(ids.astype(np.int32)).cuda()
    d_w = torch.from_numpy(w).cuda()
    offs = torch.zeros(9, dtype=torch.int32, device="cuda")
    ctx.permute(d_ids.data_ptr(), d_w.data_ptr(), 2, 2, 8, offs.data_ptr(), 0, 0, 0, 0)
    import smoe_amd
    with pytest.raises(smoe_amd.SmoeError):
        ctx.synchronize()
    ctx.synchronize()    # the flag is reported once, then cleared


def run_prefill(ctx, layer, T, index0=0, perm=False, h=None):
    h = hidden_states(ctx, T, layer.D, index0=index0) if h is None else h
    h0 = h.cpu().numpy()
    ids = torch.zeros((T, layer.K), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, layer.K), dtype=torch.float32, device="cuda")
    extra = {}
    if perm:
        offs = torch.zeros(layer.E + 1, dtype=torch.int32, device="cuda")
        tok = torch.zeros(T * layer.K, dtype=torch.int32, device="cuda")
        uni = torch.zeros(layer.E, dtype=torch.int32, device="cuda")
        nu = torch.zeros(1, dtype=torch.int32, device="cuda")
        ctx.moe_prefill(layer.shape, layer.layer, h.data_ptr(), T, ids.data_ptr(), w.data_ptr(),
                        offs.data_ptr(), tok.data_ptr(), uni.data_ptr(), nu.data_ptr())
        extra = dict(offs=offs, tok=tok, uni=uni, nu=nu)
    else:
        ctx.moe_prefill(layer.shape, layer.layer, h.data_ptr(), T, ids.data_ptr(), w.data_ptr())
    ctx.synchronize()
    return h0, h.cpu().numpy(), ids.cpu().numpy().view(np.uint32), w.cpu().numpy(), extra


F64_TOL = 5e-4


def check_against_oracle(oracle, layer, h0, got, gids, gw, rows=None, exact=False, credit=False):
    """Worst relative error of the GPU's MoE delta against the oracle's over
    `rows`, after asserting their ids / weights.

    With exact=True every checked token is also evaluated in fp64 (same ids
    and weights), and the GPU delta must lie within F64_TOL of the fp64 delta
    (asserted).  The plain distance to the oracle is returned, unless
    credit=True: then the excess of |gpu - oracle| over the oracle's own
    distance from fp64 at that element is returned instead.  That is for
    shapes where the oracle's sequential fp32 sums over 4096 and 1536 terms --
    the reference's batch-kernel arithmetic, kernels.metal:672-769 -- round to
    ~1e-3 of an element near the 1 % floor, more than the kernels do, so the
    plain distance can exceed 1e-3 while the GPU is the closer of the two to
    the exact value."""
    rows = np.arange(h0.shape[0]) if rows is None else rows
    # (threaded oracle: bit-identical to its single-threaded loops)
    with oracle.threads(oracle.usable_cores()):
        ref, rids, rw = oracle.moe_prefill_layer(layer.oracle_shape(), layer.h_norm, layer.h_router,
                                                 layer.h_pool, layer.stride, layer.off, h0[rows])
    assert (gids[rows] == rids).all(), np.argwhere(gids[rows] != rids)[:5]
    assert np.allclose(gw[rows], rw, rtol=1e-5, atol=1e-7)
    # MoE delta of every token; the residual add is rounded once on each side
    d_ref = ref.astype(np.float64) - h0[rows]
    d_got = got[rows].astype(np.float64) - h0[rows]
    slack = np.spacing(np.abs(got[rows])) + np.spacing(np.abs(ref))
    worst = 0.0
    for i in range(len(rows)):
        e, _ = rel_err(d_got[i], d_ref[i], slack=slack[i])
        worst = max(worst, e)
    print(f"prefill rel_err (delta) {worst:.2e} over {len(rows)} tokens")
    if not exact:
        return worst
    x64 = moe_delta_f64_batch(layer, h0[rows], gids[rows], gw[rows])
    w64 = w_orc = w_cred = 0.0
    for i in range(len(rows)):
        sl = np.spacing(np.abs(got[rows[i]])).astype(np.float64)
        w64 = max(w64, rel_err(d_got[i], x64[i], slack=sl)[0])
        w_orc = max(w_orc, rel_err(d_ref[i], x64[i], slack=np.spacing(np.abs(ref[i])).astype(np.float64))[0])
        w_cred = max(w_cred, rel_err(d_got[i], d_ref[i], slack=slack[i] + np.abs(d_ref[i] - x64[i]))[0])
    print(f"prefill vs fp64: gpu {w64:.2e}, oracle {w_orc:.2e}; gpu vs oracle {worst:.2e} plain, "
          f"{w_cred:.2e} beyond the oracle's own rounding")
    assert w64 <= F64_TOL
    return w_cred if credit else worst


def test_prefill_tiny_shapes(ctx, oracle):
    # (the E=4 case gives every expert about 100 pairs: two passes of the
    # grouped GEMM, the second one partial)
    for (D, E, K, I, T) in ((128, 16, 4, 128, 70), (256, 64, 8, 192, 33), (512, 200, 6, 256, 9),
                            (256, 4, 2, 128, 200)):
        layer = Layer(ctx, D, E, K, I, layer_id=100 + D)
        h0, got, gids, gw, _ = run_prefill(ctx, layer, T)
        assert check_against_oracle(oracle, layer, h0, got, gids, gw) <= TOL


def test_prefill_30b_64_tokens(ctx, oracle):
    """Qwen3-30B-A3B-shaped layer, one oracle chunk of 64 tokens, with the
    permute outputs of the same pass checked bit-exactly."""
    layer = Layer(ctx, 2048, 128, 8, 768, layer_id=3)
    h0, got, gids, gw, ex = run_prefill(ctx, layer, 64, index0=500, perm=True)
    assert check_against_oracle(oracle, layer, h0, got, gids, gw) <= TOL
    ro, rt, _, ru = oracle.permute(gids, gw, 128)
    assert (ex["offs"].cpu().numpy().view(np.uint32) == ro).all()
    assert (ex["tok"].cpu().numpy().view(np.uint32) == rt).all()
    n = int(ex["nu"].item())
    assert (ex["uni"].cpu().numpy().view(np.uint32)[:n] == ru).all()


def test_prefill_30b_512_tokens(ctx, oracle):
    """Config 4: 512 tokens through one 30B layer.  Every token's ids are
    checked against the oracle's router + top-k, and every token's hidden
    update against the oracle's whole layer."""
    layer = Layer(ctx, 2048, 128, 8, 768, layer_id=4)
    T = 512
    h0, got, gids, gw, _ = run_prefill(ctx, layer, T, index0=1000)
    for t in range(T):
        x = oracle.rms_norm_bf16(h0[t], layer.h_norm)
        logits = oracle.matvec_bf16(layer.h_router.reshape(layer.E, layer.D), x)
        rid, rw = oracle.top_k(logits, layer.K, True)
        assert (gids[t] == rid).all(), t
        assert np.allclose(gw[t], rw, rtol=1e-5, atol=1e-7)
    assert check_against_oracle(oracle, layer, h0, got, gids, gw) <= TOL


def test_prefill_235b_shape(ctx, oracle):
    layer = Layer(ctx, 4096, 128, 8, 1536, layer_id=9)
    h0, got, gids, gw, _ = run_prefill(ctx, layer, 16, index0=77)
    assert check_against_oracle(oracle, layer, h0, got, gids, gw) <= TOL


def test_prefill_235b_512_tokens(ctx, oracle):
    """512 tokens through one 235B-shaped layer (D=4096, I=1536): about 32
    pairs per expert, so the grouped GEMM runs its 32- and 48-pair pass widths
    over 64 groups.  Every token's ids exact; the hidden update on 64 tokens
    spread over the batch (tokens are independent inside the block) within
    5e-4 of an fp64 evaluation and within 1e-3 of the oracle beyond the
    oracle's own rounding (check_against_oracle, exact=True, credit=True: the
    oracle, which restates the reference's token-batch kernels with one
    sequential fp32 sum per row, is itself up to 1.7e-3 from fp64 on these 64
    tokens, and the plain GPU-oracle distance follows it to 1.6e-3, while the
    GPU stays within 1.5e-4 of fp64)."""
    layer = Layer(ctx, 4096, 128, 8, 1536, layer_id=13)
    T = 512
    h0, got, gids, gw, _ = run_prefill(ctx, layer, T, index0=2000)
    for t in range(T):
        x = oracle.rms_norm_bf16(h0[t], layer.h_norm)
        logits = oracle.matvec_bf16(layer.h_router.reshape(layer.E, layer.D), x)
        rid, rw = oracle.top_k(logits, layer.K, True)
        assert (gids[t] == rid).all(), t
        assert np.allclose(gw[t], rw, rtol=1e-5, atol=1e-7)
    rows = np.linspace(0, T - 1, 64).astype(int)
    assert check_against_oracle(oracle, layer, h0, got, gids, gw, rows=rows, exact=True, credit=True) <= TOL


def test_batched_235b_zipf_64_tokens(ctx, oracle):
    """Config 5: 64 concurrent tokens through one 235B-shaped layer (D=4096,
    E=128, k=8, I=1536) with the Zipf s=1.1 router of bench.py's batched
    workload (the same generator, seed and layer 0).  The skew puts nearly
    every token on the most popular experts, so the grouped GEMMs run their
    64-pair pass at k_dim 4096 and 1536 beside experts with 0-2 pairs (the
    reference's token-batch FFN plus its per-token fallback,
    prefill.cpp:339-417, metal_bridge.mm:544-634).  All 64 tokens: ids
    bit-exact, hidden update within 5e-4 of an fp64 evaluation and within
    1e-3 of the oracle (check_against_oracle, exact=True)."""
    from smoe_amd import synthetic
    D, E, K, I, T = 4096, 128, 8, 1536, 64
    layer = Layer(ctx, D, E, K, I, layer_id=0, host=False)
    u = synthetic.zipf_direction(D)
    synthetic.zipf_bias_router(layer.router, u, D, E, 0, 1.1)
    layer.host_copies()
    h = hidden_states(ctx, T, D, index0=0)
    synthetic.zipf_hidden(h, u)
    h0, got, gids, gw, _ = run_prefill(ctx, layer, T, h=h)
    counts = np.bincount(gids.ravel().astype(np.int64), minlength=E)
    print(f"zipf: {int((counts > 0).sum())} experts touched, busiest {int(counts.max())} pairs, "
          f"{int(((counts > 0) & (counts <= 2)).sum())} with 1-2 pairs")
    assert counts.max() >= 49            # the 64-wide pass of the grouped GEMM runs
    assert ((counts > 0) & (counts <= 2)).sum() >= 8
    assert check_against_oracle(oracle, layer, h0, got, gids, gw, exact=True) <= TOL


def test_prefill_235b_against_fp64(ctx):
    """The grouped path against an fp64 evaluation of the same layer (same
    ids and weights), tighter than the oracle bound: the fp32 oracle itself
    sits up to ~9e-4 from fp64 here (sequential sums over 4096 and 1536
    terms), the kernels ~1.4e-4."""
    layer = Layer(ctx, 4096, 128, 8, 1536, layer_id=9)
    T = 6
    h0, got, gids, gw, _ = run_prefill(ctx, layer, T, index0=77)
    mats = {}
    worst = 0.0
    for t in range(T):
        y = moe_block_f64(layer, h0[t], gids[t], gw[t], mats)
        d_got = got[t].astype(np.float64) - h0[t]
        slack = np.spacing(np.abs(got[t])).astype(np.float64)   # the fp32 residual add
        e_t, _ = rel_err(d_got, y, slack=slack)
        worst = max(worst, e_t)
    print(f"prefill 235b vs fp64: {worst:.2e}")
    assert worst <= 5e-4


def test_prefill_multi_pass_and_no_renorm(ctx, oracle):
    """More tokens than one permute pass holds (E=512 lowers the limit), and
    norm_topk off."""
    layer = Layer(ctx, 256, 512, 8, 128, layer_id=11, norm_topk=False)
    T = 300
    h0, got, gids, gw, _ = run_prefill(ctx, layer, T, index0=9)
    assert check_against_oracle(oracle, layer, h0, got, gids, gw) <= TOL


def test_prefill_matches_decode(ctx):
    """The prefill and decode entry points implement one MoE block: on the same
    tokens the ids agree and the hidden states agree within the tolerance."""
    layer = Layer(ctx, 2048, 128, 8, 768, layer_id=5, host=False)
    T = 8
    a = hidden_states(ctx, T, 2048, index0=42)
    x0 = a.cpu().numpy().astype(np.float64)
    b = a.clone()
    ia = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
    ib = torch.zeros_like(ia)
    ctx.moe_prefill(layer.shape, layer.layer, a.data_ptr(), T, ia.data_ptr())
    ctx.moe_decode(layer.shape, layer.layer, b.data_ptr(), T, ib.data_ptr())
    ctx.synchronize()
    assert (ia.cpu() == ib.cpu()).all()
    da = a.cpu().numpy() - x0
    db = b.cpu().numpy() - x0
    slack = np.spacing(np.abs(a.cpu().numpy())) + np.spacing(np.abs(b.cpu().numpy()))
    worst = max(rel_err(da[t], db[t], slack=slack[t])[0] for t in range(T))
    assert worst <= 2 * TOL   # both sides differ from the exact result by up to TOL


def test_route_counters_across_launches(ctx, oracle):
    """Short batches (under 128 tokens) split each token's router rows over 4
    blocks that count themselves on per-token counters kept across launches
    (never reset).  Consecutive calls with changing batch sizes, including
    one of 300 tokens (one block per token, no counters) in between, must keep
    every token's ids exact."""
    layer = Layer(ctx, 2048, 128, 8, 768, layer_id=12)
    for i, T in enumerate((40, 7, 127, 300, 1, 40, 64)):
        h = hidden_states(ctx, T, layer.D, index0=50 + 17 * i)
        h0 = h.cpu().numpy()
        ids = torch.zeros((T, layer.K), dtype=torch.int32, device="cuda")
        w = torch.zeros((T, layer.K), dtype=torch.float32, device="cuda")
        ctx.moe_prefill(layer.shape, layer.layer, h.data_ptr(), T, ids.data_ptr(), w.data_ptr())
        ctx.synchronize()
        gids = ids.cpu().numpy().view(np.uint32)
        gw = w.cpu().numpy()
        for t in range(T):
            x = oracle.rms_norm_bf16(h0[t], layer.h_norm)
            logits = oracle.matvec_bf16(layer.h_router.reshape(layer.E, layer.D), x)
            rid, rw = oracle.top_k(logits, layer.K, True)
            assert (gids[t] == rid).all(), (T, t)
            assert np.allclose(gw[t], rw, rtol=1e-5, atol=1e-7), (T, t)


@pytest.mark.parametrize("D,E,K,I,T", [(4096, 128, 8, 256, 200), (2048, 16, 2, 128, 1100)])
def test_route_block_shapes(ctx, oracle, D, E, K, I, T):
    """Router block shapes beyond the benchmark configurations: one token a
    block at d_model 4096 (128-511 tokens) and four tokens a block (1024 tokens
    and more in one pass, possible where E*k is small), both with the tokens
    normalised by one wave each and handed to the others through LDS.  Every
    token's ids and weights against the oracle's router + top-k; the hidden
    update of 32 tokens spread over the batch against an fp64 evaluation and
    the oracle (check_against_oracle, exact=True, credit=True: with 32 of the
    tokens at d_model 4096 the oracle's own fp32 rounding reaches 1.3e-3 of an
    element near the floor, above the plain 1e-3 bound, while the kernels stay
    within 1.1e-4 of fp64)."""
    layer = Layer(ctx, D, E, K, I, layer_id=300 + D // 64 + T)
    h0, got, gids, gw, _ = run_prefill(ctx, layer, T, index0=3000)
    for t in range(T):
        x = oracle.rms_norm_bf16(h0[t], layer.h_norm)
        logits = oracle.matvec_bf16(layer.h_router.reshape(layer.E, layer.D), x)
        rid, rw = oracle.top_k(logits, layer.K, True)
        assert (gids[t] == rid).all(), t
        assert np.allclose(gw[t], rw, rtol=1e-5, atol=1e-7), t
    rows = np.linspace(0, T - 1, 32).astype(int)
    assert check_against_oracle(oracle, layer, h0, got, gids, gw, rows=rows, exact=True, credit=True) <= TOL
