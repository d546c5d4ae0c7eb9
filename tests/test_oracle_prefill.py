"""The prefill oracle (orc_moe_prefill_layer, prefill.cpp:308-453) equals its
pinned parts composed in the reference's order, and the oracle's threaded mode
is bit-identical to its single-threaded loops.

Composition, per chunk of 64 tokens (prefill.hpp:33):
  rms_norm_bf16 of every row (prefill.cpp:272-275), then per token router
  matvec_bf16 + top_k with norm_topk (:319-332) feeding union_add (:38-68);
  per union entry in first-appearance order, per listed token, the expert
  FFN, and routed_out[tok] += w * y (:380-385); finally hidden += routed_out
  (:446-451).
The union order comes from the compiled reference's union_add where
oracle/_ref is built, else from orc_union_add (pinned against the same
reference in test_oracle_golden.py)."""
import numpy as np
import pytest

from test_oracle_ffn import tiny_expert


def make_pool(oracle, D, I, E, seed0):
    off, nb = oracle.blob_layout(D, I)
    pool = np.zeros(E * nb, np.uint8)
    for e in range(E):
        blob, _ = tiny_expert(oracle, D, I, seed0 + e)
        pool[e * nb:(e + 1) * nb] = blob
    return pool, off, nb


def union_order(oracle, chunk_ids, chunk_w):
    """[(expert, [(tok, w), ...]), ...] in union order for one chunk."""
    if oracle.ref_available():
        R = oracle.ref()
        R.ref_union_reset()
        add, size, uid = R.ref_union_add, R.ref_union_size, R.ref_union_id
        cnt, tok, wt = R.ref_union_count, R.ref_union_tok, R.ref_union_w
    else:
        L = oracle.lib()
        L.orc_union_reset()
        add, size, uid = L.orc_union_add, L.orc_union_size, L.orc_union_id
        cnt, tok, wt = L.orc_union_count, L.orc_union_tok, L.orc_union_w
    for i in range(chunk_ids.shape[0]):
        for r in range(chunk_ids.shape[1]):
            add(int(chunk_ids[i, r]), i, float(chunk_w[i, r]))
    out = []
    for u in range(size()):
        e = uid(u)
        out.append((e, [(tok(e, t), np.float32(wt(e, t))) for t in range(cnt(e))]))
    return out


@pytest.mark.parametrize("T,norm_topk", [(70, 1), (64, 0), (5, 1)])
def test_prefill_layer_composition(oracle, T, norm_topk):
    D, I, E, K = 128, 64, 16, 4
    pool, off, nb = make_pool(oracle, D, I, E, 3000)
    norm_w = oracle.gen_bf16(D, 8, 1, 0.2) + np.uint16(0)      # non-trivial norm weights
    norm_w = np.where(norm_w == 0, np.uint16(0x3F80), norm_w).astype(np.uint16)
    router = oracle.gen_bf16(E * D, 8, 2, 0.3)
    hidden = np.stack([oracle.gen_normal(D, 8, 100 + t) for t in range(T)]).astype(np.float32)
    shape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=norm_topk)
    out, ids, w = oracle.moe_prefill_layer(shape, norm_w, router, pool, nb, off, hidden)

    want = hidden.copy()
    for c0 in range(0, T, 64):
        B = min(64, T - c0)
        normed = np.stack([oracle.rms_norm_bf16(hidden[c0 + i], norm_w) for i in range(B)])
        cid = np.zeros((B, K), np.uint32)
        cw = np.zeros((B, K), np.float32)
        for i in range(B):
            lg = oracle.matvec_bf16(router.reshape(E, D), normed[i])
            cid[i], cw[i] = oracle.top_k(lg, K, bool(norm_topk))
        assert (ids[c0:c0 + B] == cid).all()
        assert (w[c0:c0 + B] == cw).all()
        routed = np.zeros((B, D), np.float32)
        for e, toks in union_order(oracle, cid, cw):
            for t, wt in toks:
                _, y = oracle.expert_ffn(pool[e * nb:(e + 1) * nb], off, D, I, normed[t])
                routed[t] = (routed[t] + wt * y).astype(np.float32)
        want[c0:c0 + B] = (want[c0:c0 + B] + routed).astype(np.float32)
    assert (out == want).all(), float(np.max(np.abs(out - want)))


def test_prefill_union_order_is_not_rank_order(oracle):
    """The composition above is only a check if some token's experts are
    summed in an order other than its rank order: make sure the fixture
    exercises that (a token whose rank-0 expert first appeared after its
    rank-1 expert in the chunk)."""
    D, E, K = 128, 16, 4
    router = oracle.gen_bf16(E * D, 8, 2, 0.3)
    norm_w = np.full(D, 0x3F80, np.uint16)
    ids = []
    for t in range(70):
        x = oracle.rms_norm_bf16(oracle.gen_normal(D, 8, 100 + t), norm_w)
        ids.append(oracle.top_k(oracle.matvec_bf16(router.reshape(E, D), x), K, True)[0])
    first = {}
    for t, row in enumerate(ids[:64]):
        for e in row:
            first.setdefault(int(e), (t, list(row).index(e)))
    swapped = any(first[int(row[0])] > first[int(row[1])] for row in ids[:64])
    assert swapped


@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_threads_bit_identical(oracle, kind):
    D, I, E, K = 256, 128, 16, 4
    pool, off, nb = make_pool(oracle, D, I, E, 4000)
    norm_w = np.full(D, 0x3F80, np.uint16)
    router = oracle.gen_bf16(E * D, 9, 2, 0.3)
    shape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=1)
    if kind == "decode":
        h = oracle.gen_normal(D, 9, 3)
        run = lambda: oracle.moe_decode_layer(shape, norm_w, router, pool, nb, off, h)
    else:
        h = np.stack([oracle.gen_normal(D, 9, 10 + t) for t in range(80)]).astype(np.float32)
        run = lambda: oracle.moe_prefill_layer(shape, norm_w, router, pool, nb, off, h)
    with oracle.threads(1):
        a = run()
    with oracle.threads(4):
        b = run()
    for x, y in zip(a, b):
        assert np.array_equal(np.asarray(x), np.asarray(y))
