"""Expert FFN oracle (kernels.metal:61-63, 308-365, 672-769 restated) pinned by
fp64 brute force on tiny shapes, the dequant identity, zero input and scale
linearity.  The reference's FFN exists only as Metal shaders, so no reference
vectors exist for it."""
import numpy as np


def tiny_expert(oracle, D, I, seed):
    off, nb = oracle.blob_layout(D, I)
    blob = np.zeros(nb, np.uint8)
    for m, (p, s) in enumerate(((off[0], off[1]), (off[2], off[3]), (off[4], off[5]))):
        w = oracle.gen_normal(D * I, seed, m, 0.02)
        packed, scales = oracle.quantize_q4(w)
        blob[p:p + packed.size] = packed
        blob[s:s + scales.size * 2] = scales.view(np.uint8)
    return blob, off


def dense(oracle, blob, off, D, I, m):
    n = D * I
    packed = blob[off[2 * m]:off[2 * m] + n // 2]
    scales = blob[off[2 * m + 1]:off[2 * m + 1] + n // 64 * 2].view(np.uint16)
    return oracle.dequant_q4(packed, scales, n).astype(np.float64)


def test_ffn_matches_fp64_brute_force(oracle):
    rng = np.random.default_rng(0)
    for D, I in ((64, 64), (128, 64), (64, 192)):
        blob, off = tiny_expert(oracle, D, I, 100 + D + I)
        x = rng.standard_normal(D).astype(np.float32)
        h, y = oracle.expert_ffn(blob, off, D, I, x)
        G = dense(oracle, blob, off, D, I, 0).reshape(I, D)
        U = dense(oracle, blob, off, D, I, 1).reshape(I, D)
        Dn = dense(oracle, blob, off, D, I, 2).reshape(D, I)
        g, u = G @ x, U @ x
        hh = g / (1 + np.exp(-g)) * u
        yy = Dn @ hh
        assert np.allclose(h, hh, rtol=1e-5, atol=1e-7)
        assert np.allclose(y, yy, rtol=1e-4, atol=1e-6)


def test_ffn_zero_input(oracle):
    blob, off = tiny_expert(oracle, 64, 128, 1)
    h, y = oracle.expert_ffn(blob, off, 64, 128, np.zeros(64, np.float32))
    assert (h == 0).all() and (y == 0).all()


def test_dequant_identity(oracle):
    """sum_j w_j x_j == s * (sum_j c_j x_j / 7.5 - sum_j x_j) per group."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal(64) * 0.05).astype(np.float32)
    packed, scales = oracle.quantize_q4(w)
    x = rng.standard_normal(64)
    deq = oracle.dequant_q4(packed, scales, 64).astype(np.float64)
    c = np.empty(64)
    c[0::2], c[1::2] = packed & 0xF, packed >> 4
    s = float(scales.view(np.float16)[0])
    assert np.isclose(deq @ x, s * ((c @ x) / 7.5 - x.sum()), rtol=1e-6)


def test_down_linear_in_down_scale(oracle):
    """Doubling every down scale doubles y and leaves h unchanged."""
    D, I = 64, 128
    blob, off = tiny_expert(oracle, D, I, 4)
    x = np.random.default_rng(4).standard_normal(D).astype(np.float32)
    h1, y1 = oracle.expert_ffn(blob, off, D, I, x)
    b2 = blob.copy()
    sc = b2[off[5]:off[5] + D * I // 64 * 2].view(np.uint16)
    sc[:] = (sc.view(np.float16) * np.float16(2)).view(np.uint16)
    h2, y2 = oracle.expert_ffn(b2, off, D, I, x)
    assert (h1 == h2).all()
    assert np.allclose(y2, 2 * y1, rtol=1e-6, atol=1e-9)


def test_decode_layer_composition(oracle):
    """The decode block equals its parts: norm -> router -> top_k -> renorm ->
    sum_r w_r FFN_r -> residual (decode.cpp:236-509)."""
    D, I, E, K = 64, 64, 16, 4
    off, nb = oracle.blob_layout(D, I)
    pool = np.zeros(E * nb, np.uint8)
    for e in range(E):
        blob, _ = tiny_expert(oracle, D, I, 1000 + e)
        pool[e * nb:(e + 1) * nb] = blob
    norm_w = np.full(D, 0x3F80, np.uint16)
    router = oracle.gen_bf16(E * D, 5, 6, 0.3)
    hidden = oracle.gen_normal(D, 5, 7)
    shape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=1)
    out, ids, w, logits, normed, yo = oracle.moe_decode_layer(shape, norm_w, router, pool, nb, off, hidden)
    nr = oracle.rms_norm_bf16(hidden, norm_w)
    assert (nr == normed).all()
    lg = oracle.matvec_bf16(router.reshape(E, D), nr)
    assert (lg == logits).all()
    rid, rw = oracle.top_k(lg, K, True)
    assert (rid == ids).all() and (rw == w).all()
    acc = np.zeros(D, np.float32)
    for r in range(K):
        e = int(ids[r])
        _, y = oracle.expert_ffn(pool[e * nb:(e + 1) * nb], off, D, I, nr)
        assert (y == yo[r]).all()
        acc = (acc + np.float32(w[r]) * y).astype(np.float32)
    assert np.allclose(out, hidden + acc, rtol=0, atol=1e-6)
    assert abs(float(w.sum()) - 1) < 1e-6
