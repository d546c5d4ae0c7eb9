"""Expert FFN oracle, both forms the reference computes it in: prefill's
token-batch kernels (kernels.metal:672-769: per-weight dequant, sequential
fp32 sums) and the decode path's qrow_dot2 / qrow_dot (kernels.metal:159-365:
lane-strided 32-code chunks, affine chunk epilogue, simd_sum).  Pinned by fp64
brute force on tiny and on Qwen3-sized shapes, the dequant identity, zero
input and scale linearity.  The reference's FFN exists only as Metal shaders,
so no reference vectors exist for it."""
import numpy as np
import pytest


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


@pytest.mark.parametrize("decode", [False, True])
def test_ffn_matches_fp64_brute_force(oracle, decode):
    rng = np.random.default_rng(0)
    for D, I in ((64, 64), (128, 64), (64, 192), (1088, 64), (64, 1088)):
        blob, off = tiny_expert(oracle, D, I, 100 + D + I)
        x = rng.standard_normal(D).astype(np.float32)
        h, y = oracle.expert_ffn(blob, off, D, I, x, decode=decode)
        G = dense(oracle, blob, off, D, I, 0).reshape(I, D)
        U = dense(oracle, blob, off, D, I, 1).reshape(I, D)
        Dn = dense(oracle, blob, off, D, I, 2).reshape(D, I)
        g, u = G @ x, U @ x
        hh = g / (1 + np.exp(-g)) * u
        yy = Dn @ hh
        assert np.allclose(h, hh, rtol=1e-5, atol=1e-7)
        assert np.allclose(y, yy, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("decode", [False, True])
def test_ffn_zero_input(oracle, decode):
    blob, off = tiny_expert(oracle, 64, 128, 1)
    h, y = oracle.expert_ffn(blob, off, 64, 128, np.zeros(64, np.float32), decode=decode)
    assert (h == 0).all() and (y == 0).all()


def rel_floor(got, ref):
    """max |g - c| / max(|c|, 1% of rms(c)): the parity tests' metric"""
    ref = np.asarray(ref, np.float64)
    tau = 1e-2 * np.sqrt(np.mean(ref ** 2))
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref) / np.maximum(np.abs(ref), tau)))


@pytest.mark.parametrize("D,I", [(2048, 768), (4096, 1536)])
def test_decode_ffn_qwen3_shapes_against_fp64(oracle, D, I):
    """At both Qwen3 shapes the decode form is within 5e-5 of an fp64
    evaluation of the same dequantised weights (its chunked sums are short:
    8 terms per accumulator, at most 4 chunks per lane, then a 32-lane tree).
    A chunk dropped or counted twice, a lane stride or nibble order off, or a
    scale taken from the wrong group moves the result by orders of magnitude
    more.  The per-weight sequential form is also checked, with the looser
    bound its long sums need."""
    blob, off = tiny_expert(oracle, D, I, 7000 + D)
    x = oracle.gen_normal(D, 77, D)
    x = (x / np.sqrt(np.mean(x.astype(np.float64) ** 2))).astype(np.float32)
    G = dense(oracle, blob, off, D, I, 0).reshape(I, D)
    U = dense(oracle, blob, off, D, I, 1).reshape(I, D)
    Dn = dense(oracle, blob, off, D, I, 2).reshape(D, I)
    g, u = G @ x.astype(np.float64), U @ x.astype(np.float64)
    hh = g / (1 + np.exp(-g)) * u
    hd, yd = oracle.expert_ffn(blob, off, D, I, x, decode=True)
    hs, ys = oracle.expert_ffn(blob, off, D, I, x, decode=False)
    e_hd, e_hs = rel_floor(hd, hh), rel_floor(hs, hh)
    # down judged on each form's own h (the fp64 product of the same h)
    e_yd, e_ys = rel_floor(yd, Dn @ hd.astype(np.float64)), rel_floor(ys, Dn @ hs.astype(np.float64))
    print(f"D={D} I={I}: decode form h {e_hd:.2e} y {e_yd:.2e}; sequential form h {e_hs:.2e} y {e_ys:.2e}")
    assert e_hd <= 2e-4 and e_yd <= 2e-4
    assert e_hs <= 2e-3 and e_ys <= 2e-3


def test_decode_ffn_chunk_order(oracle):
    """Which chunk feeds which lane, and the chunk's scale: one nonzero input
    column per chunk position, so each output is one scaled code of a known
    (row, column) -- exact in fp32 -- read back from the decode form."""
    D, I = 256, 64
    blob, off = tiny_expert(oracle, D, I, 31)
    G = dense(oracle, blob, off, D, I, 0).reshape(I, D)
    for col in (0, 1, 7, 8, 31, 32, 63, 64, 200, 255):
        x = np.zeros(D, np.float32)
        x[col] = 1.0
        h, _ = oracle.expert_ffn(blob, off, D, I, x, decode=True)
        # h = silu(g) * u with g = G[:, col]; recover g from a second run with
        # the up scales of the row zeroed is not needed: compare silu(g)*u
        U = dense(oracle, blob, off, D, I, 1).reshape(I, D)
        g, u = G[:, col], U[:, col]
        ref = g / (1 + np.exp(-g)) * u
        assert np.allclose(h, ref, rtol=1e-5, atol=1e-9), col


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


@pytest.mark.parametrize("decode", [False, True])
def test_down_linear_in_down_scale(oracle, decode):
    """Doubling every down scale doubles y exactly (a power of two commutes
    with every rounding) and leaves h unchanged."""
    D, I = 64, 128
    blob, off = tiny_expert(oracle, D, I, 4)
    x = np.random.default_rng(4).standard_normal(D).astype(np.float32)
    h1, y1 = oracle.expert_ffn(blob, off, D, I, x, decode=decode)
    b2 = blob.copy()
    sc = b2[off[5]:off[5] + D * I // 64 * 2].view(np.uint16)
    sc[:] = (sc.view(np.float16) * np.float16(2)).view(np.uint16)
    h2, y2 = oracle.expert_ffn(b2, off, D, I, x, decode=decode)
    assert (h1 == h2).all()
    assert (y2 == 2 * y1).all()


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
        _, y = oracle.expert_ffn(pool[e * nb:(e + 1) * nb], off, D, I, nr, decode=True)
        assert (y == yo[r]).all()
        acc = (acc + np.float32(w[r]) * y).astype(np.float32)
    assert np.allclose(out, hidden + acc, rtol=0, atol=1e-6)
    assert abs(float(w.sum()) - 1) < 1e-6
