"""The scale+min 4-bit format of the benchmark configurations ("4-bit with
group size 64 and a per-group bf16 scale and min"), which the reference does
not have: its oracle quantizer pinned by known answers, and its decode-path
FFN by fp64 brute force.

Format (this build's definition, the same on the GPU): per group of 64
  m = bf16(min w), s = bf16((max w - min w) / 15)  (bf16 1.0 when that is 0),
  code = clamp(rint((w - m) / s), 0, 15) from the rounded s and m, ties to
  even, low nibble = even index; w' = code * s + m.
"""
import numpy as np
import pytest


def bf16(x):
    """round-to-nearest-even to bf16, as float32 (for building expectations)"""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def codes(packed):
    c = np.empty(packed.size * 2, np.int64)
    c[0::2], c[1::2] = packed & 15, packed >> 4
    return c


def test_extremes_map_to_0_and_15(oracle):
    """A group spanning [-1, 2] (both exact in bf16): the minimum gets code 0,
    the maximum 15; the stored min is -1 and the scale bf16(0.2)."""
    w = np.linspace(-1.0, 2.0, 64).astype(np.float32)
    p, s, m = oracle.quantize_q4_min(w)
    c = codes(p)
    assert c[0] == 0 and c[-1] == 15
    assert s.view(np.uint16)[0] == np.float32(bf16(np.float32(3.0) / np.float32(15.0))).view(np.uint32) >> 16
    assert m.view(np.uint16)[0] == np.float32(-1.0).view(np.uint32) >> 16
    assert (np.diff(c) >= 0).all()          # monotone in w


def test_constant_group(oracle):
    """All 64 weights equal (0.375, exact in bf16): scale 1.0, min = the value,
    every code 0, so the group reconstructs exactly."""
    w = np.full(64, 0.375, np.float32)
    p, s, m = oracle.quantize_q4_min(w)
    assert s[0] == 0x3F80 and (codes(p) == 0).all()
    assert (oracle.dequant_q4_min(p, s, m, 64) == w).all()


def test_ties_round_half_even(oracle):
    """min 0 and max 15 make the scale exactly 1: w = k + 0.5 lands on a tie
    and rounds to the even neighbour."""
    w = np.zeros(64, np.float32)
    w[1] = 15.0
    ties = [0.5, 1.5, 2.5, 3.5, 6.5, 13.5, 14.5]
    for i, t in enumerate(ties):
        w[2 + i] = t
    p, s, m = oracle.quantize_q4_min(w)
    assert s[0] == 0x3F80 and m[0] == 0
    c = codes(p)
    assert c[0] == 0 and c[1] == 15
    assert list(c[2:2 + len(ties)]) == [0, 2, 2, 4, 6, 14, 14]


def test_nibble_order(oracle):
    """Even index in the low nibble: codes 0, 15, 1, 14, ... pack as 0xF0, 0xE1, ..."""
    w = np.zeros(64, np.float32)
    w[1] = 15.0
    w[2], w[3] = 1.0, 14.0
    p, _, _ = oracle.quantize_q4_min(w)
    assert p[0] == 0xF0 and p[1] == 0xE1


def test_reconstruction_bound(oracle):
    """Random groups: |w' - w| <= s / 2 plus the small part of a step the
    bf16-rounded min and scale move the grid by, and codes within 0..15."""
    rng = np.random.default_rng(7)
    w = (rng.standard_normal(64 * 500) * 0.02).astype(np.float32)
    w[:64] += 0.5                             # a group far from zero
    p, s, m = oracle.quantize_q4_min(w)
    d = oracle.dequant_q4_min(p, s, m, w.size)
    sf = np.repeat((s.astype(np.uint32) << 16).view(np.float32), 64)
    err = np.abs(d.astype(np.float64) - w)
    assert (err <= 0.55 * sf).all(), float(np.max(err / sf))
    c = codes(p)
    assert c.min() == 0 and c.max() == 15


def dense_min(oracle, blob, off, D, I, k):
    n = D * I
    p = blob[off[2 * k]:off[2 * k] + n // 2]
    s = blob[off[2 * k + 1]:off[2 * k + 1] + n // 32].view(np.uint16)
    m = blob[off[2 * k + 1] + n // 32:off[2 * k + 1] + n // 16].view(np.uint16)
    c = codes(p).astype(np.float64)
    sf = np.repeat((s.astype(np.uint32) << 16).view(np.float32).astype(np.float64), 64)
    mf = np.repeat((m.astype(np.uint32) << 16).view(np.float32).astype(np.float64), 64)
    return (c * sf + mf).reshape((I, D) if k < 2 else (D, I))


def expert_min(oracle, D, I, seed):
    off, nb = oracle.blob_layout(D, I, quant=1)
    blob = np.zeros(nb, np.uint8)
    for k in range(3):
        w = oracle.gen_normal(D * I, seed, k, 0.02)
        p, s, m = oracle.quantize_q4_min(w)
        blob[off[2 * k]:off[2 * k] + p.size] = p
        blob[off[2 * k + 1]:off[2 * k + 1] + 2 * s.size] = s.view(np.uint8)
        blob[off[2 * k + 1] + 2 * s.size:off[2 * k + 1] + 4 * s.size] = m.view(np.uint8)
    return blob, off


def rel_floor(got, ref):
    ref = np.asarray(ref, np.float64)
    tau = 1e-2 * np.sqrt(np.mean(ref ** 2))
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref) / np.maximum(np.abs(ref), tau)))


@pytest.mark.parametrize("D,I", [(64, 64), (1088, 64), (64, 1088), (2048, 768)])
def test_ffn_min_against_fp64(oracle, D, I):
    """The decode-path FFN of the scale+min format (the lanes and chunks of
    kernels.metal:159-365 with the chunk epilogue s * A + m * X) within 2e-4
    of an fp64 evaluation of the same dequantised weights; the per-weight
    dequant of the oracle agrees with the fp64 matrix."""
    blob, off = expert_min(oracle, D, I, 900 + D + I)
    x = oracle.gen_normal(D, 91, D)
    x = (x / np.sqrt(np.mean(x.astype(np.float64) ** 2))).astype(np.float32)
    G, U, Dn = (dense_min(oracle, blob, off, D, I, k) for k in range(3))
    n = D * I
    pw = blob[off[0]:off[0] + n // 2]
    sw = blob[off[1]:off[1] + n // 32].view(np.uint16)
    mw = blob[off[1] + n // 32:off[1] + n // 16].view(np.uint16)
    assert np.array_equal(oracle.dequant_q4_min(pw, sw, mw, min(n, 4096)).astype(np.float64),
                          G.ravel()[:min(n, 4096)])
    g, u = G @ x.astype(np.float64), U @ x.astype(np.float64)
    hh = g / (1 + np.exp(-g)) * u
    h, y = oracle.expert_ffn(blob, off, D, I, x, decode=True, quant=1)
    eh, ey = rel_floor(h, hh), rel_floor(y, Dn @ h.astype(np.float64))
    print(f"D={D} I={I}: scale+min decode form h {eh:.2e} y {ey:.2e}")
    assert eh <= 2e-4 and ey <= 2e-4


def test_decode_layer_min_composition(oracle):
    """The decode block in the scale+min format equals its parts: the router
    and top-k as in SMOE-Q4, then sum_r w_r FFN_r with the format's FFN."""
    D, I, E, K = 64, 64, 16, 4
    off, nb = oracle.blob_layout(D, I, quant=1)
    pool = np.zeros(E * nb, np.uint8)
    for e in range(E):
        blob, _ = expert_min(oracle, D, I, 3000 + e)
        pool[e * nb:(e + 1) * nb] = blob
    norm_w = np.full(D, 0x3F80, np.uint16)
    router = oracle.gen_bf16(E * D, 5, 6, 0.3)
    hidden = oracle.gen_normal(D, 5, 7)
    shape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=1, quant=1)
    out, ids, w, logits, normed, yo = oracle.moe_decode_layer(shape, norm_w, router, pool, nb, off, hidden)
    nr = oracle.rms_norm_bf16(hidden, norm_w)
    rid, rw = oracle.top_k(oracle.matvec_bf16(router.reshape(E, D), nr), K, True)
    assert (rid == ids).all() and (rw == w).all()
    acc = np.zeros(D, np.float32)
    for r in range(K):
        e = int(ids[r])
        _, y = oracle.expert_ffn(pool[e * nb:(e + 1) * nb], off, D, I, nr, decode=True, quant=1)
        assert (y == yo[r]).all()
        acc = (acc + np.float32(w[r]) * y).astype(np.float32)
    assert np.allclose(out, hidden + acc, rtol=0, atol=1e-6)
