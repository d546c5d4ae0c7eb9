"""The attention oracle (orc_attention_layer, decode.cpp:150-229) against what
the mathematics fixes: one attended position returns its V row exactly,
identical keys average the V rows, RoPE at angle 0 is the identity and at 90
degrees maps (a, b) to (-b, a), a normed head with unit weights has unit RMS,
GQA maps query head h to KV head h / (num_heads / num_kv_heads), and only the
`valid` ring rows counted back from `slot` matter.  CPU only."""
import numpy as np

D, HD, NH, NKV = 64, 64, 4, 2
QD, KVD = NH * HD, NKV * HD


def bf16(a):
    a = np.asarray(a, np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)     # truncation: exact values for the test


def setup(rng, ctx=8):
    w = {n: bf16(rng.normal(0, 0.1, (r, c)).astype(np.float32))
         for n, (r, c) in dict(q=(QD, D), k=(KVD, D), v=(KVD, D), o=(D, QD)).items()}
    x = rng.normal(0, 1, D).astype(np.float32)
    kc = rng.normal(0, 1, (ctx, KVD)).astype(np.float32)
    vc = rng.normal(0, 1, (ctx, KVD)).astype(np.float32)
    return w, x, kc, vc


def run(oracle, w, x, kc, vc, slot, valid, cos=None, sin=None, qn=None, kn=None):
    cos = np.ones(HD // 2, np.float32) if cos is None else cos
    sin = np.zeros(HD // 2, np.float32) if sin is None else sin
    return oracle.attention_layer(w["q"], w["k"], w["v"], w["o"], qn, kn, cos, sin, x, kc, vc, HD, NH, NKV, slot,
                                  valid, 1.0 / np.sqrt(HD))


def f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def test_one_position_returns_its_v_row(oracle):
    w, x, kc, vc = setup(np.random.default_rng(1))
    o, kc2, vc2 = run(oracle, w, x, kc, vc, slot=5, valid=1)
    v = np.zeros(KVD, np.float32)
    oracle.lib().orc_matvec_bf16(v, w["v"], x, KVD, D)
    assert np.array_equal(vc2[5], v)
    att = np.concatenate([v[(h // (NH // NKV)) * HD:(h // (NH // NKV) + 1) * HD] for h in range(NH)])
    ref = np.zeros(D, np.float32)
    oracle.lib().orc_matvec_bf16(ref, w["o"], np.ascontiguousarray(att), D, QD)
    assert np.array_equal(o, ref)


def test_identical_keys_average_the_values(oracle):
    rng = np.random.default_rng(2)
    w, x, kc, vc = setup(rng)
    # zero key weights make the current key 0, and every cached key 0 too
    w["k"][:] = 0
    kc[:] = 0
    o, _, vc2 = run(oracle, w, x, kc, vc, slot=3, valid=6)
    rows = [(3 - i) % 8 for i in range(6)]
    mean = vc2[rows].astype(np.float64).mean(0)
    att = np.concatenate([mean[(h // (NH // NKV)) * HD:(h // (NH // NKV) + 1) * HD] for h in range(NH)])
    ref = f32(w["o"]).astype(np.float64) @ att
    assert np.allclose(o, ref, rtol=1e-5, atol=1e-6)


def test_rope_identity_and_quarter_turn(oracle):
    w, x, kc, vc = setup(np.random.default_rng(3))
    k = np.zeros(KVD, np.float32)
    oracle.lib().orc_matvec_bf16(k, w["k"], x, KVD, D)
    _, kc0, _ = run(oracle, w, x, kc, vc, slot=0, valid=1)
    assert np.array_equal(kc0[0], k)
    half = HD // 2
    _, kc1, _ = run(oracle, w, x, kc, vc, slot=1, valid=1, cos=np.zeros(half, np.float32),
                    sin=np.ones(half, np.float32))
    for h in range(NKV):
        a, b = k[h * HD:h * HD + half], k[h * HD + half:(h + 1) * HD]
        assert np.array_equal(kc1[1][h * HD:h * HD + half], -b)
        assert np.array_equal(kc1[1][h * HD + half:(h + 1) * HD], a)


def test_qk_norm_gives_unit_rms(oracle):
    w, x, kc, vc = setup(np.random.default_rng(4))
    ones = np.full(HD, 0x3F80, np.uint16)
    _, kc2, _ = run(oracle, w, x, kc, vc, slot=2, valid=1, qn=ones, kn=ones)
    for h in range(NKV):
        r = kc2[2][h * HD:(h + 1) * HD].astype(np.float64)
        assert abs(np.sqrt(np.mean(r * r)) - 1.0) < 1e-5


def test_only_the_window_counts(oracle):
    w, x, kc, vc = setup(np.random.default_rng(5))
    o1, _, _ = run(oracle, w, x, kc, vc, slot=2, valid=5)          # rows 2, 1, 0, 7, 6
    kc_b, vc_b = kc.copy(), vc.copy()
    kc_b[3:6] += 5.0
    vc_b[3:6] -= 7.0
    o2, _, _ = run(oracle, w, x, kc_b, vc_b, slot=2, valid=5)
    assert np.array_equal(o1, o2)
    vc_c = vc.copy()
    vc_c[6] += 1.0
    o3, _, _ = run(oracle, w, x, kc, vc_c, slot=2, valid=5)
    assert not np.array_equal(o1, o3)
