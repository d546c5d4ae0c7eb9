"""Known-answer tests for the SMOE-Q4 quantizer / dequant restatement
(scripts/shatter_moe.py:331-387, src/compute/kernels.metal:90-105)."""
import numpy as np


def codes_of(packed, n):
    c = np.empty(packed.size * 2, np.uint8)
    c[0::2] = packed & 0xF
    c[1::2] = packed >> 4
    return c[:n]


def test_absmax_maps_to_extremes(oracle):
    w = np.linspace(-1, 1, 64).astype(np.float32) * 0.37
    packed, scales = oracle.quantize_q4(w)
    c = codes_of(packed, 64)
    assert c[0] == 0 and c[-1] == 15                       # -absmax -> 0, +absmax -> 15
    assert scales[0] == np.float32(0.37).astype(np.float16).view(np.uint16)


def test_zero_group_scale_one_code_eight(oracle):
    packed, scales = oracle.quantize_q4(np.zeros(64, np.float32))
    assert (codes_of(packed, 64) == 8).all()               # rint(7.5) = 8 (half to even)
    assert scales[0] == np.float16(1.0).view(np.uint16)


def test_half_even_ties(oracle):
    # w/absmax*7.5 + 7.5 lands exactly on k + 0.5 for these weights
    absmax = np.float32(7.5)
    vals = np.array([7.5, -7.5, 0.5, 1.5, 2.5, -0.5, -1.5, 3.5], np.float32)
    w = np.zeros(64, np.float32)
    w[:vals.size] = vals
    c = codes_of(oracle.quantize_q4(w)[0], 64)[:vals.size].astype(int)
    expect = [int(np.round(np.float32(v) / absmax * np.float32(7.5) + np.float32(7.5))) for v in vals]
    assert c.tolist() == expect
    assert c.tolist() == [15, 0, 8, 9, 10, 7, 6, 11]     # 8.0, 9.0, 10.0 / 7.0, 6.0 ties -> even


def test_nibble_order_low_is_even(oracle):
    w = np.zeros(64, np.float32)
    w[0], w[1] = -1.0, 1.0                                 # codes 0 and 15
    packed, _ = oracle.quantize_q4(w)
    assert packed[0] == 0xF0


def test_fp16_scale_cast_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)).astype(np.float32)
    v = np.concatenate([v, np.float32([65504, 65519, 65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0, 1e-30])])
    ours = np.array([oracle.lib().orc_f32_to_f16(float(x)) for x in v], np.uint16)
    with np.errstate(over="ignore"):
        assert (ours == v.astype(np.float16).view(np.uint16)).all()
    back = np.array([oracle.lib().orc_f16_to_f32(int(h)) for h in ours], np.float32)
    assert (back.view(np.uint32) == ours.view(np.float16).astype(np.float32).view(np.uint32)).all()


def test_reconstruction_bound_and_numpy_semantics(oracle):
    rng = np.random.default_rng(9)
    w = (rng.standard_normal(64 * 512) * 0.02).astype(np.float32)
    packed, scales = oracle.quantize_q4(w)
    deq = oracle.dequant_q4(packed, scales, w.size)
    g = w.reshape(-1, 64)
    absmax = np.abs(g).max(1, keepdims=True)
    err = np.abs(deq.reshape(-1, 64) - g)
    # half a quantisation step (absmax/15) plus the fp16 rounding of the scale
    bound = absmax / 15 + absmax * 2.0 ** -11 + 1e-12
    assert (err <= bound).all()
    # codes equal numpy's own float32 pipeline, op for op
    q = np.clip(np.round((g / np.where(absmax == 0, 1, absmax)) * np.float32(7.5) + np.float32(7.5)), 0, 15)
    assert (codes_of(packed, w.size) == q.astype(np.uint8).ravel()).all()
    # kernel dequant form: (c - 7.5f) * (1/7.5f) * scale, evaluated left to right
    c = codes_of(packed, w.size).astype(np.float32)
    s = np.repeat(scales.view(np.float16).astype(np.float32), 64)
    ref = (c - np.float32(7.5)) * np.float32(1.0 / 7.5) * s
    assert (deq.view(np.uint32) == ref.astype(np.float32).view(np.uint32)).all()


def test_generator_is_deterministic_and_normal(oracle):
    a = oracle.gen_normal(1 << 18, 1, 2)
    b = oracle.gen_normal(1 << 18, 1, 2)
    c = oracle.gen_normal(1 << 18, 1, 3)
    assert (a.view(np.uint32) == b.view(np.uint32)).all()
    assert not np.allclose(a, c)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    # fourth moment of N(0,1) is 3
    assert abs((a.astype(np.float64) ** 4).mean() - 3) < 0.1
    bf = oracle.gen_bf16(4096, 1, 2, 0.02)
    ref = (oracle.gen_normal(4096, 1, 2) * np.float32(0.02)).astype(np.float32)
    u = ref.view(np.uint32)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert (bf == rne).all()
