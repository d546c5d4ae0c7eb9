"""The oracle against the reference's own routines (golden vectors written by
tests/golden/make_golden.py from the compiled reference, plus a live check
against oracle/_ref when it is built).  Bit-exact: these are the reference's
scalar CPU loops restated, same operations in the same order."""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_topk_golden(oracle, gold):
    n, k, norm = gold["topk_n"], gold["topk_k"], gold["topk_norm"]
    so = np.concatenate([[0], np.cumsum(n)]).astype(np.int64)
    ko = np.concatenate([[0], np.cumsum(k)]).astype(np.int64)
    for i in range(n.size):
        s = gold["topk_scores"][so[i]:so[i + 1]]
        ids, w = oracle.top_k(s, int(k[i]), bool(norm[i]))
        cnt = int(gold["topk_count"][i])
        assert ids.size == cnt
        assert (ids == gold["topk_ids"][ko[i]:ko[i] + cnt]).all(), i
        assert (bits(w) == bits(gold["topk_w"][ko[i]:ko[i] + cnt])).all(), i


def test_topk_swap_counterexample(oracle):
    # p = (0.5, 0.5, 0.9): round 0 takes e2 and swaps it with e0, so round 1
    # finds e1 first -- "ties go to the lower index" would give e0
    ids, _ = oracle.top_k(np.log(np.array([0.5, 0.5, 0.9], np.float32)), 2)
    assert list(ids) == [2, 1]


def test_rmsnorm_matvec_axpy_golden(oracle, gold):
    for D in (64, 2048, 4096):
        y = oracle.rms_norm_bf16(gold[f"rms_x_{D}"], gold[f"rms_w_{D}"])
        assert (bits(y) == bits(gold[f"rms_y_{D}"])).all()
    for rows, cols in ((32, 2048), (16, 64), (128, 256)):
        W = gold[f"mv_W_{rows}x{cols}"].reshape(rows, cols)
        y = oracle.matvec_bf16(W, gold[f"mv_x_{rows}x{cols}"])
        assert (bits(y) == bits(gold[f"mv_y_{rows}x{cols}"])).all()
    y = gold["axpy_y0"].copy()
    oracle.lib().orc_axpy_f32(y, float(gold["axpy_a"][0]), gold["axpy_x"], y.size)
    assert (bits(y) == bits(gold["axpy_y"])).all()


def test_union_add_golden(oracle, gold):
    L = oracle.lib()
    ids, w = gold["union_ids_in"], gold["union_w_in"]
    L.orc_union_reset()
    for t in range(ids.shape[0]):
        for r in range(ids.shape[1]):
            assert L.orc_union_add(int(ids[t, r]), t, float(w[t, r])) == gold["union_fresh"][t, r]
    nu = L.orc_union_size()
    assert nu == gold["union_ids"].size
    assert [L.orc_union_id(u) for u in range(nu)] == list(gold["union_ids"])
    toks, ws = [], []
    for e in gold["union_ids"]:
        c = L.orc_union_count(int(e))
        toks += [L.orc_union_tok(int(e), t) for t in range(c)]
        ws += [L.orc_union_w(int(e), t) for t in range(c)]
    assert toks == list(gold["union_toks"])
    assert (bits(np.array(ws, np.float32)) == bits(gold["union_ws"])).all()


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref",
                                                    "libsmoe_ref.so")), reason="oracle/_ref not built")
def test_topk_live_reference(oracle):
    """Random and tie-heavy inputs against the compiled reference top_k."""
    R = oracle.ref()
    rng = np.random.default_rng(5)
    for trial in range(300):
        n = int(rng.choice([3, 16, 64, 128, 200, 512]))
        k = int(rng.choice([1, 2, 8, 16]))
        s = rng.standard_normal(n).astype(np.float32)
        if trial % 2:
            s = np.round(s * 2) / 2          # heavy ties
        norm = trial % 3 == 0
        ids, w = oracle.top_k(s, k, norm)
        rid = np.zeros(k, np.uint32)
        rw = np.zeros(k, np.float32)
        cnt = R.ref_top_k(s, n, k, rid, rw, int(norm))
        assert cnt == ids.size
        assert (ids == rid[:cnt]).all() and (bits(w) == bits(rw[:cnt])).all()
