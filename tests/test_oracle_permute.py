"""Token-by-expert permute (prefill.cpp:38-68, :315-332): the whole-prompt
stable counting sort against brute force, and its equivalence with the
reference's per-chunk union_add lists concatenated in chunk order."""
import numpy as np


def routing(rng, T, K, E, skew=False):
    ids = np.zeros((T, K), np.uint32)
    p = None
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        p /= p.sum()
    for t in range(T):
        ids[t] = rng.choice(E, K, replace=False, p=p)
    return ids, rng.random((T, K)).astype(np.float32)


def test_permute_vs_brute_force(oracle):
    rng = np.random.default_rng(1)
    for T, K, E, skew in ((1, 8, 128, False), (64, 8, 128, True), (512, 8, 128, False), (37, 4, 16, True)):
        ids, w = routing(rng, T, K, E, skew)
        off, tok, wo, uni = oracle.permute(ids, w, E)
        pairs = sorted(((int(ids[t, r]), t, r) for t in range(T) for r in range(K)))
        assert [p[1] for p in pairs] == list(tok)
        assert [w[p[1], p[2]] for p in pairs] == list(wo)
        counts = np.bincount(ids.ravel(), minlength=E)
        assert (np.diff(off) == counts).all() and off[0] == 0
        first = {}
        for i, e in enumerate(ids.ravel()):
            first.setdefault(int(e), i)
        assert list(uni) == sorted(first, key=first.get)


def test_permute_equals_chunked_union_lists(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(2)
    T, K, E, CH = 512, 8, 128, 64
    ids, w = routing(rng, T, K, E, True)
    off, tok, wo, _ = oracle.permute(ids, w, E)
    per_expert = {e: [] for e in range(E)}
    for c0 in range(0, T, CH):
        L.orc_union_reset()
        for i in range(min(CH, T - c0)):
            for r in range(K):
                L.orc_union_add(int(ids[c0 + i, r]), i, float(w[c0 + i, r]))
        for u in range(L.orc_union_size()):
            e = L.orc_union_id(u)
            per_expert[e] += [c0 + L.orc_union_tok(e, t) for t in range(L.orc_union_count(e))]
    for e in range(E):
        assert list(tok[off[e]:off[e + 1]]) == per_expert[e]
