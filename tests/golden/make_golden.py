"""Write tests/golden/ref_vectors.npz from the reference's own routines.

The routines are compiled from the reference sources by `make -C oracle ref`
(oracle/ref_driver.cpp): top_k (src/scout/scout.cpp:77-123), rms_norm_bf16,
matvec_bf16, axpy_f32 (src/common.hpp:245-256, 293-306, 346-349) and union_add
(src/prefill.cpp:48-68).  Inputs are seeded; the file holds inputs and the
reference's outputs, nothing else.  Run in a container that has the reference
tree:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def topk_cases(rng):
    cases = []
    for n, k in ((128, 8), (128, 16), (64, 8), (512, 8), (256, 16), (4, 8), (16, 16)):
        for norm in (0, 1):
            cases.append((rng.standard_normal(n).astype(np.float32) * 2, k, norm))
    # constructed ties: duplicated logits (equal probabilities)
    for rep in range(6):
        s = rng.standard_normal(128).astype(np.float32)
        top = np.argsort(-s)[:12]
        s[top[rng.permutation(12)[:6]]] = s[top[0]]
        s[rng.integers(0, 128, 8)] = s[top[3]]
        cases.append((s, 8, rep % 2))
    # the swap counter-example: p0 = p1 = 0.5, p2 = 0.9 (unnormalised)
    cases.append((np.log(np.array([0.5, 0.5, 0.9], np.float32)), 2, 0))
    cases.append((np.log(np.array([0.5, 0.5, 0.9], np.float32)), 3, 1))
    cases.append((np.zeros(128, np.float32), 8, 1))                  # all tied
    cases.append((np.full(128, -50.0, np.float32), 16, 0))           # all tied, large negative
    s = np.repeat(rng.standard_normal(16).astype(np.float32), 8)     # 16 values x 8 copies
    cases.append((s, 16, 1))
    return cases


def main():
    if not O.ref_available():
        O.build()
    R = O.ref()
    rng = np.random.default_rng(20261201)
    out = {}
    cases = topk_cases(rng)
    out["topk_n"] = np.array([c[0].size for c in cases], np.uint32)
    out["topk_k"] = np.array([c[1] for c in cases], np.uint32)
    out["topk_norm"] = np.array([c[2] for c in cases], np.uint32)
    out["topk_scores"] = np.concatenate([c[0] for c in cases]).astype(np.float32)
    ids_all, w_all, cnt_all = [], [], []
    for s, k, norm in cases:
        ids = np.zeros(k, np.uint32)
        w = np.zeros(k, np.float32)
        cnt = R.ref_top_k(np.ascontiguousarray(s), s.size, k, ids, w, norm)
        ids_all.append(ids)
        w_all.append(w)
        cnt_all.append(cnt)
    out["topk_count"] = np.array(cnt_all, np.uint32)
    out["topk_ids"] = np.concatenate(ids_all)
    out["topk_w"] = np.concatenate(w_all)

    for D in (64, 2048, 4096):
        x = (rng.standard_normal(D) * 3).astype(np.float32)
        w = O.gen_bf16(D, 7, D, 0.5)
        y = x.copy()
        R.ref_rms_norm_bf16(y, w, D)
        out[f"rms_x_{D}"], out[f"rms_w_{D}"], out[f"rms_y_{D}"] = x, w, y

    for rows, cols in ((32, 2048), (16, 64), (128, 256)):
        W = O.gen_bf16(rows * cols, 11, rows, 0.02)
        x = rng.standard_normal(cols).astype(np.float32)
        y = np.zeros(rows, np.float32)
        R.ref_matvec_bf16(y, W, x, rows, cols)
        out[f"mv_W_{rows}x{cols}"], out[f"mv_x_{rows}x{cols}"], out[f"mv_y_{rows}x{cols}"] = W, x, y

    y0 = rng.standard_normal(2048).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    a = np.float32(0.3717)
    y = y0.copy()
    R.ref_axpy_f32(y, float(a), x, 2048)
    out["axpy_y0"], out["axpy_x"], out["axpy_a"], out["axpy_y"] = y0, x, np.array([a]), y

    # union_add over one 64-token chunk of top-8 routing
    T, K, E = 64, 8, 128
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.uint32)
    ids[:, :3] = rng.integers(0, 12, (T, 3))          # popular experts (dupes removed below)
    for t in range(T):
        seen = []
        for r in range(K):
            e = int(ids[t, r])
            while e in seen:
                e = (e + 1) % E
            ids[t, r] = e
            seen.append(e)
    wts = rng.random((T, K)).astype(np.float32)
    R.ref_union_reset()
    fresh = np.zeros((T, K), np.uint8)
    for t in range(T):
        for r in range(K):
            fresh[t, r] = R.ref_union_add(int(ids[t, r]), t, float(wts[t, r]))
    nu = R.ref_union_size()
    uids = np.array([R.ref_union_id(u) for u in range(nu)], np.uint32)
    counts = np.array([R.ref_union_count(int(e)) for e in uids], np.uint32)
    toks = np.concatenate([[R.ref_union_tok(int(e), t) for t in range(R.ref_union_count(int(e)))]
                           for e in uids]).astype(np.uint32)
    ws = np.concatenate([[R.ref_union_w(int(e), t) for t in range(R.ref_union_count(int(e)))]
                         for e in uids]).astype(np.float32)
    out.update(union_ids_in=ids, union_w_in=wts, union_fresh=fresh, union_ids=uids,
               union_counts=counts, union_toks=toks, union_ws=ws)

    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
