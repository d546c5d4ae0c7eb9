"""smoe_hip_compute_top_k against the oracle (= the compiled reference top_k,
pinned by tests/test_oracle_golden.py) on identical score vectors, including
constructed ties and the swap counter-example.  Indices bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def gpu_topk(ctx, scores, k, norm):
    rows, n = scores.shape
    d = torch.from_numpy(np.ascontiguousarray(scores, np.float32)).cuda()
    ids = torch.zeros((rows, k), dtype=torch.int32, device="cuda")
    w = torch.zeros((rows, k), dtype=torch.float32, device="cuda")
    ctx.compute_top_k(d.data_ptr(), rows, n, k, ids.data_ptr(), w.data_ptr(), norm)
    torch.cuda.synchronize()
    return ids.cpu().numpy().view(np.uint32), w.cpu().numpy()


@pytest.mark.parametrize("n,k", [(128, 8), (128, 16), (64, 8), (256, 8), (512, 16), (3, 2), (40, 8)])
def test_topk_random_and_ties(ctx, oracle, n, k):
    rng = np.random.default_rng(n * 31 + k)
    rows = []
    for r in range(64):
        s = rng.standard_normal(n).astype(np.float32)
        if r % 2:
            s = np.round(s * 2) / 2                       # many exact ties
        if r % 7 == 0:
            s[:] = s[0]                                   # all tied
        rows.append(s)
    S = np.stack(rows)
    for norm in (False, True):
        gi, gw = gpu_topk(ctx, S, k, norm)
        for r in range(S.shape[0]):
            oi, ow = oracle.top_k(S[r], k, norm)
            c = oi.size
            assert (gi[r, :c] == oi).all(), (r, gi[r, :c], oi)
            # softmax sums differ in order (parallel vs sequential) and exp implementation
            assert np.allclose(gw[r, :c], ow, rtol=1e-5, atol=1e-9)


def test_swap_counterexample(ctx, oracle):
    S = np.log(np.array([[0.5, 0.5, 0.9]], np.float32))
    gi, _ = gpu_topk(ctx, S, 2, False)
    assert list(gi[0]) == [2, 1]


@pytest.mark.parametrize("n,k", [(128, 8), (100, 6), (64, 8), (8, 8), (5, 8), (128, 1)])
def test_topk_network_edges(ctx, oracle, n, k):
    """Rows aimed at the sorting-network path (n <= 128, k <= 8), which
    proposes ranks from the scores' top 25 bits and must hand every row whose
    probabilities are not strictly ordered to the exact selection.
    One-ulp neighbours are compared with the exact selection on the GPU's own
    probabilities: the same row padded to 129 scores with -inf runs the
    max-extraction path with bit-identical probabilities (the padding adds
    exp(-inf) = 0 to every sum).  Against the oracle only rows whose
    probabilities cannot depend on the exp implementation's last ulp: +0 and
    -0 on top, an exact tie between ranks 8 and 9, -inf and +inf scores."""
    rng = np.random.default_rng(n * 131 + k)
    rows, exact = [], []
    for r in range(48):
        s = rng.standard_normal(n).astype(np.float32)
        order = np.argsort(-s, kind="stable")
        kind = r % 7
        if kind == 1 and n > 1:          # rank i+1 one ulp above rank i (later position larger)
            for i in range(0, min(9, n) - 1, 2):
                a, b = sorted(order[i:i + 2])
                s[b] = np.nextafter(s[a], np.float32(np.inf))
        elif kind == 2 and n > 1:        # earlier position one ulp larger
            for i in range(0, min(9, n) - 1, 2):
                a, b = sorted(order[i:i + 2])
                s[a] = np.nextafter(s[b], np.float32(np.inf))
        elif kind == 3 and n > 1:        # +0 and -0 on top
            s = -np.abs(s) - 1
            s[0] = np.float32(-0.0)
            s[n - 1] = np.float32(0.0)
        elif kind == 4 and n > 8:        # ranks 8 and 9 tie exactly
            s[order[8]] = s[order[7]]
        elif kind == 5:                  # -inf scores
            s[rng.choice(n, size=max(1, n // 4), replace=False)] = -np.inf
        elif kind == 6:                  # one +inf score
            s[rng.integers(n)] = np.inf
        rows.append(s.astype(np.float32))
        exact.append(kind not in (1, 2))
    S = np.stack(rows)
    P = np.full((S.shape[0], 129), -np.inf, np.float32)
    P[:, :n] = S
    for norm in (False, True):
        gi, gw = gpu_topk(ctx, S, k, norm)
        pi, pw = gpu_topk(ctx, P, k, norm)
        for r in range(S.shape[0]):
            if n >= k:
                assert (gi[r] == pi[r]).all(), (r, gi[r], pi[r])
                assert np.array_equal(gw[r], pw[r], equal_nan=True), r
            if not exact[r]:
                continue
            oi, ow = oracle.top_k(S[r], k, norm)
            c = oi.size
            assert (gi[r, :c] == oi).all(), (r, gi[r, :c], oi)
            fin = np.isfinite(ow)
            assert (fin == np.isfinite(gw[r, :c])).all(), r
            assert np.allclose(gw[r, :c][fin], ow[fin], rtol=1e-5, atol=1e-9), r
