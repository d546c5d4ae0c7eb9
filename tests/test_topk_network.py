"""CPU model of the sorting network in topk_net (s-moe_amd/csrc/topk.hpp):
64 lanes holding two keys each, one merge per lane bit in the kernel's order
(v_permlane32_swap, v_permlane16_swap, row_ror:8, row_half_mirror, quad_perm
xor 2, quad_perm xor 1).  Every lane must end with the 8 largest keys of the
128, in descending order, for any keys and any number of padding positions.
This pins the network's pairing and merge steps; the GPU tests pin the
kernel itself (tests/test_gpu_topk.py)."""
import numpy as np

L = np.arange(64)


def permlane_swap(v, bit):
    """The two results of v_permlane{32,16}_swap(v, v): each lane gets its own
    value and its partner's (lane ^ 2^bit), in an order that depends on the
    lane."""
    part = v[L ^ (1 << bit)]
    low = (L & (1 << bit)) == 0
    return np.where(low, v, part), np.where(low, part, v)


def dpp(v, kind):
    src = {"ror8": (L & ~15) | ((L + 8) & 15),      # row_ror:8
           "half_mirror": (L & ~7) | (7 - (L & 7)),  # row_half_mirror
           "xor2": L ^ 2, "xor1": L ^ 1}[kind]       # quad_perm
    return v[src]


def cmp_swap(hi, lo):
    return np.maximum(hi, lo), np.minimum(hi, lo)


def network(keys):
    """keys: [128] -> [64 lanes, 8] as the kernel's registers c[0..7]."""
    k0, k1 = keys[L], keys[L + 64]
    a0, a1 = np.maximum(k0, k1), np.minimum(k0, k1)
    # lane bit 5: 2 + 2 keys
    x0, y0 = permlane_swap(a0, 5)
    x1, y1 = permlane_swap(a1, 5)
    c = [np.maximum(x0, y0), None, None, np.minimum(x1, y1)]
    mid1, mid0 = cmp_swap(np.maximum(x1, y1), np.minimum(x0, y0))
    c[1], c[2] = mid1, mid0
    # lane bit 4: 4 + 4 keys, odd-even merge
    x, y = [None] * 4, [None] * 4
    for i in range(4):
        x[i], y[i] = cmp_swap(*permlane_swap(c[i], 4))
    e0, e1, e2, e3 = x[0], y[0], x[2], y[2]
    e1, e2 = cmp_swap(e1, e2)
    o0, o1, o2, o3 = x[1], y[1], x[3], y[3]
    o1, o2 = cmp_swap(o1, o2)
    o0, e1 = cmp_swap(o0, e1)
    o1, e2 = cmp_swap(o1, e2)
    o2, e3 = cmp_swap(o2, e3)
    c = [e0, o0, e1, o1, e2, o2, e3, o3]
    # lane bits 3..0: bitonic top-8 merges
    for kind in ("ror8", "half_mirror", "xor2", "xor1"):
        h = [np.maximum(c[i], dpp(c[7 - i], kind)) for i in range(8)]
        for d in (4, 2, 1):
            for i in range(8):
                if i & d == 0:
                    h[i], h[i + d] = cmp_swap(h[i], h[i + d])
        c = h
    return np.stack(c, axis=1)


def test_network_top8_every_lane():
    rng = np.random.default_rng(7)
    for trial in range(1500):
        n = int(rng.integers(1, 129))
        keys = np.zeros(128, np.uint64)          # padding positions hold key 0
        if trial % 3 == 0:
            keys[:n] = rng.permutation(n) + 1
        else:
            keys[:n] = rng.choice(2 ** 31, size=n, replace=False) + 1
        if trial % 5 == 0:
            keys[:n] = keys[:n][rng.permutation(n)]
        out = network(keys)
        want = np.sort(keys)[::-1][:8]
        assert (out == want[None, :]).all(), (trial, n)


def test_network_keeps_duplicates():
    """Equal keys (the kernel's keys are distinct, but the merges must not
    lose or invent values when they are not)."""
    rng = np.random.default_rng(11)
    for _ in range(300):
        keys = rng.integers(0, 6, size=128).astype(np.uint64)
        out = network(keys)
        assert (out == np.sort(keys)[::-1][:8][None, :]).all()
