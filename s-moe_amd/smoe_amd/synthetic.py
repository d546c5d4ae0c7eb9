"""Synthetic inputs of the batched-decode workload (64 tokens, Zipf-skewed
expert popularity) shared by bench.py and the GPU tests.

The reference router is a bias-free bf16 matvec (common.hpp:293-306), so the
skew is built into the weights: router rows N(0, 0.02) plus b_e * u with
b_e = -s * ln(rank_e + 1) / 8 (rank = a seeded permutation of the experts),
and hidden states carry a fixed component of length 8 along the unit vector
u.  Logits then differ by about -s * ln(rank + 1), so popularity falls off as
(rank + 1)^-s.  This is a generator choice of this build, not reference
behaviour.
"""
from __future__ import annotations

ZIPF_SEED = 20261201
ZIPF_MAGNITUDE = 8.0     # |x . u| of every hidden state (of a norm ~sqrt(D))


def zipf_direction(D: int, seed: int = ZIPF_SEED):
    """The unit vector u (float32, on cuda:0)."""
    import torch
    u = torch.randn(D, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    return (u / u.norm()).float().cuda()


def zipf_bias_router(router, u, D: int, E: int, layer: int, s_exp: float, seed: int = ZIPF_SEED) -> None:
    """Add b_e * u to every row e of a bf16 router [E x D] (int16 storage on
    the device), in float64, rounded once to bf16."""
    import torch
    g = torch.Generator().manual_seed(seed + layer)
    rank = torch.randperm(E, generator=g).double()
    b = -s_exp * torch.log(rank + 1.0) / 8.0
    w = router.view(torch.bfloat16).float().view(E, D).double().cpu()
    w = w + b[:, None] * u.double().cpu()[None, :]
    router.copy_(w.float().to(torch.bfloat16).view(torch.int16).view(-1).cuda())


def zipf_hidden(h, u) -> None:
    """h [T x D] += ZIPF_MAGNITUDE * u (in place)."""
    h += ZIPF_MAGNITUDE * u[None, :]
