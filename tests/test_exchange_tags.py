"""Tags of the one-launch decode kernels' exchange words, walked across their
32-bit wrap on the host through smoe_hip_exchange_tags (the same
__host__ __device__ functions k_moe_layer and k_moe_chain call).

Every decode step must be exact however long the engine runs
(decode.cpp:121-123 runs the layer loop once per token, without end), so:
no tag is 0 (every exchange word's value at allocation), no two consecutive
layers share a tag -- inside a launch, and from the last layer of one launch
to the first of the next -- and the abort value of a launch is never 0 (the
abort word's value at allocation).  The expected sequence is derived here
from the arithmetic alone: tags count 1, 2, ..., 2^32 - 1, 1, 2, ...
"""
import pytest

import smoe_amd

M = 2**32 - 1


def expected_tags(epoch, n):
    e = epoch % M
    return [((e + l) % M) + 1 for l in range(n)]


@pytest.mark.parametrize("n_layers", [1, 2, 47, 48, 94])
def test_tags_across_the_wrap(n_layers):
    """Consecutive launches started just below the wrap: every tag in 1..M,
    consecutive layers (across launch boundaries too) differ, the sequence
    counts up by one modulo M, and the abort value is the launch's first tag."""
    epoch = M - 3 * n_layers - 5
    prev_tag = None
    seen = []
    for _ in range(12):
        tags, abort_val, nxt = smoe_amd.exchange_tags(epoch, n_layers)
        assert tags == expected_tags(epoch, n_layers)
        assert abort_val == tags[0] and abort_val != 0
        assert all(1 <= t <= M for t in tags)
        for t in tags:
            if prev_tag is not None:
                assert t != prev_tag
                assert t == prev_tag % M + 1, (prev_tag, t)
            prev_tag = t
        seen.extend(tags)
        assert nxt == (epoch + n_layers) % M
        epoch = nxt
    # the walk crossed the wrap
    assert M in seen and 1 in seen


@pytest.mark.parametrize("epoch", [0, 1, M - 1, M, 2**32 - 2])
@pytest.mark.parametrize("n_layers", [1, 47, 48, 94])
def test_tags_at_edges(epoch, n_layers):
    """Epoch words at the edges of the range, including the one value (2^32 - 1)
    that no launch stores: it reads as 0."""
    tags, abort_val, nxt = smoe_amd.exchange_tags(epoch, n_layers)
    assert tags == expected_tags(epoch, n_layers)
    assert 0 not in tags and abort_val != 0
    assert len(set(tags)) == n_layers
    assert nxt == (epoch % M + n_layers) % M
    # the next launch starts with a tag the last layer did not use
    nxt_tags, _, _ = smoe_amd.exchange_tags(nxt, 1)
    assert nxt_tags[0] != tags[-1]


def test_single_layer_kernel_sequence():
    """k_moe_layer advances the epoch by one per launch: its tags walk 1, 2,
    ..., M, 1 with no repeat, and its stored epoch is the tag it just used
    (except at M, where it stores 0)."""
    epoch = M - 3
    got = []
    for _ in range(6):
        tags, _, nxt = smoe_amd.exchange_tags(epoch, 1)
        got.append(tags[0])
        assert nxt == tags[0] % M
        epoch = nxt
    assert got == [M - 2, M - 1, M, 1, 2, 3]


def test_long_run_has_no_zero_tag():
    """A run of 2^32 / 48 + 2 launches of 48 layers (the 30B stack) modelled
    with the closed form: the launch whose layers straddle the wrap has tags
    ... M - 1, M, 1, 2 ..., and its abort value is not 0."""
    n = 48
    k = M // n + 1                                 # first launch that reaches the wrap
    epoch = (k - 1) * n % M
    tags, abort_val, nxt = smoe_amd.exchange_tags(epoch, n)
    assert tags == expected_tags(epoch, n)
    assert 0 not in tags and abort_val != 0
    i = tags.index(M)
    assert tags[i + 1] == 1 if i + 1 < n else True
