"""The prefill layer loop on device (smoe_hip_moe_prefill_stack): equal to
one smoe_hip_moe_prefill call per layer bit for bit, equal to the
reference's chunk order (64-token chunks, prefill.hpp:33) bit for bit since
tokens are independent inside the MoE block, and every layer within 1e-3 of
the CPU oracle of prefill.cpp:308-453 on the GPU's own input of that layer
(teacher-forced; ids bit-exact)."""
import numpy as np
import pytest
import torch

from gpu_helpers import Layer, hidden_states
from test_gpu_prefill import TOL, check_against_oracle

pytestmark = pytest.mark.gpu


def test_prefill_stack_matches_per_layer_calls_chunks_and_oracle(ctx, oracle):
    D, E, K, I, T = 2048, 128, 8, 768, 150
    layers = [Layer(ctx, D, E, K, I, layer_id=80 + i) for i in range(3)]
    x0 = hidden_states(ctx, T, D, index0=300)
    full = x0.clone()
    ids = torch.zeros((3, T, K), dtype=torch.int32, device="cuda")
    ctx.moe_prefill_stack(layers[0].shape, [l.layer for l in layers], full.data_ptr(), T, ids.data_ptr())
    ctx.synchronize()

    # one call per layer, each checked against the oracle on its own input
    step = x0.clone()
    worst = 0.0
    rows = np.linspace(0, T - 1, 12).astype(int)
    for i, l in enumerate(layers):
        h_in = step.cpu().numpy()
        li = torch.zeros((T, K), dtype=torch.int32, device="cuda")
        lw = torch.zeros((T, K), dtype=torch.float32, device="cuda")
        ctx.moe_prefill(l.shape, l.layer, step.data_ptr(), T, li.data_ptr(), lw.data_ptr())
        ctx.synchronize()
        assert torch.equal(li, ids[i])
        worst = max(worst, check_against_oracle(oracle, l, h_in, step.cpu().numpy(),
                                                li.cpu().numpy().view(np.uint32), lw.cpu().numpy(), rows=rows))
    assert torch.equal(full, step)
    assert worst <= TOL

    # the reference's order: the stack over each 64-token chunk
    chunked = x0.clone()
    for t0 in range(0, T, 64):
        n = min(64, T - t0)
        ctx.moe_prefill_stack(layers[0].shape, [l.layer for l in layers], chunked[t0:].data_ptr(), n)
    ctx.synchronize()
    assert torch.equal(chunked, full)
