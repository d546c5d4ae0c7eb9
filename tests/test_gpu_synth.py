"""GPU generator and quantizer against the CPU oracle: bit-exact."""
import numpy as np
import pytest
import torch

import smoe_amd

pytestmark = pytest.mark.gpu


def test_normal_and_bf16_bit_exact(ctx, oracle):
    n = 1 << 20
    d = torch.empty(n, dtype=torch.float32, device="cuda")
    ctx.synth_normal(d.data_ptr(), n, 7, 12345, 0.02)
    ref = oracle.gen_normal(n, 7, 12345, 0.02)
    got = d.cpu().numpy()
    assert (got.view(np.uint32) == ref.view(np.uint32)).all()
    b = torch.empty(n, dtype=torch.int16, device="cuda")
    ctx.synth_bf16(b.data_ptr(), n, 7, 999, 0.02)
    assert (b.cpu().numpy().view(np.uint16) == oracle.gen_bf16(n, 7, 999, 0.02)).all()


def test_quantize_bit_exact_with_edge_groups(ctx, oracle):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal(64 * 4096) * 0.02).astype(np.float32)
    g = w.reshape(-1, 64)
    g[0] = 0                                          # zero group -> scale 1, codes 8
    g[1] = np.linspace(-1, 1, 64)                     # +-absmax
    g[2, :8] = [7.5, -7.5, 0.5, 1.5, 2.5, -0.5, -1.5, 3.5]   # exact .5 ties
    g[2, 8:] = 0
    g[3] *= 1e-6                                      # tiny scale (fp16 subnormal range)
    g[4] *= 1e4                                       # large scale
    dw = torch.from_numpy(w).cuda()
    dp = torch.zeros(w.size // 2, dtype=torch.uint8, device="cuda")
    ds = torch.zeros(w.size // 64, dtype=torch.int16, device="cuda")
    ctx.quantize_q4(dw.data_ptr(), w.size, 64, dp.data_ptr(), ds.data_ptr())
    p, s = oracle.quantize_q4(w)
    assert (dp.cpu().numpy() == p).all()
    assert (ds.cpu().numpy().view(np.uint16) == s).all()


def test_quantize_bit_exact_many_groups(ctx, oracle):
    """16M weights: enough for values within an ulp of a rounding boundary of
    w / absmax * 7.5 + 7.5, where fusing the multiply and the add into one
    fma (a single rounding) would change a code."""
    w = oracle.gen_normal(1 << 24, 3, 4242, 0.02)
    dw = torch.from_numpy(w).cuda()
    dp = torch.zeros(w.size // 2, dtype=torch.uint8, device="cuda")
    ds = torch.zeros(w.size // 64, dtype=torch.int16, device="cuda")
    ctx.quantize_q4(dw.data_ptr(), w.size, 64, dp.data_ptr(), ds.data_ptr())
    p, s = oracle.quantize_q4(w)
    assert (ds.cpu().numpy().view(np.uint16) == s).all()
    bad = np.nonzero(dp.cpu().numpy() != p)[0]
    assert bad.size == 0, (bad.size, bad[:4])


@pytest.mark.parametrize("D,I", [(64, 64), (2048, 768), (4096, 1536)])
def test_expert_pool_bit_exact(ctx, oracle, D, I):
    shape = smoe_amd.make_shape(D, 4, 2, I)
    off, raw, stride = smoe_amd.blob_layout(D, I)
    pool = torch.zeros(3 * 4 * stride, dtype=torch.uint8, device="cuda")
    ctx.synth_expert_pool(pool.data_ptr(), 5, 3, 4, stride, shape, 42, 0.02)
    host = pool.cpu().numpy()
    for (l, e) in ((0, 0), (2, 3), (1, 2)):
        blob = host[(l * 4 + e) * stride:(l * 4 + e) * stride + raw]
        for m in range(3):
            rows, cols = (I, D) if m < 2 else (D, I)
            pk, sc = oracle.synth_q4(rows, cols, 42, smoe_amd.expert_stream(5 + l, e, m), 0.02)
            assert (blob[off[2 * m]:off[2 * m] + pk.size] == pk).all(), (l, e, m)
            assert (blob[off[2 * m + 1]:off[2 * m + 1] + sc.size * 2].view(np.uint16) == sc).all()
