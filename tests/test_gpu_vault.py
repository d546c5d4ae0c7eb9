"""Vault -> HBM-resident pool (smoe_hip_vault_load): the loaded pool equals
the written blobs bit for bit, in the writer's layer-major order (one copy
segment) and in a shuffled file order (one segment per blob), and decode
through the layers the vault describes matches decode on the source pool bit
for bit and the CPU oracle of decode.cpp:236-509 within 1e-3."""
import numpy as np
import pytest
import torch

import smoe_amd
from smoe_amd import vault as V
from gpu_helpers import Layer, hidden_states, moe_delta_err, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
D, E, K, I = 2048, 16, 8, 768          # 30B-shaped experts, 16 per layer (80 MB of vault)
LAYER_IDS = [5, 9]


@pytest.fixture(scope="module")
def layers(ctx):
    return [Layer(ctx, D, E, K, I, layer_id=70 + i) for i in range(len(LAYER_IDS))]


def write(layers, path, order=None):
    _, raw, stride = smoe_amd.blob_layout(D, I)

    def blob(l, e):
        src = layers[LAYER_IDS.index(l)].h_pool
        return src[e * stride:e * stride + raw].tobytes()
    V.write_vault(path, LAYER_IDS, E, D, I, blob, order=order)


@pytest.mark.parametrize("shuffled", [False, True], ids=["layer_major", "shuffled"])
def test_vault_load_is_bit_exact(ctx, layers, tmp_path, shuffled):
    order = None
    if shuffled:
        pairs = [(l, e) for l in LAYER_IDS for e in range(E)]
        order = [pairs[i] for i in np.random.default_rng(3).permutation(len(pairs))]
    path = str(tmp_path / "t.smoe")
    write(layers, path, order)
    v = smoe_amd.Vault(path)
    assert v.info.num_moe_layers == len(LAYER_IDS) and v.info.experts_per_layer == E
    pool = torch.full((v.pool_bytes,), 0xA5, dtype=torch.uint8, device="cuda")
    v.load(pool.data_ptr(), pool.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    n = E * v.info.stride
    for m in range(len(LAYER_IDS)):
        assert v.layer_id(m) == LAYER_IDS[m]
        assert torch.equal(pool[m * n:(m + 1) * n], layers[m].pool)
    v.close()


def test_decode_through_vault_layers(ctx, oracle, layers, tmp_path):
    path = str(tmp_path / "d.smoe")
    write(layers, path)
    v = smoe_amd.Vault(path)
    pool = torch.empty((v.pool_bytes,), dtype=torch.uint8, device="cuda")
    v.load(pool.data_ptr(), pool.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for m, src in enumerate(layers):
        L = v.layer(m, pool.data_ptr(), norm_w=src.norm_w.data_ptr(), router_w=src.router.data_ptr())
        x0 = hidden_states(ctx, 1, D, 40 + m)[0]
        h0 = x0.cpu().numpy()
        a, b = x0.clone(), x0.clone()
        ids = torch.zeros(K, dtype=torch.int32, device="cuda")
        w = torch.zeros(K, dtype=torch.float32, device="cuda")
        ctx.moe_decode(src.shape, L, a.data_ptr(), 1, ids.data_ptr(), w.data_ptr())
        ctx.moe_decode(src.shape, src.layer, b.data_ptr(), 1)
        ctx.synchronize()
        assert torch.equal(a, b)
        out, oid, ow, _lg, _nr, yo = src.oracle_decode(oracle, h0)
        assert (ids.cpu().numpy().view(np.uint32) == oid).all()
        e1, _ = moe_delta_err(a.cpu().numpy(), h0, yo, ow)
        e2, _ = rel_err(a.cpu().numpy(), out)
        print(f"vault layer {m}: rel_err delta={e1:.2e} hidden={e2:.2e}")
        assert max(e1, e2) <= TOL
    v.close()
