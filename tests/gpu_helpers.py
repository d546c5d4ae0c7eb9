"""Shared helpers of the GPU tests: synthetic layers built on the device by the
library's generator, copied back for the CPU oracle, and the tolerance metric."""
import numpy as np
import torch

import smoe_amd

SEED = 20261201


def rel_err(got, ref, floor_frac=1e-2, slack=None):
    """max (|g - c| - slack) / max(|c|, tau), tau = floor_frac * rms(c): the
    per-element relative error with a floor so that elements near zero are
    judged against the vector's scale.  `slack` (absolute, per element)
    discounts a rounding both sides share by construction, e.g. the fp32
    residual add when a delta is read back as hidden_out - hidden_in.
    Returns (max_rel, n_below_floor)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    tau = floor_frac * np.sqrt(np.mean(ref ** 2)) + 1e-30
    den = np.maximum(np.abs(ref), tau)
    diff = np.abs(got - ref)
    if slack is not None:
        diff = np.maximum(diff - np.asarray(slack, np.float64), 0.0)
    return float(np.max(diff / den)), int(np.sum(np.abs(ref) < tau))


def moe_delta_err(got_hidden, h0, expert_out, weights):
    """Relative error of the GPU's MoE delta (hidden_out - hidden_in) against
    the oracle's sum_r w_r * y_r, with one ulp of hidden_out as slack for the
    fp32 residual add (decode.cpp:506-509) that both sides round."""
    got_hidden = np.asarray(got_hidden, np.float32)
    ref = (np.asarray(weights, np.float64)[:, None] * np.asarray(expert_out, np.float64)).sum(0)
    delta = got_hidden.astype(np.float64) - np.asarray(h0, np.float64)
    return rel_err(delta, ref, slack=np.spacing(np.abs(got_hidden)))


class Layer:
    """One MoE layer of a given shape, resident on cuda:0, plus host copies."""

    def __init__(self, ctx, D, E, K, I, layer_id=0, seed=SEED, norm_topk=True, router_std=0.02,
                 host=True, quant=0):
        self.D, self.E, self.K, self.I, self.quant = D, E, K, I, quant
        self.shape = smoe_amd.make_shape(D, E, K, I, 64, norm_topk, quant=quant)
        self.off, self.raw, self.stride = smoe_amd.blob_layout(D, I, quant=quant)
        dev = torch.device("cuda", 0)
        self.pool = torch.zeros(E * self.stride, dtype=torch.uint8, device=dev)
        ctx.synth_expert_pool(self.pool.data_ptr(), layer_id, 1, E, self.stride, self.shape, seed, 0.02)
        self.router = torch.empty(E * D, dtype=torch.int16, device=dev)
        ctx.synth_bf16(self.router.data_ptr(), E * D, seed, smoe_amd.router_stream(layer_id), router_std)
        self.norm_w = torch.full((D,), 0x3F80, dtype=torch.int16, device=dev)   # bf16 1.0
        self.layer = smoe_amd.make_layer(self.norm_w.data_ptr(), self.router.data_ptr(),
                                         self.pool.data_ptr(), self.stride, self.off)
        torch.cuda.synchronize()
        if host:
            self.host_copies()

    def host_copies(self):
        """Copies of the device weights for the oracle (again after a change)."""
        torch.cuda.synchronize()
        self.h_pool = self.pool.cpu().numpy()
        self.h_router = self.router.cpu().numpy().view(np.uint16)
        self.h_norm = self.norm_w.cpu().numpy().view(np.uint16)

    def oracle_shape(self):
        return dict(d_model=self.D, n_experts=self.E, top_k=self.K, d_ff=self.I, group_size=64,
                    norm_topk=self.shape.norm_topk, quant=self.quant)

    def oracle_decode(self, oracle, hidden):
        return oracle.moe_decode_layer(self.oracle_shape(), self.h_norm, self.h_router, self.h_pool,
                                       self.stride, self.off, hidden)


def hidden_states(ctx, T, D, index0=0, seed=SEED):
    h = torch.empty((T, D), dtype=torch.float32, device="cuda")
    for t in range(T):
        ctx.synth_normal(h[t].data_ptr(), D, seed, smoe_amd.hidden_stream(index0 + t), 1.0)
    return h


def q4_matrix_f64(layer, e, k):
    """Matrix k (0 gate [I x D], 1 up [I x D], 2 down [D x I]) of expert e,
    dequantised in fp64: (c - 7.5) / 7.5 * scale per 64-group, low nibble
    first (shatter_moe.py:371-387); for the scale+min format c * s + m with
    the bf16 scales and the mins after them."""
    blob = layer.h_pool[e * layer.stride:(e + 1) * layer.stride]
    n = layer.D * layer.I
    pk = blob[layer.off[2 * k]:layer.off[2 * k] + n // 2]
    codes = np.empty(n, np.float64)
    codes[0::2] = pk & 15
    codes[1::2] = pk >> 4
    if getattr(layer, "quant", 0):
        so = layer.off[2 * k + 1]
        bf = lambda a: (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        sc = bf(blob[so:so + 2 * (n // 64)].view(np.uint16))
        mn = bf(blob[so + 2 * (n // 64):so + 4 * (n // 64)].view(np.uint16))
        w = codes * np.repeat(sc, 64) + np.repeat(mn, 64)
        return w.reshape((layer.I, layer.D) if k < 2 else (layer.D, layer.I))
    sc = blob[layer.off[2 * k + 1]:layer.off[2 * k + 1] + 2 * (n // 64)].view(np.float16).astype(np.float64)
    w = (codes - 7.5) / 7.5 * np.repeat(sc, 64)
    return w.reshape((layer.I, layer.D) if k < 2 else (layer.D, layer.I))


def moe_block_f64(layer, x, ids, w, mats=None):
    """The MoE delta of one token in fp64 for given ids and weights: RMSNorm
    (norm weights 1), then sum_r w_r * down(silu(gate x) * (up x))."""
    mats = {} if mats is None else mats
    x = np.asarray(x, np.float64)
    xn = x / np.sqrt(np.mean(x * x) + 1e-6)
    y = np.zeros(layer.D)
    for r in range(len(ids)):
        e = int(ids[r])
        if e not in mats:
            mats[e] = [q4_matrix_f64(layer, e, k) for k in range(3)]
        g, u = mats[e][0] @ xn, mats[e][1] @ xn
        y += float(w[r]) * (mats[e][2] @ (g / (1.0 + np.exp(-g)) * u))
    return y


def moe_delta_f64_batch(layer, X, ids, w):
    """The MoE delta of every row of X [T x D] in fp64 for given ids / weights
    [T x K] (RMSNorm with norm weights 1, then sum_r w_r * down(silu(gate x) *
    (up x)) in rank order), one expert's matrices dequantised at a time."""
    X = np.asarray(X, np.float64)
    Xn = X / np.sqrt(np.mean(X * X, axis=1, keepdims=True) + 1e-6)
    T, K = ids.shape
    Y = np.zeros((T, K, layer.D))
    for e in np.unique(ids):
        t, r = np.nonzero(ids == e)
        G, U, Dn = (q4_matrix_f64(layer, int(e), k) for k in range(3))
        g, u = Xn[t] @ G.T, Xn[t] @ U.T
        Y[t, r] = (g / (1.0 + np.exp(-g)) * u) @ Dn.T
    out = np.zeros((T, layer.D))
    for r in range(K):
        out += np.asarray(w, np.float64)[:, r:r + 1] * Y[:, r]
    return out
