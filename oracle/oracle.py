"""ctypes binding of the CPU oracle (liboracle_smoe.so) and of the compiled
reference routines (_ref/libsmoe_ref.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg.  The product never imports it.
Each wrapper names the reference file:line its C function restates; see
smoe_oracle.h for how each one is pinned.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_smoe.so")
REF_PATH = os.path.join(HERE, "_ref", "libsmoe_ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def build(reference_root: str | None = None) -> None:
    """Compile the oracle (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-B", "liboracle_smoe.so"], cwd=HERE, check=True)
    ref = reference_root or "/root/reference"
    if os.path.isdir(os.path.join(ref, "src")):
        subprocess.run(["make", "-s", "-B", "ref", f"REF={ref}"], cwd=HERE, check=True)


class OrcShape(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("d_model", "n_experts", "top_k", "d_ff", "group_size", "norm_topk", "quant")]


class OrcLayer(C.Structure):
    _fields_ = [("norm_w", C.c_void_p), ("router_w", C.c_void_p), ("experts", C.c_void_p),
                ("stride", C.c_uint64)] + [(n, C.c_uint64) for n in (
                    "gate_packed", "gate_scales", "up_packed", "up_scales",
                    "down_packed", "down_scales")]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_stream_key.restype = C.c_uint64
        L.orc_stream_key.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_rand64.restype = C.c_uint64
        L.orc_rand64.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_normal.restype = C.c_float
        L.orc_normal.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_gen_normal.argtypes = [_f32p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float]
        L.orc_gen_bf16.argtypes = [_u16p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float]
        L.orc_quantize_q4.argtypes = [_f32p, C.c_size_t, C.c_uint32, _u8p, _u16p]
        L.orc_dequant_q4_all.argtypes = [_u8p, _u16p, C.c_size_t, C.c_uint32, _f32p]
        L.orc_synth_q4.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.c_uint32,
                                   C.c_uint64, C.c_uint64, C.c_float]
        L.orc_rms_norm_bf16.argtypes = [_f32p, _u16p, C.c_uint32]
        L.orc_matvec_bf16.argtypes = [_f32p, _u16p, _f32p, C.c_uint32, C.c_uint32]
        L.orc_axpy_f32.argtypes = [_f32p, C.c_float, _f32p, C.c_uint32]
        L.orc_top_k.restype = C.c_uint32
        L.orc_top_k.argtypes = [_f32p, C.c_uint32, C.c_uint32, _u32p, _f32p, C.c_int]
        L.orc_silu.restype = C.c_float
        L.orc_silu.argtypes = [C.c_float]
        L.orc_expert_ffn.argtypes = [_u8p, _u16p, _u8p, _u16p, _u8p, _u16p, _f32p, _f32p,
                                     _f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_expert_ffn_decode.argtypes = [_u8p, _u16p, _u8p, _u16p, _u8p, _u16p, _f32p, _f32p,
                                            _f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_expert_ffn_decode_min.argtypes = [_u8p, _u16p, _u16p, _u8p, _u16p, _u16p, _u8p, _u16p, _u16p,
                                                _f32p, _f32p, _f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_quantize_q4_min.argtypes = [_f32p, C.c_size_t, C.c_uint32, _u8p, _u16p, _u16p]
        L.orc_dequant_q4_min.restype = C.c_float
        L.orc_dequant_q4_min.argtypes = [_u8p, _u16p, _u16p, C.c_size_t, C.c_uint32]
        L.orc_blob_layout.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32,
                                      C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        L.orc_moe_decode_layer.argtypes = [C.POINTER(OrcShape), C.POINTER(OrcLayer), _f32p,
                                           _u32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p]
        _u16n = C.c_void_p   # optional bf16 norm weights (None skips the norm)
        L.orc_attention_layer.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16n, _u16n, _f32p, _f32p, _f32p,
                                          _f32p, _f32p, _f32p] + [C.c_uint32] * 7 + [C.c_float]
        L.orc_permute.restype = C.c_uint32
        L.orc_permute.argtypes = [_u32p, _f32p, C.c_uint32, C.c_uint32, C.c_uint32, _u32p,
                                  _u32p, _f32p, _u32p]
        L.orc_union_reset.argtypes = []
        L.orc_union_add.restype = C.c_int
        L.orc_union_add.argtypes = [C.c_uint32, C.c_uint32, C.c_float]
        for n in ("orc_union_size",):
            getattr(L, n).restype = C.c_uint32
        for n in ("orc_union_id", "orc_union_count"):
            getattr(L, n).restype = C.c_uint32
            getattr(L, n).argtypes = [C.c_uint32]
        L.orc_union_tok.restype = C.c_uint32
        L.orc_union_tok.argtypes = [C.c_uint32, C.c_uint32]
        L.orc_union_w.restype = C.c_float
        L.orc_union_w.argtypes = [C.c_uint32, C.c_uint32]
        L.orc_moe_prefill_layer.argtypes = [C.POINTER(OrcShape), C.POINTER(OrcLayer), _f32p,
                                            C.c_uint32, _u32p, _f32p]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_get_threads.restype = C.c_int
        L.orc_max_threads.restype = C.c_int
        _lib = L
    return _lib


_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own top_k / common.hpp / union_add, compiled from its
    sources by `make ref` (oracle/Makefile)."""
    global _ref
    if _ref is None:
        R = C.CDLL(REF_PATH)
        R.ref_top_k.restype = C.c_uint32
        R.ref_top_k.argtypes = [_f32p, C.c_uint32, C.c_uint32, _u32p, _f32p, C.c_int]
        R.ref_rms_norm_bf16.argtypes = [_f32p, _u16p, C.c_uint32]
        R.ref_matvec_bf16.argtypes = [_f32p, _u16p, _f32p, C.c_uint32, C.c_uint32]
        R.ref_axpy_f32.argtypes = [_f32p, C.c_float, _f32p, C.c_uint32]
        R.ref_bf16_to_f32.restype = C.c_float
        R.ref_bf16_to_f32.argtypes = [C.c_uint16]
        R.ref_union_add.restype = C.c_int
        R.ref_union_add.argtypes = [C.c_uint32, C.c_uint32, C.c_float]
        R.ref_union_size.restype = C.c_uint32
        for n in ("ref_union_id", "ref_union_count"):
            getattr(R, n).restype = C.c_uint32
            getattr(R, n).argtypes = [C.c_uint32]
        R.ref_union_tok.restype = C.c_uint32
        R.ref_union_tok.argtypes = [C.c_uint32, C.c_uint32]
        R.ref_union_w.restype = C.c_float
        R.ref_union_w.argtypes = [C.c_uint32, C.c_uint32]
        _ref = R
    return _ref


# --------------------------------------------------------------------------
# numpy-level helpers
# --------------------------------------------------------------------------

def usable_cores() -> int:
    """Host cores this process may use: the CPU affinity mask, capped by
    OMP_NUM_THREADS when that is set."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


class threads:
    """Context manager: the oracle's row-parallel loops on n threads (results
    are bit-identical for any n)."""

    def __init__(self, n: int):
        self.n = max(1, int(n))

    def __enter__(self):
        self.prev = lib().orc_get_threads()
        lib().orc_set_threads(self.n)
        return self

    def __exit__(self, *exc):
        lib().orc_set_threads(self.prev)
        return False


def gen_normal(n, seed, stream, stddev=1.0):
    out = np.empty(n, np.float32)
    lib().orc_gen_normal(out, n, seed, stream, stddev)
    return out


def gen_bf16(n, seed, stream, stddev=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_gen_bf16(out, n, seed, stream, stddev)
    return out


def quantize_q4(w, group=64):
    w = np.ascontiguousarray(w, np.float32).ravel()
    n = w.size
    packed = np.zeros((n + 1) // 2, np.uint8)
    scales = np.zeros((n + group - 1) // group, np.uint16)
    lib().orc_quantize_q4(w, n, group, packed, scales)
    return packed, scales


def dequant_q4(packed, scales, n, group=64):
    out = np.empty(n, np.float32)
    lib().orc_dequant_q4_all(np.ascontiguousarray(packed), np.ascontiguousarray(scales), n, group, out)
    return out


def synth_q4(rows, cols, seed, stream, stddev=0.02, group=64):
    packed = np.zeros(rows * cols // 2, np.uint8)
    scales = np.zeros(rows * cols // group, np.uint16)
    lib().orc_synth_q4(packed, scales, rows, cols, group, seed, stream, stddev)
    return packed, scales


def rms_norm_bf16(x, w):
    x = np.array(x, np.float32, copy=True)
    lib().orc_rms_norm_bf16(x, np.ascontiguousarray(w, np.uint16), x.size)
    return x


def matvec_bf16(W, x):
    rows, cols = W.shape
    out = np.empty(rows, np.float32)
    lib().orc_matvec_bf16(out, np.ascontiguousarray(W, np.uint16), np.ascontiguousarray(x, np.float32), rows, cols)
    return out


def top_k(scores, k, norm_topk=False):
    scores = np.ascontiguousarray(scores, np.float32)
    ids = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    cnt = lib().orc_top_k(scores, scores.size, k, ids, w, int(norm_topk))
    return ids[:cnt], w[:cnt]


def expert_ffn(blob, off, D, I, x, group=64, decode=False, quant=0):
    """Run one expert given its blob bytes and the 6 offsets: the prefill
    token-batch arithmetic (orc_expert_ffn), or with decode=True the decode
    path's (orc_expert_ffn_decode, kernels.metal:159-365); quant=1: the
    scale+min format on the decode path's lanes and chunks."""
    blob = np.ascontiguousarray(blob, np.uint8)

    def u8(o, n):
        return np.ascontiguousarray(blob[o:o + n])

    def u16(o, n):
        return np.ascontiguousarray(blob[o:o + 2 * n]).view(np.uint16)

    n = D * I
    h = np.empty(I, np.float32)
    y = np.empty(D, np.float32)
    if quant:
        ng = n // group
        lib().orc_expert_ffn_decode_min(u8(off[0], n // 2), u16(off[1], ng), u16(off[1] + 2 * ng, ng),
                                        u8(off[2], n // 2), u16(off[3], ng), u16(off[3] + 2 * ng, ng),
                                        u8(off[4], n // 2), u16(off[5], ng), u16(off[5] + 2 * ng, ng),
                                        np.ascontiguousarray(x, np.float32), h, y, I, D, group)
        return h, y
    fn = lib().orc_expert_ffn_decode if decode else lib().orc_expert_ffn
    fn(u8(off[0], n // 2), u16(off[1], n // group), u8(off[2], n // 2),
       u16(off[3], n // group), u8(off[4], n // 2), u16(off[5], n // group),
       np.ascontiguousarray(x, np.float32), h, y, I, D, group)
    return h, y


def blob_layout(D, I, group=64, quant=0):
    """Offsets of the six tensors of one expert blob and its size; quant=1
    (the scale+min format): each matrix's mins follow its scales, inside the
    scales' region, which doubles."""
    if quant:
        n = D * I
        pb, sb = n // 2, 2 * (n // group * 2)
        return [0, pb, pb + sb, 2 * pb + sb, 2 * (pb + sb), 3 * pb + 2 * sb], 3 * (pb + sb)
    off = (C.c_uint64 * 6)()
    nb = C.c_uint64()
    lib().orc_blob_layout(D, I, group, off, C.byref(nb))
    return [int(v) for v in off], int(nb.value)


def quantize_q4_min(w, group=64):
    """The scale+min format: (packed, scales, mins) of w, bf16 bits."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    n = w.size
    packed = np.zeros(n // 2, np.uint8)
    scales = np.zeros(n // group, np.uint16)
    mins = np.zeros(n // group, np.uint16)
    lib().orc_quantize_q4_min(w, n, group, packed, scales, mins)
    return packed, scales, mins


def dequant_q4_min(packed, scales, mins, n, group=64):
    p, s, m = (np.ascontiguousarray(a) for a in (packed, scales, mins))
    return np.array([lib().orc_dequant_q4_min(p, s, m, i, group) for i in range(n)], np.float32)


def _layer_struct(norm_w, router_w, experts, stride, off):
    L = OrcLayer()
    L.norm_w = norm_w.ctypes.data
    L.router_w = router_w.ctypes.data
    L.experts = experts.ctypes.data
    L.stride = stride
    (L.gate_packed, L.gate_scales, L.up_packed, L.up_scales, L.down_packed,
     L.down_scales) = off
    return L


def moe_decode_layer(shape: dict, norm_w, router_w, experts, stride, off, hidden):
    """One decode MoE block.  experts: uint8 array holding n_experts blobs of
    `stride` bytes.  Returns (hidden_out, ids, weights, logits, normed, expert_out)."""
    S = OrcShape(**shape)
    L = _layer_struct(norm_w, router_w, experts, stride, off)
    h = np.array(hidden, np.float32, copy=True)
    K = shape["top_k"]
    ids = np.zeros(K, np.uint32)
    w = np.zeros(K, np.float32)
    logits = np.zeros(shape["n_experts"], np.float32)
    normed = np.zeros(shape["d_model"], np.float32)
    yo = np.zeros((K, shape["d_model"]), np.float32)
    lib().orc_moe_decode_layer(C.byref(S), C.byref(L), h, ids, w, logits.ctypes.data,
                               normed.ctypes.data, yo.ctypes.data)
    return h, ids, w, logits, normed, yo


def moe_prefill_layer(shape: dict, norm_w, router_w, experts, stride, off, hidden):
    S = OrcShape(**shape)
    L = _layer_struct(norm_w, router_w, experts, stride, off)
    h = np.array(hidden, np.float32, copy=True)
    T = h.shape[0]
    K = shape["top_k"]
    ids = np.zeros((T, K), np.uint32)
    w = np.zeros((T, K), np.float32)
    lib().orc_moe_prefill_layer(C.byref(S), C.byref(L), h, T, ids, w)
    return h, ids, w


def permute(ids, w, n_experts):
    ids = np.ascontiguousarray(ids, np.uint32)
    w = np.ascontiguousarray(w, np.float32)
    T, K = ids.shape
    offsets = np.zeros(n_experts + 1, np.uint32)
    tok = np.zeros(T * K, np.uint32)
    wo = np.zeros(T * K, np.float32)
    uni = np.zeros(n_experts, np.uint32)
    nu = lib().orc_permute(ids, w, T, K, n_experts, offsets, tok, wo, uni)
    return offsets, tok, wo, uni[:nu]


def attention_layer(w_q, w_k, w_v, w_o, q_norm_w, k_norm_w, rope_cos, rope_sin, normed_in, k_cache, v_cache,
                    head_dim, num_heads, num_kv_heads, slot, valid, scale):
    """decode.cpp:150-229 (CPU branch).  Weights uint16 bf16 bits (norm weights
    may be None); k_cache / v_cache [attn_ctx x kv_dim] are copied and the copies
    updated.  Returns (o_out, k_cache, v_cache)."""
    kc = np.array(k_cache, np.float32, copy=True)
    vc = np.array(v_cache, np.float32, copy=True)
    d_model = len(normed_in)
    o = np.zeros(d_model, np.float32)
    c16 = lambda a: np.ascontiguousarray(a, np.uint16)
    qn = c16(q_norm_w) if q_norm_w is not None else None
    kn = c16(k_norm_w) if k_norm_w is not None else None
    lib().orc_attention_layer(c16(w_q), c16(w_k), c16(w_v), c16(w_o),
                              qn.ctypes.data if qn is not None else None, kn.ctypes.data if kn is not None else None,
                              np.ascontiguousarray(rope_cos, np.float32), np.ascontiguousarray(rope_sin, np.float32),
                              np.ascontiguousarray(normed_in, np.float32), kc, vc, o, d_model, head_dim, num_heads,
                              num_kv_heads, slot, valid, kc.shape[0], scale)
    return o, kc, vc

