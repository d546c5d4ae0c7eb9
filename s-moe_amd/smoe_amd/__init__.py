"""Python binding of libsmoe_hip.so (the C ABI declared in include/smoe_hip.h).

Plain ctypes over the C ABI: pointers are integers (device addresses from any
allocator, e.g. torch tensors' data_ptr()), sizes are integers.  Importing this
module loads the HIP library and raises if it is missing: there is no CPU
fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsmoe_hip.so")

SMOE_OK = 0
SMOE_ERR_ARG = -1
SMOE_ERR_SHAPE = -2
SMOE_ERR_BITS = -3
SMOE_ERR_HIP = -4
SMOE_ERR_CAPACITY = -5
SMOE_ERR_CAPTURE = -6
SMOE_ERR_VAULT = -7
_ERR_NAMES = {v: k for k, v in globals().items() if k.startswith("SMOE_ERR_")}

SMOE_MAX_ACTIVE = 16
SMOE_MAX_FFN_BATCH = 64
PAGE = 16384  # vault blob padding (shatter_moe.py:999-1005)

# synthetic-input stream ids (shared with the host generator in oracle/)
MATRIX_GATE, MATRIX_UP, MATRIX_DOWN = 0, 1, 2


def expert_stream(layer: int, expert: int, matrix: int) -> int:
    return (layer << 32) | (expert << 4) | matrix


def router_stream(layer: int) -> int:
    return (layer << 32) | 0xFFFFFF00


def hidden_stream(index: int) -> int:
    return (0xFFFF << 48) | index


class SmoeMoeShape(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("d_model", "n_experts", "top_k", "d_ff", "group_size", "bits", "norm_topk", "quant")]


QUANT_SMOEQ4, QUANT_Q4_SCALE_MIN = 0, 1


class SmoeMoeLayer(C.Structure):
    _fields_ = [("norm_w", C.c_void_p), ("router_w", C.c_void_p), ("experts", C.c_void_p),
                ("expert_stride", C.c_uint64)] + [(n, C.c_uint64) for n in (
                    "gate_packed_offset", "gate_scales_offset", "up_packed_offset",
                    "up_scales_offset", "down_packed_offset", "down_scales_offset")]


class SmoeVaultInfo(C.Structure):
    _fields_ = ([(n, C.c_uint32) for n in ("version", "num_moe_layers", "experts_per_layer", "total_experts",
                                           "group_size", "bits", "d_model", "d_ff", "vocab_size", "ffn_dim")]
                + [(n, C.c_uint64) for n in ("blob_bytes", "stride", "gate_packed_offset", "gate_scales_offset",
                                             "up_packed_offset", "up_scales_offset", "down_packed_offset",
                                             "down_scales_offset")]
                + [(n, C.c_uint32) for n in ("arch_valid", "arch_flags", "num_heads", "num_kv_heads", "head_dim",
                                             "moe_top_k", "moe_ffn_dim", "dense_ffn_dim", "shared_expert_ffn_dim",
                                             "num_hidden_layers")]
                + [("rope_theta", C.c_float), ("rms_norm_eps", C.c_float), ("model_type", C.c_char * 24)])


class SmoeAttnLayerArgs(C.Structure):
    _fields_ = ([(n, C.c_void_p) for n in ("w_q", "w_k", "w_v", "w_o", "q_norm_w", "k_norm_w", "rope_cos",
                                           "rope_sin", "normed_in", "qbuf", "kbuf", "vbuf", "k_cache", "v_cache",
                                           "attn_out", "o_out")]
                + [(n, C.c_uint32) for n in ("d_model", "q_dim", "kv_dim", "head_dim", "num_heads", "num_kv_heads",
                                             "slot", "valid", "attn_ctx")]
                + [("attn_scale", C.c_float)])


class SmoeExpertBlob(C.Structure):
    _fields_ = [("packed_gate", C.c_void_p), ("scales_gate", C.c_void_p),
                ("packed_up", C.c_void_p), ("scales_up", C.c_void_p),
                ("packed_down", C.c_void_p), ("scales_down", C.c_void_p),
                ("slot", C.c_uint32)]


# (name, restype, argtypes) of every exported entry point, in header order
_VP, _U32, _U64, _F, _SZ, _I = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_size_t, C.c_int
_SHP, _LAY = C.POINTER(SmoeMoeShape), C.POINTER(SmoeMoeLayer)
SIGNATURES = [
    ("smoe_metal_init", _VP, [_SZ]),
    ("smoe_metal_destroy", None, [_VP]),
    ("smoe_metal_fused_ffn", _VP, [_VP] + [_VP] * 6 + [_VP, _VP, _VP] + [_U32] * 7),
    ("smoe_metal_wait", None, [_VP, _VP, _VP, _U32, _U32]),
    ("smoe_metal_fused_ffn_group", _VP, [_VP, C.POINTER(SmoeExpertBlob), _U32, _VP] + [_U32] * 6),
    ("smoe_metal_fused_ffn_batch", _VP, [_VP] + [_VP] * 6 + [_VP, _U32] + [_U32] * 6),
    ("smoe_metal_wait_ffn_batch", None, [_VP, _VP, _VP, _U32, _U32]),
    ("smoe_metal_register_buffer", None, [_VP, _VP, _SZ]),
    ("smoe_metal_kernel_dispatches", _U64, [_VP]),
    ("smoe_metal_scout_matvec_bf16", None, [_VP, _VP, _VP, _VP, _U32, _U32]),
    ("smoe_metal_scout_matvec_batch_bf16", None, [_VP, _VP, _VP, _VP, _VP, _VP, _U32]),
    ("smoe_metal_scout_matvec_group_bf16", None, [_VP, _VP, _VP, _VP, _VP, _VP, _U32]),
    ("smoe_metal_attention_layer", None, [_VP, C.POINTER(SmoeAttnLayerArgs)]),
    ("smoe_hip_set_stream", _I, [_VP, _VP]),
    ("smoe_hip_synchronize", _I, [_VP]),
    ("smoe_hip_exchange_tags", None, [_U32, _U32, _VP, _VP, _VP]),
    ("smoe_hip_exchange_epoch", _I, [_VP, _VP, _VP, _VP, _VP]),
    ("smoe_hip_reserve", _I, [_VP, _SHP, _U32]),
    ("smoe_hip_moe_decode", _I, [_VP, _SHP, _LAY, _VP, _U32, _VP, _VP]),
    ("smoe_hip_moe_decode_stack", _I, [_VP, _SHP, _LAY, _U32, _VP, _VP, _VP]),
    ("smoe_hip_set_decode_engine", _I, [_VP, _I]),
    ("smoe_hip_moe_prefill", _I, [_VP, _SHP, _LAY, _VP, _U32, _VP, _VP, _VP, _VP, _VP, _VP]),
    ("smoe_hip_moe_prefill_stack", _I, [_VP, _SHP, _LAY, _U32, _VP, _U32, _VP, _VP]),
    ("smoe_hip_compute_top_k", _I, [_VP, _VP, _U32, _U32, _U32, _VP, _VP, _I]),
    ("smoe_hip_permute", _I, [_VP, _VP, _VP, _U32, _U32, _U32, _VP, _VP, _VP, _VP, _VP]),
    ("smoe_hip_quantize_q4", _I, [_VP, _VP, _U64, _U32, _VP, _VP]),
    ("smoe_hip_quantize_q4_scale_min", _I, [_VP, _VP, _U64, _U32, _VP, _VP, _VP]),
    ("smoe_hip_synth_normal", _I, [_VP, _VP, _U64, _U64, _U64, _F]),
    ("smoe_hip_synth_bf16", _I, [_VP, _VP, _U64, _U64, _U64, _F]),
    ("smoe_hip_synth_expert_pool", _I, [_VP, _VP, _U32, _U32, _U32, _U64, _SHP, _U64, _F]),
    ("smoe_hip_matvec_bf16", _I, [_VP, _VP, _VP, _VP, _U32, _U32]),
    ("smoe_hip_matvec_group_bf16", _I, [_VP, C.POINTER(_VP), C.POINTER(_VP), C.POINTER(_VP),
                                        C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), _U32]),
    ("smoe_hip_attention_layer", _I, [_VP, C.POINTER(SmoeAttnLayerArgs)]),
    ("smoe_hip_vault_open", _I, [C.c_char_p, C.POINTER(_VP)]),
    ("smoe_hip_vault_close", None, [_VP]),
    ("smoe_hip_vault_info", _I, [_VP, C.POINTER(SmoeVaultInfo)]),
    ("smoe_hip_vault_layer_id", _I, [_VP, _U32, C.POINTER(C.c_uint32)]),
    ("smoe_hip_vault_layer", _I, [_VP, _U32, _VP, _LAY]),
    ("smoe_hip_vault_load", _I, [_VP, _VP, _U64, _VP]),
    ("smoe_hip_vault_error", C.c_char_p, []),
    ("smoe_hip_profile_enable", _I, [_VP, _I]),
    ("smoe_hip_profile_read", _I, [_VP, _U32, C.POINTER(C.c_uint64), C.POINTER(C.c_double)]),
    ("smoe_hip_last_error", C.c_char_p, [_VP]),
    ("smoe_hip_stream_read", _I, [_VP, _VP, _U64, _VP]),
    ("smoe_hip_moe_decode_static", _I, [C.POINTER(SmoeMoeShape), C.POINTER(SmoeMoeLayer), _VP, _VP, _VP, _VP,
                                        _VP]),
]

KERNEL_MOE_UP, KERNEL_GATE_UP, KERNEL_MOE_DOWN, KERNEL_DOWN_SLOTS, KERNEL_TOPK = 0, 1, 2, 3, 4
KERNEL_PERMUTE, KERNEL_GROUPED_GATE_UP, KERNEL_GROUPED_DOWN, KERNEL_SCATTER = 5, 6, 7, 8
KERNEL_ROUTE, KERNEL_SPLIT, KERNEL_MOE_LAYER = 9, 10, 12
KERNEL_GEMV, KERNEL_ATTENTION, KERNEL_STREAM, KERNEL_CHAIN = 13, 14, 15, 17
DECODE_LAUNCHES, DECODE_SPLIT, DECODE_CHAIN = 0, 2, 4
KERNEL_NAMES = {0: "moe_up", 1: "gate_up", 2: "moe_down", 3: "down_slots", 4: "topk",
                5: "permute", 6: "grouped_gate_up", 7: "grouped_down", 8: "combine", 9: "route",
                10: "split", 12: "moe_layer", 13: "gemv", 14: "attention",
                15: "stream_read", 17: "moe_chain"}

_lib = None


def lib():
    """Load libsmoe_hip.so (raises OSError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: run s-moe_amd/build.py (the HIP path has no fallback)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class SmoeError(RuntimeError):
    """A non-zero status of the C ABI; `code` is the SMOE_ERR_* value."""

    def __init__(self, msg, code=None):
        super().__init__(msg)
        self.code = code


def blob_layout(d_model: int, d_ff: int, group: int = 64, quant: int = 0):
    """Offsets of the six tensors in one expert blob (build_expert_blob,
    shatter_moe.py:627-674), the raw blob size and the 16 KB-padded stride.
    quant=QUANT_Q4_SCALE_MIN: each matrix's bf16 mins follow its bf16 scales
    inside the scales' region (twice the SMOE-Q4 size)."""
    n = d_model * d_ff
    pb, sb = n // 2, n // group * 2 * (2 if quant == QUANT_Q4_SCALE_MIN else 1)
    off = [0, pb, pb + sb, 2 * pb + sb, 2 * (pb + sb), 3 * pb + 2 * sb]
    raw = 3 * (pb + sb)
    stride = (raw + PAGE - 1) // PAGE * PAGE
    return off, raw, stride


def make_shape(d_model, n_experts, top_k, d_ff, group_size=64, norm_topk=True, bits=4, quant=QUANT_SMOEQ4):
    return SmoeMoeShape(d_model, n_experts, top_k, d_ff, group_size, bits, 1 if norm_topk else 0, quant)


def make_layer(norm_w: int, router_w: int, experts: int, stride: int, off):
    L = SmoeMoeLayer()
    L.norm_w, L.router_w, L.experts, L.expert_stride = norm_w, router_w, experts, stride
    (L.gate_packed_offset, L.gate_scales_offset, L.up_packed_offset, L.up_scales_offset,
     L.down_packed_offset, L.down_scales_offset) = off
    return L


class Context:
    """Owns one SmoeMetalCtx.  Device-resident entry points raise SmoeError on
    a non-zero status."""

    def __init__(self, slot_bytes: int = 0):
        self.lib = lib()
        self.ptr = self.lib.smoe_metal_init(slot_bytes)
        if not self.ptr:
            raise SmoeError("smoe_metal_init failed (no HIP device?)")

    def close(self):
        if self.ptr:
            self.lib.smoe_metal_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != SMOE_OK:
            msg = self.lib.smoe_hip_last_error(self.ptr)
            raise SmoeError(f"{what}: {_ERR_NAMES.get(rc, rc)} {msg.decode() if msg else ''}", rc)

    # -- stream -------------------------------------------------------------
    def set_stream(self, stream_handle: int | None):
        """Launch on this hipStream_t from now on (0 / None = the null stream)."""
        self._check(self.lib.smoe_hip_set_stream(self.ptr, stream_handle or None), "set_stream")

    def synchronize(self):
        self._check(self.lib.smoe_hip_synchronize(self.ptr), "synchronize")

    def reserve(self, shape: SmoeMoeShape, max_tokens: int):
        self._check(self.lib.smoe_hip_reserve(self.ptr, C.byref(shape), max_tokens), "reserve")

    # -- MoE block ----------------------------------------------------------
    def moe_decode(self, shape, layer, hidden: int, n_tokens: int, ids: int = 0, weights: int = 0):
        self._check(self.lib.smoe_hip_moe_decode(self.ptr, C.byref(shape), C.byref(layer), hidden,
                                                 n_tokens, ids or None, weights or None), "moe_decode")

    def moe_prefill_stack(self, shape, layers, hidden: int, n_tokens: int, ids: int = 0, weights: int = 0):
        """layers: a sequence of SmoeMoeLayer (or a ctypes array of them)."""
        if not isinstance(layers, C.Array):
            layers = (SmoeMoeLayer * len(layers))(*layers)
        self._check(self.lib.smoe_hip_moe_prefill_stack(self.ptr, C.byref(shape), layers, len(layers), hidden,
                                                        n_tokens, ids or None, weights or None),
                    "moe_prefill_stack")

    # -- dense trunk ------------------------------------------------------------
    def matvec_bf16(self, w: int, x: int, y: int, rows: int, cols: int):
        self._check(self.lib.smoe_hip_matvec_bf16(self.ptr, w, x, y, rows, cols), "matvec_bf16")

    def matvec_group_bf16(self, ws, xs, ys, rows, cols):
        n = len(ws)
        arr = lambda v, t: (t * n)(*v)
        self._check(self.lib.smoe_hip_matvec_group_bf16(self.ptr, arr(ws, C.c_void_p), arr(xs, C.c_void_p),
                                                        arr(ys, C.c_void_p), arr(rows, C.c_uint32),
                                                        arr(cols, C.c_uint32), n), "matvec_group_bf16")

    def attention_layer(self, args: "SmoeAttnLayerArgs", sync: bool = False):
        """smoe_hip_attention_layer (async); sync=True uses the reference-surface
        smoe_metal_attention_layer instead (synchronous, errors to stderr)."""
        if sync:
            self.lib.smoe_metal_attention_layer(self.ptr, C.byref(args))
        else:
            self._check(self.lib.smoe_hip_attention_layer(self.ptr, C.byref(args)), "attention_layer")

    def set_decode_engine(self, engine: int):
        """DECODE_CHAIN (one launch per step, the default), DECODE_LAUNCHES (per-layer
        calls) or DECODE_SPLIT (per-layer calls, always two launches per layer)."""
        self._check(self.lib.smoe_hip_set_decode_engine(self.ptr, engine), "set_decode_engine")

    def exchange_epoch(self, set_chain=None, set_layer=None):
        """smoe_hip_exchange_epoch: optionally set the chained kernel's and the
        one-launch layer kernel's epoch words; returns (chain, layer) as read
        afterwards (None for words not allocated yet)."""
        out = []
        for i, v in enumerate((set_chain, set_layer)):
            val = C.c_uint32(v or 0)
            got = C.c_uint32(0)
            args = [None, None, None, None]
            if v is not None:
                args[i] = C.byref(val)
            args[2 + i] = C.byref(got)
            rc = self.lib.smoe_hip_exchange_epoch(self.ptr, *args)
            if rc == SMOE_ERR_ARG and v is None:
                out.append(None)
                continue
            self._check(rc, "exchange_epoch")
            out.append(got.value)
        return tuple(out)

    def moe_decode_stack(self, shape, layers, hidden: int, ids: int = 0, weights: int = 0):
        """layers: a sequence of SmoeMoeLayer (or a ctypes array of them)."""
        if not isinstance(layers, C.Array):
            arr = (SmoeMoeLayer * len(layers))(*layers)
        else:
            arr = layers
        self._check(self.lib.smoe_hip_moe_decode_stack(self.ptr, C.byref(shape), arr, len(arr), hidden,
                                                       ids or None, weights or None), "moe_decode_stack")

    def moe_prefill(self, shape, layer, hidden: int, n_tokens: int, ids: int = 0, weights: int = 0,
                    expert_offsets: int = 0, sorted_tokens: int = 0, union_ids: int = 0,
                    union_size: int = 0):
        self._check(self.lib.smoe_hip_moe_prefill(
            self.ptr, C.byref(shape), C.byref(layer), hidden, n_tokens, ids or None, weights or None,
            expert_offsets or None, sorted_tokens or None, union_ids or None, union_size or None),
            "moe_prefill")

    def compute_top_k(self, scores: int, n_rows: int, n: int, k: int, ids: int, weights: int,
                      norm_topk: bool):
        self._check(self.lib.smoe_hip_compute_top_k(self.ptr, scores, n_rows, n, k, ids, weights,
                                                    1 if norm_topk else 0), "compute_top_k")

    def permute(self, ids: int, weights: int, n_tokens: int, top_k: int, n_experts: int,
                expert_offsets: int, sorted_tokens: int, sorted_weights: int, union_ids: int,
                union_size: int):
        self._check(self.lib.smoe_hip_permute(self.ptr, ids, weights, n_tokens, top_k, n_experts,
                                              expert_offsets, sorted_tokens, sorted_weights,
                                              union_ids, union_size), "permute")

    # -- synthetic inputs -----------------------------------------------------
    def quantize_q4(self, w: int, n: int, group: int, packed: int, scales: int):
        self._check(self.lib.smoe_hip_quantize_q4(self.ptr, w, n, group, packed, scales), "quantize_q4")

    def quantize_q4_scale_min(self, w: int, n: int, group: int, packed: int, scales: int, mins: int):
        self._check(self.lib.smoe_hip_quantize_q4_scale_min(self.ptr, w, n, group, packed, scales, mins),
                    "quantize_q4_scale_min")

    def synth_normal(self, out: int, n: int, seed: int, stream: int, stddev: float):
        self._check(self.lib.smoe_hip_synth_normal(self.ptr, out, n, seed, stream, stddev), "synth_normal")

    def synth_bf16(self, out: int, n: int, seed: int, stream: int, stddev: float):
        self._check(self.lib.smoe_hip_synth_bf16(self.ptr, out, n, seed, stream, stddev), "synth_bf16")

    def synth_expert_pool(self, base: int, first_layer: int, n_layers: int, n_experts: int,
                          stride: int, shape: SmoeMoeShape, seed: int, stddev: float):
        self._check(self.lib.smoe_hip_synth_expert_pool(self.ptr, base, first_layer, n_layers, n_experts,
                                                        stride, C.byref(shape), seed, stddev),
                    "synth_expert_pool")

    # -- reference surface (metal_bridge.h) ----------------------------------
    def fused_ffn_group(self, blobs, input_vec_host, gate_rows, gate_cols, group=64, bits=4):
        arr = (SmoeExpertBlob * len(blobs))(*blobs)
        return self.lib.smoe_metal_fused_ffn_group(self.ptr, arr, len(blobs), input_vec_host, gate_rows,
                                                   gate_cols, gate_cols, gate_rows, group, bits)

    def wait(self, handle, out_host, slot, cols):
        self.lib.smoe_metal_wait(self.ptr, handle, out_host, slot, cols)

    def profile_enable(self, on: bool = True):
        self._check(self.lib.smoe_hip_profile_enable(self.ptr, 1 if on else 0), "profile_enable")

    def profile_read(self, kernel: int):
        """(launches, total_ms) of one kernel kind since profile_enable."""
        n = C.c_uint64()
        ms = C.c_double()
        self._check(self.lib.smoe_hip_profile_read(self.ptr, kernel, C.byref(n), C.byref(ms)), "profile_read")
        return int(n.value), float(ms.value)

    def stream_read(self, src: int, nbytes: int, sink: int):
        """Measurement: one streaming read of nbytes at src (the HBM ceiling)."""
        self._check(self.lib.smoe_hip_stream_read(self.ptr, src, nbytes, sink), "stream_read")

    def dispatches(self) -> int:
        return int(self.lib.smoe_metal_kernel_dispatches(self.ptr))


class Vault:
    """A parsed and checked .smoe vault (smoe_hip_vault_open); raises
    SmoeError with the library's message when the file is malformed."""

    def __init__(self, path: str):
        self.lib = lib()
        self.ptr = C.c_void_p()
        rc = self.lib.smoe_hip_vault_open(os.fsencode(path), C.byref(self.ptr))
        if rc != SMOE_OK:
            self.ptr = None
            raise SmoeError(f"vault_open: {_ERR_NAMES.get(rc, rc)} {self.lib.smoe_hip_vault_error().decode()}",
                            rc)
        self.info = SmoeVaultInfo()
        self._check(self.lib.smoe_hip_vault_info(self.ptr, C.byref(self.info)), "vault_info")

    def _check(self, rc, what):
        if rc != SMOE_OK:
            raise SmoeError(f"{what}: {_ERR_NAMES.get(rc, rc)} {self.lib.smoe_hip_vault_error().decode()}", rc)

    def close(self):
        if self.ptr:
            self.lib.smoe_hip_vault_close(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pool_bytes(self) -> int:
        return self.info.num_moe_layers * self.info.experts_per_layer * self.info.stride

    def layer_id(self, moe_index: int) -> int:
        out = C.c_uint32()
        self._check(self.lib.smoe_hip_vault_layer_id(self.ptr, moe_index, C.byref(out)), "vault_layer_id")
        return int(out.value)

    def layer(self, moe_index: int, dev_pool: int, norm_w: int = 0, router_w: int = 0) -> SmoeMoeLayer:
        L = SmoeMoeLayer()
        L.norm_w, L.router_w = norm_w or None, router_w or None
        self._check(self.lib.smoe_hip_vault_layer(self.ptr, moe_index, dev_pool, C.byref(L)), "vault_layer")
        return L

    def load(self, dev_pool: int, pool_bytes: int, stream: int | None = None):
        self._check(self.lib.smoe_hip_vault_load(self.ptr, dev_pool, pool_bytes, stream or None), "vault_load")


def exchange_tags(epoch: int, n_layers: int):
    """smoe_hip_exchange_tags (host only): (tags [n_layers], abort value, next
    epoch) of a one-launch decode of n_layers layers that reads `epoch`."""
    tags = (C.c_uint32 * max(n_layers, 1))()
    ab, nxt = C.c_uint32(0), C.c_uint32(0)
    lib().smoe_hip_exchange_tags(epoch, n_layers, tags, C.byref(ab), C.byref(nxt))
    return [int(t) for t in tags[:n_layers]], ab.value, nxt.value
