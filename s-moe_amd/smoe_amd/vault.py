"""Writer of .smoe vaults (the format of common.hpp:57-181, as laid out by
shatter_moe.py:947-1098), for synthetic layers: header, expert table, three
tensor descriptors per expert, the v2 arch block in the gap before the data,
then every blob 16 KB aligned in layer-major order.  The struct layouts are
the format's and must stay byte-identical; the reader is smoe_hip_vault_open
(smoe_amd.Vault)."""
from __future__ import annotations

import struct

from . import PAGE, blob_layout

MAGIC = b"SMOE\xDE\xEA\x00\x01"
ARCH_MAGIC = b"SARC"
HEADER = struct.Struct("<8sIIIIQQIIIIII")           # 64 bytes
ENTRY = struct.Struct("<IIQQQIQxxxx")              # 48 bytes
DESC = struct.Struct("<BBxxIIQQQQ")                # 44 bytes
ARCH = struct.Struct("<4sIIIfIIIIIIIIIf24s44x")    # 128 bytes
ARCH_NORM_TOPK, ARCH_QK_NORM, ARCH_DENSE_LAYER_0 = 1, 2, 4

QWEN3_30B_ARCH = dict(flags=ARCH_NORM_TOPK | ARCH_QK_NORM, rope_theta=1e6, num_heads=32, num_kv_heads=4,
                      head_dim=128, moe_top_k=8, moe_ffn_dim=768, dense_ffn_dim=0, shared_expert_ffn_dim=0,
                      activation=0, num_hidden_layers=48, rms_norm_eps=1e-6, model_type="qwen3_moe")


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def layout(n_experts_total: int):
    """(arch_offset, data_offset) of a vault with this many table entries."""
    meta = HEADER.size + n_experts_total * (ENTRY.size + 3 * DESC.size)
    arch_offset = _align(meta, 64)
    return arch_offset, _align(arch_offset + ARCH.size, PAGE)


def write_vault(path, layer_ids, n_experts: int, d_model: int, d_ff: int, blob_fn, *, version: int = 2,
                arch: dict | None = None, vocab_size: int = 151936, ffn_dim: int = 0, group_size: int = 64,
                bits: int = 4, order=None):
    """Write a vault whose expert (l, e) blob is blob_fn(l, e) (bytes of the
    blob_layout(d_model, d_ff) size) for every l in layer_ids, e < n_experts,
    in file order `order` (a permutation of those (l, e) pairs; default
    layer-major, as the reference's writer).  Returns the list of
    (layer_id, expert_id, byte_offset) written."""
    off, raw, stride = blob_layout(d_model, d_ff, group_size)
    n = d_model * d_ff
    pb, sb = n // 2, n // group_size * 2
    entries = [(l, e) for l in layer_ids for e in range(n_experts)]
    if order is not None:
        if sorted(order) != sorted(entries):
            raise ValueError("order must list every (layer, expert) pair once")
        entries = list(order)
    arch_offset, data_offset = layout(len(entries))
    if version < 2:
        arch_offset = 0
    written = []
    with open(path, "wb") as f:
        f.seek(data_offset)
        for l, e in entries:
            blob = blob_fn(l, e)
            if len(blob) != raw:
                raise ValueError(f"blob of layer {l} expert {e} has {len(blob)} bytes, expected {raw}")
            pos = f.tell()
            f.write(blob)
            f.write(b"\0" * (stride - raw))
            written.append((l, e, pos))
        f.seek(0)
        f.write(HEADER.pack(MAGIC, version, len(layer_ids), n_experts, len(entries), HEADER.size, data_offset,
                            group_size, bits, d_model, vocab_size, ffn_dim, arch_offset))
        for (l, e, pos) in written:
            f.write(ENTRY.pack(l, e, pos, raw, stride, group_size, 3 * n // group_size))
        for _ in written:
            # gate [I x D], up [I x D], down [D x I]: packed then scales each
            f.write(DESC.pack(0, 2, d_ff, d_model, off[0], pb, off[1], sb))
            f.write(DESC.pack(1, 2, d_ff, d_model, off[2], pb, off[3], sb))
            f.write(DESC.pack(2, 2, d_model, d_ff, off[4], pb, off[5], sb))
        if version >= 2:
            a = dict(QWEN3_30B_ARCH, moe_ffn_dim=d_ff)
            a.update(arch or {})
            f.write(b"\0" * (arch_offset - f.tell()))
            f.write(ARCH.pack(ARCH_MAGIC, 1, ARCH.size, a["flags"], a["rope_theta"], a["num_heads"],
                              a["num_kv_heads"], a["head_dim"], a["moe_top_k"], a["moe_ffn_dim"],
                              a["dense_ffn_dim"], a["shared_expert_ffn_dim"], a["activation"],
                              a["num_hidden_layers"], a["rms_norm_eps"], a["model_type"].encode()[:24]))
        f.write(b"\0" * (data_offset - f.tell()))
    return written
