""".smoe vault reader (smoe_hip_vault_open, the checks of main.cpp:96-157 and
streamer.cpp:183-212 plus every expert's descriptors) on files written in the
format of common.hpp:57-181 by smoe_amd.vault.  Host code only: no GPU."""
import os
import struct

import numpy as np
import pytest

import smoe_amd
from smoe_amd import vault as V

D, I, E = 64, 128, 4
LAYERS = [1, 3]


def blob(l, e):
    _, raw, _ = smoe_amd.blob_layout(D, I)
    rng = np.random.default_rng(1000 * l + e)
    return rng.integers(0, 256, raw, dtype=np.uint8).tobytes()


def write(tmp_path, name="v.smoe", **kw):
    p = str(tmp_path / name)
    V.write_vault(p, LAYERS, E, D, I, blob, **kw)
    return p


def patch(path, offset, fmt, value):
    with open(path, "r+b") as f:
        f.seek(offset)
        f.write(struct.pack(fmt, value))


def expect_error(path, code, text):
    with pytest.raises(smoe_amd.SmoeError) as ei:
        smoe_amd.Vault(path)
    assert ei.value.code == code, ei.value
    assert text in str(ei.value), ei.value


def test_v2_vault_is_read(tmp_path):
    p = write(tmp_path)
    v = smoe_amd.Vault(p)
    f = v.info
    off, raw, stride = smoe_amd.blob_layout(D, I)
    assert (f.version, f.num_moe_layers, f.experts_per_layer, f.total_experts) == (2, 2, E, 2 * E)
    assert (f.d_model, f.d_ff, f.group_size, f.bits) == (D, I, 64, 4)
    assert (f.blob_bytes, f.stride) == (raw, stride)
    assert [f.gate_packed_offset, f.gate_scales_offset, f.up_packed_offset, f.up_scales_offset,
            f.down_packed_offset, f.down_scales_offset] == off
    assert f.arch_valid == 1 and f.moe_top_k == 8 and f.num_heads == 32 and f.num_kv_heads == 4
    assert f.model_type == b"qwen3_moe" and abs(f.rms_norm_eps - 1e-6) < 1e-12
    assert [v.layer_id(m) for m in range(2)] == LAYERS
    assert v.pool_bytes == 2 * E * stride
    base = 1 << 40
    L = v.layer(1, base, norm_w=0x1000, router_w=0x2000)
    assert L.experts == base + E * stride and L.expert_stride == stride
    assert L.down_scales_offset == off[5] and L.norm_w == 0x1000 and L.router_w == 0x2000
    with pytest.raises(smoe_amd.SmoeError):
        v.layer_id(2)
    v.close()


def test_v1_vault_has_no_arch_block(tmp_path):
    v = smoe_amd.Vault(write(tmp_path, version=1))
    assert v.info.version == 1 and v.info.arch_valid == 0


def test_blobs_land_where_the_table_says(tmp_path):
    p = write(tmp_path)
    raw = open(p, "rb").read()
    hdr = V.HEADER.unpack_from(raw, 0)
    n = hdr[4]
    for i in range(n):
        l, e, pos, rsz, psz, g, ng = V.ENTRY.unpack_from(raw, V.HEADER.size + i * V.ENTRY.size)
        assert pos % smoe_amd.PAGE == 0 and psz % smoe_amd.PAGE == 0
        assert raw[pos:pos + rsz] == blob(l, e)


@pytest.mark.parametrize("case", [
    "truncated", "magic", "version3", "no_arch", "arch_magic", "activation", "top_k", "heads",
    "bits2", "group32", "misaligned", "past_eof", "packed_size", "tensor_type", "layout", "missing",
    "duplicate", "layer_count", "table_overlaps_data", "d_model", "packed_offset_wraps", "scales_offset_wraps",
    "packed_misaligned", "scales_misaligned", "table_offset_wraps", "arch_offset_wraps"])
def test_malformed_vaults_are_rejected(tmp_path, case):
    p = write(tmp_path)
    n = 2 * E
    arch_off, data_off = V.layout(n)
    ent = lambda i: V.HEADER.size + i * V.ENTRY.size
    desc = lambda i, t: V.HEADER.size + n * V.ENTRY.size + (3 * i + t) * V.DESC.size
    code, text = smoe_amd.SMOE_ERR_VAULT, ""
    if case == "truncated":
        with open(p, "r+b") as f:
            f.truncate(40)
        text = "too small"
    elif case == "magic":
        patch(p, 0, "<4s", b"SMOF")
        text = "magic"
    elif case == "version3":
        patch(p, 8, "<I", 3)
        text = "version 3"
    elif case == "no_arch":
        patch(p, 60, "<I", 0)
        text = "arch-block offset"
    elif case == "arch_magic":
        patch(p, arch_off, "<4s", b"SARK")
        text = "corrupt arch block"
    elif case == "activation":
        patch(p, arch_off + 48, "<I", 1)
        text = "SiLU only"
    elif case == "top_k":
        patch(p, arch_off + 32, "<I", 17)
        text = "engine limits"
    elif case == "heads":
        patch(p, arch_off + 24, "<I", 5)             # 32 query heads over 5 kv heads
        text = "engine limits"
    elif case == "bits2":
        patch(p, 44, "<I", 2)
        code, text = smoe_amd.SMOE_ERR_BITS, "2-bit"
    elif case == "group32":
        patch(p, 40, "<I", 32)
        code, text = smoe_amd.SMOE_ERR_SHAPE, "group size 32"
    elif case == "misaligned":
        patch(p, ent(3) + 8, "<Q", data_off + 4096)
        text = "misplaced"
    elif case == "past_eof":
        patch(p, ent(n - 1) + 8, "<Q", os.path.getsize(p))
        text = "misplaced"
    elif case == "packed_size":
        patch(p, desc(2, 1) + 20, "<Q", D * I // 2 - 16)
        text = "does not describe"
    elif case == "tensor_type":
        patch(p, desc(5, 2), "<B", 1)
        text = "does not describe"
    elif case == "layout":
        # expert 6 moves its down scales (still inside the blob, unlike expert 0)
        patch(p, desc(6, 2) + 28, "<Q", smoe_amd.blob_layout(D, I)[0][5] - 64)
        text = "unlike expert 0"
    elif case == "missing":
        patch(p, ent(5) + 4, "<I", 7)                # expert id past max_experts_per_layer
        text = "max_experts_per_layer"
    elif case == "duplicate":
        patch(p, ent(5) + 4, "<I", 0)                # layer 3 gets expert 0 twice, loses expert 1
        text = "twice"
    elif case == "layer_count":
        patch(p, 12, "<I", 3)
        text = "MoE layers"
    elif case == "table_overlaps_data":
        patch(p, 32, "<Q", V.HEADER.size + n * V.ENTRY.size)   # data offset inside the descriptors
        text = "does not fit"
    elif case == "d_model":
        patch(p, 48, "<I", 2 * D)
        code, text = smoe_amd.SMOE_ERR_SHAPE, "d_model"
    elif case == "packed_offset_wraps":
        # offset + size wraps around 2^64 to a value inside the blob
        patch(p, desc(0, 0) + 12, "<Q", (1 << 64) - 16)
        text = "does not describe"
    elif case == "scales_offset_wraps":
        patch(p, desc(0, 1) + 28, "<Q", (1 << 64) - 2)
        text = "does not describe"
    elif case == "packed_misaligned":
        patch(p, desc(0, 0) + 12, "<Q", 8)            # inside the blob, not 16-byte aligned
        text = "not aligned"
    elif case == "scales_misaligned":
        patch(p, desc(0, 2) + 28, "<Q", smoe_amd.blob_layout(D, I)[0][5] - 1)
        text = "not aligned"
    elif case == "table_offset_wraps":
        patch(p, 24, "<Q", (1 << 64) - 64)
        text = "does not fit"
    elif case == "arch_offset_wraps":
        # the arch-block offset is 32-bit: largest value, past the data offset
        patch(p, 60, "<I", 0xFFFFFFFF)
        text = "arch-block offset"
    expect_error(p, code, text)


def test_missing_file_and_null_arguments(tmp_path):
    expect_error(str(tmp_path / "absent.smoe"), smoe_amd.SMOE_ERR_VAULT, "cannot open")
    L = smoe_amd.lib()
    assert L.smoe_hip_vault_open(None, None) == smoe_amd.SMOE_ERR_ARG
    assert L.smoe_hip_vault_info(None, None) == smoe_amd.SMOE_ERR_ARG
    assert L.smoe_hip_vault_load(None, None, 0, None) == smoe_amd.SMOE_ERR_ARG
    L.smoe_hip_vault_close(None)


def test_load_rejects_a_small_pool(tmp_path):
    v = smoe_amd.Vault(write(tmp_path))
    with pytest.raises(smoe_amd.SmoeError) as ei:
        v.load(1 << 40, v.pool_bytes - 1)
    assert ei.value.code == smoe_amd.SMOE_ERR_CAPACITY
