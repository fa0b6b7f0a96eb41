"""BMTS shard reading and Hadamard sign slices (ouroboros_amd/shard.py)
against the reference's own tests of the format (bmts.rs:433-509) and the
HadRuntime rules (qwen35.rs:585-627).  CPU only: no device is touched."""
import json
import struct

import numpy as np
import pytest

from ouroboros_amd.quant import QuantKind
from ouroboros_amd.shard import (BMTS_MAGIC, BmtsShard, BmtsTensor, HadRuntime, ShardError, write_shard)


def two_tensor_shard(path):
    blob = bytes(range(64))
    tensors = [BmtsTensor("blk.0.attn_q.weight", [8, 8], 34, 0, 32),
               BmtsTensor("blk.0.attn_k.weight", [8, 8], 34, 32, 32)]
    write_shard(str(path), 1, tensors, blob)
    return blob


def test_bmts_roundtrip(tmp_path):  # bmts.rs:433-496
    blob = two_tensor_shard(tmp_path / "shard_1.bmts")
    with BmtsShard(str(tmp_path / "shard_1.bmts")) as shard:
        assert shard.node == 1 and len(shard.tensors) == 2 and shard.data_len() == 64
        assert shard.read_tensor("blk.0.attn_q.weight") == blob[0:32]
        assert shard.read_tensor("blk.0.attn_k.weight") == blob[32:64]
        with pytest.raises(ShardError):
            shard.read_tensor("missing")
        # a sub-span of a tensor, size-stamp checked; the full span equals the tensor
        assert bytes(shard.read_span("blk.0.attn_q.weight", 8, 16)) == blob[8:24]
        assert bytes(shard.read_span("blk.0.attn_q.weight", 0, 32)) == blob[0:32]
        with pytest.raises(ShardError):
            shard.read_span("blk.0.attn_q.weight", 0, 33)
        assert shard.layers() == [0]


def test_bmts_bad_magic(tmp_path):  # bmts.rs:498-507
    p = tmp_path / "bad.bmts"
    p.write_bytes(bytes(32))
    with pytest.raises(ShardError):
        BmtsShard(str(p))


def test_bmts_malformed_headers(tmp_path):
    meta = json.dumps([{"name": "a", "shape": [4], "dtype": 0, "offset": 0, "length": 16}]).encode()
    cases = {
        "short": b"OURO",
        "truncated_meta": struct.pack("<IHHII", BMTS_MAGIC, 1, 1, 1, len(meta) + 10) + meta,
        "count_mismatch": struct.pack("<IHHII", BMTS_MAGIC, 1, 1, 2, len(meta)) + meta + bytes(16),
        "v2_capnp": struct.pack("<IHHII", BMTS_MAGIC, 2, 1, 1, 8) + bytes(8),
        "unknown_version": struct.pack("<IHHII", BMTS_MAGIC, 7, 1, 1, len(meta)) + meta,
        "bad_json": struct.pack("<IHHII", BMTS_MAGIC, 1, 1, 1, 5) + b"[{]]]",
    }
    for name, raw in cases.items():
        p = tmp_path / f"{name}.bmts"
        p.write_bytes(raw)
        with pytest.raises(ShardError):
            BmtsShard(str(p))


def test_tensor_range_beyond_file_refused(tmp_path):
    p = tmp_path / "short_data.bmts"
    write_shard(str(p), 3, [BmtsTensor("w", [256, 2], 0, 0, 2048)], bytes(100))
    with BmtsShard(str(p)) as shard:
        with pytest.raises(ShardError):
            shard.tensor_bytes("w")


def test_weight_shape_follows_stage_from_shard(tmp_path):  # mod.rs:114-123
    p = tmp_path / "shapes.bmts"
    tensors = [BmtsTensor("blk.3.ffn_up.weight", [2560, 6912], 143, 0, 0),
               BmtsTensor("blk.3.attn_norm.weight", [2560], 0, 0, 0),
               BmtsTensor("output.weight", [5120, 248320], 34, 0, 0),
               BmtsTensor("blk.12.bad", [2, 2, 2], 0, 0, 0),
               BmtsTensor("blk.12.q4k", [256, 1], 12, 0, 0),
               BmtsTensor("blk.12.q6k", [512, 3], 14, 0, 0),
               BmtsTensor("blk.12.i2s", [256, 4], 36, 0, 0),
               BmtsTensor("blk.12.q2k", [256, 4], 10, 0, 0)]
    write_shard(str(p), 2, tensors, b"")
    with BmtsShard(str(p)) as shard:
        assert shard.weight_shape("blk.3.ffn_up.weight") == (QuantKind.TL1, 6912, 2560)
        assert shard.weight_shape("blk.3.attn_norm.weight") == (QuantKind.F32, 1, 2560)
        assert shard.weight_shape("output.weight") == (QuantKind.TQ1_0, 248320, 5120)
        with pytest.raises(ShardError):
            shard.weight_shape("blk.12.bad")  # rank 3
        # the K-quant ids of QuantKind::from_dtype (dequant.rs:334-348)
        assert shard.weight_shape("blk.12.q4k") == (QuantKind.Q4K, 1, 256)
        assert shard.weight_shape("blk.12.q6k") == (QuantKind.Q6K, 3, 512)
        # from_dtype's None: I2_S (36) and Q2_K (10) are not in the reference's set
        for name in ("blk.12.i2s", "blk.12.q2k"):
            with pytest.raises(ShardError):
                shard.weight_shape(name)
        assert shard.layers() == [3, 12]


def test_had_runtime_offsets(tmp_path):  # qwen35.rs:603-613
    widths = [2560, 6912, 4096]
    signs = np.concatenate([np.full(w, (-1) ** i) for i, w in enumerate(widths)])
    cfg = {"block_size": 256, "sign_widths": widths, "signs": [int(v) for v in signs], "gdn_v_grouped": True}
    p = tmp_path / "hadamard.json"
    p.write_text(json.dumps(cfg))
    had = HadRuntime.from_json(str(p))
    assert had.block == 256 and had.gdn_v_grouped
    assert [had.offset_for(w) for w in widths] == [0, 2560, 2560 + 6912]
    assert (had.signs[had.offset_for(6912):had.offset_for(6912) + 6912] == -1).all()
    with pytest.raises(ShardError):
        had.offset_for(1024)
    with pytest.raises(ShardError):
        HadRuntime(256, [8, 8], np.ones(15))
    assert not HadRuntime.from_json(json.dumps({"block_size": 4, "sign_widths": [4], "signs": [1, 1, 1, 1]})).gdn_v_grouped
