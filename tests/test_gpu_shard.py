"""Tensors read from a memory-mapped BMTS shard (the reference's on-disk
format) decoded on the GPU: PTQ1_0 (TL1), TQ1_0 and F16 matrices uploaded
straight from the mapping into resident weights, against the oracle on the
same bytes at the reference's matvec bar (rel 1e-5, ops.rs:800-838); the
Hadamard sign slice for a width drives ouro_fwht_rows exactly as the
oracle's rotate_fwd on that slice."""
import json

import numpy as np
import pytest

from ouroboros_amd import _lib
from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.shard import BmtsShard, BmtsTensor, HadRuntime, write_shard
from test_gpu_matvec_q import close, tl1_payload, tq1_payload

pytestmark = pytest.mark.gpu


def build_shard(path, rng):
    parts = {
        "blk.0.ffn_up.weight": (143, [2560, 512], tl1_payload(rng, 512, 2560)),
        "blk.0.attn_qkv.weight": (34, [2560, 256], tq1_payload(rng, 256, 2560)),
        "blk.1.ffn_down.weight": (1, [512, 64],
                                  rng.standard_normal(64 * 512).astype(np.float16).view(np.uint8)),
    }
    tensors, blob, off = [], bytearray(), 0
    for name, (dtype, shape, payload) in parts.items():
        b = payload.tobytes()
        tensors.append(BmtsTensor(name, shape, dtype, off, len(b)))
        blob += b
        off += len(b)
        blob += bytes((-off) % 64)  # the reference's sharder aligns tensors; any offset must work
        off = len(blob)
    write_shard(str(path), 1, tensors, bytes(blob))
    return parts


def test_shard_tensors_decode_on_gpu(gpu, orc, tmp_path):
    rng = np.random.default_rng(8)
    parts = build_shard(tmp_path / "stage_1.bmts", rng)
    shard = BmtsShard(str(tmp_path / "stage_1.bmts"))
    weights = shard.upload_all()
    for name, (dtype, shape, payload) in parts.items():
        kind, out_len, in_len = shard.weight_shape(name)
        x = rng.standard_normal(in_len).astype(np.float32)
        want = orc.matvec_q(payload, int(kind), out_len, in_len, x)
        got = weights[name].matvec(x)
        assert close(got, want, 1e-5).all(), name
    for w in weights.values():
        w.free()
    shard.close()


def test_sign_slices_drive_the_rotation(gpu, orc, tmp_path):
    rng = np.random.default_rng(9)
    widths = [512, 2560]
    signs = rng.choice([-1, 1], sum(widths))
    p = tmp_path / "hadamard.json"
    p.write_text(json.dumps({"block_size": 512, "sign_widths": widths, "signs": [int(v) for v in signs]}))
    had = HadRuntime.from_json(str(p))
    x = rng.standard_normal((4, 2560)).astype(np.float32)
    want = x.copy()
    off = had.offset_for(2560)
    orc.rotate_rows(want, had.signs[off:off + 2560], had.block)
    sp, block = had.fwht_args(2560)
    xd, yd = DeviceBuffer.from_host(x), DeviceBuffer((4, 2560), np.float32)
    _lib.call("ouro_fwht_rows", xd.ptr, _lib.DT_F32, yd.ptr, _lib.DT_F32, 4, 2560, block, sp, 0, None, None, None)
    assert np.array_equal(yd.download(), want)
