"""BMTS shards and Hadamard sign slices on the host side of the boundary:
what Stage::from_shard / Qwen35Stage::from_shard do before the kernels run
(cluster/src/bmts.rs, cluster/src/infer/mod.rs:112-135,
cluster/src/infer/qwen35.rs:345-356, 585-627).

A shard is memory-mapped and its tensors are handed to the device straight
from the mapping (no host copy): PTQ1_0 / TQ1_0 / dense payloads go to
`ops.Weight` handles, which decode them on the GPU.  Version-1 shards (JSON
tensor table) are read; version 2 (a Cap'n Proto table) is refused, as the
reference's default build refuses it (bmts.rs:196-211, the `capnp2`
feature).
"""
from __future__ import annotations

import json
import mmap
import os
import re
import struct
from dataclasses import dataclass

import numpy as np

from .quant import QuantKind

BMTS_MAGIC = 0x4F55524F  # "OURO" little-endian (bmts.rs:21)
BMTS_VERSION = 1
BMTS_VERSION_V2 = 2
BMTS_HEADER_LEN = 16


class ShardError(ValueError):
    """A malformed shard or a bad request against one (the reference bails)."""


@dataclass
class BmtsTensor:
    """One tensor of the table (bmts.rs:29-37): ggml shape [in_len, out_len]
    for matrices, dtype = ggml type id, offset/length within the data section."""
    name: str
    shape: list
    dtype: int
    offset: int
    length: int


class BmtsShard:
    """BmtsShard::open and its accessors (bmts.rs:171-308)."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size < BMTS_HEADER_LEN:
                raise ShardError(f"BMTS file too short: {path}")
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        magic, version, node, n_tensors, meta_len = struct.unpack_from("<IHHII", self._map, 0)
        if magic != BMTS_MAGIC:
            raise ShardError(f"bad BMTS magic {magic:#010x} in {path}")
        if size < BMTS_HEADER_LEN + meta_len:
            raise ShardError(f"BMTS meta truncated: {path}")
        meta = bytes(self._map[BMTS_HEADER_LEN:BMTS_HEADER_LEN + meta_len])
        if version == BMTS_VERSION:
            try:
                table = json.loads(meta)
                tensors = [BmtsTensor(str(t["name"]), [int(d) for d in t["shape"]], int(t["dtype"]),
                                      int(t["offset"]), int(t["length"])) for t in table]
            except (ValueError, KeyError, TypeError) as e:
                raise ShardError(f"BMTS tensor table unreadable in {path}: {e}") from e
        elif version == BMTS_VERSION_V2:
            raise ShardError(f"BMTS v{BMTS_VERSION_V2} (Cap'n Proto meta) is not read by this library: {path}")
        else:
            raise ShardError(f"unsupported BMTS version {version} in {path}")
        if len(tensors) != n_tensors:
            raise ShardError(f"BMTS tensor count mismatch: header {n_tensors} vs meta {len(tensors)}")
        self.node = node
        self.tensors = tensors
        self.data_start = BMTS_HEADER_LEN + meta_len
        self._by_name = {t.name: t for t in tensors}

    def close(self) -> None:
        """Unmap now if no tensor view is alive; otherwise the mapping goes
        when the last view does."""
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:
                pass
            self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def data_len(self) -> int:
        """Total declared tensor payload bytes (bmts.rs:273-276)."""
        return sum(t.length for t in self.tensors)

    def _range(self, name: str, offset: int, length: int) -> np.ndarray:
        start = self.data_start + offset
        if start + length > len(self._map):
            raise ShardError(f"tensor {name} range {start}..{start + length} exceeds file {len(self._map)}")
        return np.frombuffer(self._map, dtype=np.uint8, count=length, offset=start)

    def tensor(self, name: str) -> BmtsTensor:
        t = self._by_name.get(name)
        if t is None:
            raise ShardError(f"tensor {name} not in shard")
        return t

    def tensor_bytes(self, name: str) -> np.ndarray:
        """Zero-copy bytes of a tensor: a read-only view of the mapping (bmts.rs:258-271)."""
        t = self.tensor(name)
        return self._range(name, t.offset, t.length)

    def read_tensor(self, name: str) -> bytes:
        return bytes(self.tensor_bytes(name))

    def read_span(self, name: str, offset: int, length: int) -> np.ndarray:
        """A byte span of a tensor, refused (never truncated) past its declared
        length (bmts.rs:286-308)."""
        t = self.tensor(name)
        if offset < 0 or length < 0 or offset + length > t.length:
            raise ShardError(f"span [{offset}, {offset + length}) exceeds tensor {name} of {t.length} bytes "
                             f"(size-stamp {t.length})")
        return self._range(name, t.offset + offset, length)

    def layers(self) -> list:
        """Layer indices owned by the shard, from the blk.N.* names (mod.rs:125-133)."""
        out = set()
        for t in self.tensors:
            m = re.match(r"blk\.(\d+)\.", t.name)
            if m:
                out.add(int(m.group(1)))
        return sorted(out)

    def weight_shape(self, name: str) -> tuple:
        """(kind, out_len, in_len) of a tensor as Stage::from_shard reads it
        (mod.rs:114-123): rank 1 = [in], rank 2 = [in, out]."""
        t = self.tensor(name)
        kind = QuantKind.from_dtype(t.dtype)
        if kind is None:
            raise ShardError(f"unsupported dtype {t.dtype} on {t.name}")
        if len(t.shape) == 1:
            return kind, 1, t.shape[0]
        if len(t.shape) == 2:
            return kind, t.shape[1], t.shape[0]
        raise ShardError(f"tensor {t.name} has rank {len(t.shape)}")

    def upload(self, name: str, max_cols: int = 8):
        """A resident device weight of one tensor, uploaded from the mapping."""
        from .ops import Weight

        kind, out_len, in_len = self.weight_shape(name)
        return Weight(kind, self.tensor_bytes(name), out_len, in_len, max_cols=max_cols)

    def upload_all(self, max_cols: int = 8) -> dict:
        """Every tensor as a resident weight, by name (Stage::from_shard)."""
        return {t.name: self.upload(t.name, max_cols) for t in self.tensors}


def write_shard(path: str, node: int, tensors: list, data: bytes) -> None:
    """A version-1 shard (bmts.rs:311-324): header, JSON table, data."""
    meta = json.dumps([{"name": t.name, "shape": list(t.shape), "dtype": t.dtype, "offset": t.offset,
                        "length": t.length} for t in tensors]).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<IHHII", BMTS_MAGIC, BMTS_VERSION, node, len(tensors), len(meta)))
        f.write(meta)
        f.write(data)


class HadRuntime:
    """The Hadamard fold of a model (HadamardCfg / HadRuntime,
    qwen35.rs:345-356, 585-627): block size, per-width ±1 sign slices
    concatenated, and the V-grouped flag."""

    def __init__(self, block_size: int, sign_widths: list, signs, gdn_v_grouped: bool = False):
        self.block = int(block_size)
        self.widths = [int(w) for w in sign_widths]
        self.signs = np.asarray(signs, dtype=np.float32)
        self.gdn_v_grouped = bool(gdn_v_grouped)
        if self.signs.size != sum(self.widths):
            raise ShardError(f"hadamard signs: {self.signs.size} values for widths {self.widths}")
        self._dev = None

    @classmethod
    def from_json(cls, path_or_text: str) -> "HadRuntime":
        text = path_or_text
        if os.path.exists(path_or_text):
            with open(path_or_text) as f:
                text = f.read()
        cfg = json.loads(text)
        return cls(cfg["block_size"], cfg["sign_widths"], cfg["signs"], cfg.get("gdn_v_grouped", False))

    def offset_for(self, n: int) -> int:
        """Offset of the sign slice whose width is n (qwen35.rs:603-613)."""
        acc = 0
        for w in self.widths:
            if w == n:
                return acc
            acc += w
        raise ShardError(f"no hadamard sign slice for width {n}")

    def device_signs(self):
        """All slices in one device buffer (uploaded once)."""
        from .device import DeviceBuffer

        if self._dev is None:
            self._dev = DeviceBuffer.from_host(self.signs)
        return self._dev

    def fwht_args(self, n: int) -> tuple:
        """(signs device pointer, block) for ouro_fwht_rows on rows of width n:
        the x' = H (s o x) of rotate_fwd_for / wh (qwen35.rs:615-619, 683-692)."""
        return self.device_signs().ptr + 4 * self.offset_for(n), self.block
