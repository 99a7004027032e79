"""Minimal GGUF reader for the float64 host reference of the qwen35moe graph.

TEST INFRASTRUCTURE ONLY (the checker, never the product path). Parses the
GGUF container the way the reference's streaming reader does
(metal_model.cpp:451-562: magic 0x46554747, version 2 or 3, typed metadata,
tensor directory, `general.alignment` data start) and hands out raw tensor
bytes through a read-only memory map. Dequantization goes through the
oracle's bit-exact C++ restatement of model.cpp:543-683 (oracle.dequant_rows).
"""

from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = 0x46554747
BLOCK = {0: (1, 4), 1: (1, 2), 6: (32, 22), 8: (32, 34), 12: (256, 144), 14: (256, 210)}

# metadata value types (GGUF spec; metal_model.cpp:88-187)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GgufFile:
    def __init__(self, path):
        self.path = str(path)
        self.data = np.memmap(self.path, dtype=np.uint8, mode="r")
        self.pos = 0
        if self._u32() != GGUF_MAGIC:
            raise ValueError("not a GGUF file")
        version = self._u32()
        if version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {version}")
        n_tensors, n_kv = self._u64(), self._u64()
        self.meta = {}
        for _ in range(n_kv):
            key = self._str()
            self.meta[key] = self._value(self._u32())
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._str()
            nd = self._u32()
            dims = [self._u64() for _ in range(nd)]
            qtype = self._u32()
            off = self._u64()
            self.tensors[name] = (dims, qtype, off)
        align = int(self.meta.get("general.alignment", 32))
        self.data_start = (self.pos + align - 1) // align * align

    def _take(self, n):
        b = bytes(self.data[self.pos:self.pos + n])
        self.pos += n
        return b

    def _u32(self):
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self):
        return struct.unpack("<Q", self._take(8))[0]

    def _str(self):
        return self._take(self._u64()).decode("utf-8")

    def _value(self, t):
        if t in _SCALAR:
            fmt = _SCALAR[t]
            return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]
        if t == 8:
            return self._str()
        if t == 9:
            et, n = self._u32(), self._u64()
            return [self._value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF metadata type {t}")

    def dims(self, name):
        return self.tensors[name][0]

    def qtype(self, name):
        return self.tensors[name][1]

    def raw_rows(self, name, r0=0, r1=None):
        """Native bytes of rows [r0, r1) as a [rows, row_bytes] uint8 array."""
        dims, qtype, off = self.tensors[name]
        cols = dims[0]
        rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
        r1 = rows if r1 is None else r1
        be, bb = BLOCK[qtype]
        rb = cols // be * bb
        start = self.data_start + off + r0 * rb
        return np.asarray(self.data[start:start + (r1 - r0) * rb]).reshape(r1 - r0, rb), cols

    def f32_rows(self, name, r0=0, r1=None):
        """FP32 dequantized rows [r0, r1) (bit-exact to the reference's CPU path)."""
        import oracle
        raw, cols = self.raw_rows(name, r0, r1)
        return oracle.dequant_rows(self.qtype(name), raw, cols)
