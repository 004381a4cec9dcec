"""GGUF v3 writer and reader (host side, numpy).

The reader mirrors the header walk of the reference's own parser
(`src/model/formats/mmap_gguf.rs:187-275`): magic, version 2/3, tensor and KV
counts, KV pairs, tensor infos with dims stored fastest-first and reversed to
row-major on read (`gguf.rs:277-291`), data section aligned.  Unlike
`mmap_gguf.rs:329-336` it sizes every KV value type per the GGUF spec, and it
honours `general.alignment` (the reference always uses 32, `:256-257`).

The writer emits only u32/i32/f32/u64/string KV types and 32-byte alignment,
so files it writes are also readable by the reference's parser.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747  # b"GGUF" little-endian
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q6_K = 0, 1, 2, 8, 14
BLOCK_BYTES = {GGML_Q4_0: 18, GGML_Q8_0: 34}
_KV_U32, _KV_I32, _KV_F32, _KV_STR, _KV_ARR, _KV_U64 = 4, 5, 6, 8, 9, 10
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B",
           10: "<Q", 11: "<q", 12: "<d"}


def tensor_nbytes(gtype: int, nelem: int) -> int:
    """Byte size of a tensor (`mmap_gguf.rs:353-379`)."""
    if gtype == GGML_F32:
        return nelem * 4
    if gtype == GGML_F16:
        return nelem * 2
    if gtype in BLOCK_BYTES:
        if nelem % 32:
            raise ValueError("quantised tensor size must be a multiple of 32")
        return nelem // 32 * BLOCK_BYTES[gtype]
    if gtype == GGML_Q6_K:
        return nelem // 256 * 210
    raise ValueError(f"unsupported GGUF tensor type {gtype}")


@dataclass
class GGUFTensor:
    name: str
    gtype: int
    shape: tuple          # row-major (reference order): W[N, K]
    data: bytes | np.ndarray


@dataclass
class GGUFWriter:
    kv: list = field(default_factory=list)
    tensors: list = field(default_factory=list)
    alignment: int = 32

    def add_u32(self, key: str, v: int):
        self.kv.append((key, _KV_U32, int(v)))

    def add_f32(self, key: str, v: float):
        self.kv.append((key, _KV_F32, float(v)))

    def add_str(self, key: str, v: str):
        self.kv.append((key, _KV_STR, v))

    def add_tensor(self, name: str, gtype: int, shape, data):
        nelem = int(np.prod(shape))
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        if len(raw) != tensor_nbytes(gtype, nelem):
            raise ValueError(f"{name}: {len(raw)} bytes for shape {shape} type {gtype}")
        self.tensors.append(GGUFTensor(name, gtype, tuple(int(s) for s in shape), raw))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def write(self, path: str):
        head = bytearray()
        head += struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kv))
        for key, t, v in self.kv:
            head += self._str(key) + struct.pack("<I", t)
            if t == _KV_STR:
                head += self._str(v)
            else:
                head += struct.pack(_SCALAR[t], v)
        offsets, off = [], 0
        for t in self.tensors:
            offsets.append(off)
            off += len(t.data)
            off = (off + self.alignment - 1) // self.alignment * self.alignment
        for t, o in zip(self.tensors, offsets):
            head += self._str(t.name) + struct.pack("<I", len(t.shape))
            for d in reversed(t.shape):            # GGUF stores fastest dim first
                head += struct.pack("<Q", d)
            head += struct.pack("<IQ", t.gtype, o)
        pad = (-len(head)) % self.alignment
        with open(path, "wb") as f:
            f.write(head)
            f.write(b"\0" * pad)
            pos = 0
            for t, o in zip(self.tensors, offsets):
                if o > pos:
                    f.write(b"\0" * (o - pos))
                    pos = o
                f.write(t.data)
                pos += len(t.data)


@dataclass
class GGUFInfo:
    name: str
    gtype: int
    shape: tuple
    offset: int
    nbytes: int


class GGUFReader:
    """Spec-correct GGUF reader over a numpy memmap."""

    def __init__(self, path: str):
        self.buf = np.memmap(path, dtype=np.uint8, mode="r")
        self.pos = 0
        magic, version = self._unpack("<II")
        if magic != GGUF_MAGIC:
            raise ValueError(f"invalid GGUF magic 0x{magic:08x}")
        if version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {version}")
        n_tensors, n_kv = self._unpack("<QQ")
        self.kv = {}
        for _ in range(n_kv):
            key = self._read_str()
            (t,) = self._unpack("<I")
            self.kv[key] = self._read_value(t)
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._read_str()
            (nd,) = self._unpack("<I")
            dims = self._unpack("<" + "Q" * nd)
            gtype, off = self._unpack("<IQ")
            shape = tuple(reversed(dims))
            self.tensors[name] = GGUFInfo(name, gtype, shape, off,
                                          tensor_nbytes(gtype, int(np.prod(shape))))
        align = int(self.kv.get("general.alignment", 32)) or 32
        self.data_offset = (self.pos + align - 1) // align * align
        for ti in self.tensors.values():
            if self.data_offset + ti.offset + ti.nbytes > len(self.buf):
                raise ValueError(f"tensor {ti.name} exceeds file bounds")

    def _unpack(self, fmt):
        n = struct.calcsize(fmt)
        if self.pos + n > len(self.buf):
            raise ValueError("unexpected end of GGUF header")
        v = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += n
        return v

    def _read_str(self):
        (n,) = self._unpack("<Q")
        if self.pos + n > len(self.buf):
            raise ValueError("string exceeds bounds")
        s = bytes(self.buf[self.pos:self.pos + n]).decode()
        self.pos += n
        return s

    def _read_value(self, t):
        if t == _KV_STR:
            return self._read_str()
        if t == _KV_ARR:
            at, n = self._unpack("<IQ")
            return [self._read_value(at) for _ in range(n)]
        if t not in _SCALAR:
            raise ValueError(f"unknown GGUF metadata type {t}")
        return self._unpack(_SCALAR[t])[0]

    def raw(self, name: str) -> np.ndarray:
        ti = self.tensors[name]
        o = self.data_offset + ti.offset
        return self.buf[o:o + ti.nbytes]
