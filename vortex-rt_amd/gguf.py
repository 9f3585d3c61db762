"""GGUF v2/v3 reader and writer (host side).

The reader mirrors ``GgufFile`` of the reference (src/gguf.cpp:312-403 parse, :640-664
validate, :188-201 type layouts, :546-638 Q8_0 row dequant); it memory-maps the file so
a 285 MB model is never copied into Python objects. The writer produces files the
reference loader accepts: little-endian, ``general.alignment`` honoured, every tensor
offset aligned (src/gguf.cpp:640-664).
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF", src/gguf.cpp:14
MAX_STRING = 1 << 30     # src/gguf.cpp:15
MAX_ARRAY = 1 << 28      # src/gguf.cpp:16
MAX_DEPTH = 8            # src/gguf.cpp:17

# GgufValueType (include/vortexrt/gguf.hpp:14-28)
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
               T_F32: "<f", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}

# ggml tensor types with (block elements, block bytes), src/gguf.cpp:188-201
GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
TYPE_LAYOUT = {0: (1, 4), 1: (1, 2), 8: (32, 34), 24: (1, 1), 25: (1, 2), 26: (1, 4),
               27: (1, 8), 28: (1, 8), 30: (1, 2)}


class GgufError(RuntimeError):
    pass


@dataclass
class TensorInfo:
    name: str
    dims: list
    type: int
    offset: int

    def nbytes(self) -> int | None:
        lay = TYPE_LAYOUT.get(self.type)
        if lay is None:
            return None
        elems = 1
        for d in self.dims:
            if d == 0:
                return 0
            elems *= d
        if elems % lay[0]:
            raise GgufError("GGUF tensor element count is not divisible by quant block size")
        return elems // lay[0] * lay[1]


@dataclass
class GgufFile:
    path: str
    version: int = 0
    file_size: int = 0
    data_offset: int = 0
    alignment: int = 32
    metadata: dict = field(default_factory=dict)       # key -> (type, value)
    tensors: dict = field(default_factory=dict)        # name -> TensorInfo
    _mm: object = None

    @classmethod
    def open(cls, path: str) -> "GgufFile":
        f = cls(path=str(path))
        with open(path, "rb") as fp:
            f._mm = mmap.mmap(fp.fileno(), 0, access=mmap.ACCESS_READ)
        f.file_size = len(f._mm)
        f._parse()
        return f

    # -- parsing --------------------------------------------------------------------
    def _parse(self):
        mm, pos = self._mm, 0

        def take(n):
            nonlocal pos
            if n > self.file_size - pos:
                raise GgufError("Unexpected end of GGUF file")
            b = mm[pos:pos + n]
            pos += n
            return b

        def pod(fmt):
            return struct.unpack(fmt, take(struct.calcsize(fmt)))[0]

        def string():
            n = pod("<Q")
            if n > MAX_STRING:
                raise GgufError("GGUF string length exceeds safety limit")
            return take(n).decode("utf-8", errors="surrogateescape")

        def value(t, depth):
            if t in _SCALAR_FMT:
                return pod(_SCALAR_FMT[t])
            if t == T_BOOL:
                v = pod("<B")
                if v > 1:
                    raise GgufError("GGUF boolean value is not 0/1")
                return bool(v)
            if t == T_STR:
                return string()
            if t == T_ARR:
                if depth >= MAX_DEPTH:
                    raise GgufError("GGUF array nesting is too deep")
                et = pod("<I")
                if et > T_F64:
                    raise GgufError("GGUF array has invalid element type")
                n = pod("<Q")
                if n > MAX_ARRAY:
                    raise GgufError("GGUF array length exceeds safety limit")
                if et in _SCALAR_FMT:  # bulk decode numeric arrays
                    sz = struct.calcsize(_SCALAR_FMT[et])
                    arr = np.frombuffer(take(n * sz), dtype=np.dtype(_SCALAR_FMT[et]))
                    return (et, arr)
                return (et, [value(et, depth + 1) for _ in range(n)])
            raise GgufError("GGUF metadata has invalid value type")

        if pod("<I") != GGUF_MAGIC:
            raise GgufError("Invalid GGUF magic")
        self.version = pod("<I")
        if self.version < 2 or self.version > 3:
            raise GgufError(f"Unsupported GGUF version: {self.version}")
        n_tensors, n_kv = pod("<Q"), pod("<Q")
        if n_tensors > 1_000_000 or n_kv > 1_000_000:
            raise GgufError("GGUF header counts exceed safety limits")
        for _ in range(n_kv):
            key = string()
            t = pod("<I")
            if t > T_F64:
                raise GgufError("GGUF metadata has invalid value type")
            v = value(t, 0)
            self.metadata.setdefault(key, (t, v))
        al = self.metadata.get("general.alignment")
        if al is not None:
            a = self.as_u64(al)
            if a is None or a == 0 or a > 0xFFFFFFFF:
                raise GgufError("Invalid general.alignment metadata")
            self.alignment = a
        if self.alignment & (self.alignment - 1):
            raise GgufError("GGUF alignment must be a power of two")
        for _ in range(n_tensors):
            name = string()
            nd = pod("<I")
            if nd == 0 or nd > 8:
                raise GgufError("GGUF tensor has invalid dimension count")
            dims = [pod("<Q") for _ in range(nd)]
            ttype = pod("<I")
            off = pod("<Q")
            self.tensors.setdefault(name, TensorInfo(name, dims, ttype, off))
        self.data_offset = (pos + self.alignment - 1) // self.alignment * self.alignment
        self.validate()

    def validate(self):
        """src/gguf.cpp:640-664."""
        if self.data_offset > self.file_size:
            raise GgufError("GGUF tensor data offset lies beyond end of file")
        for t in self.tensors.values():
            if t.offset % self.alignment:
                raise GgufError(f"GGUF tensor offset is not aligned: {t.name}")
            if t.offset > self.file_size - self.data_offset:
                raise GgufError(f"GGUF tensor offset lies beyond end of file: {t.name}")
            nb = t.nbytes()
            if nb is not None and nb > self.file_size - self.data_offset - t.offset:
                raise GgufError(f"GGUF tensor payload lies beyond end of file: {t.name}")

    # -- typed accessors (GgufValue::as_*, src/gguf.cpp:266-310) ------------------------
    @staticmethod
    def as_u64(tv):
        t, v = tv
        if t in (T_U8, T_U16, T_U32, T_U64):
            return int(v)
        if t in (T_I8, T_I16, T_I32, T_I64) and v >= 0:
            return int(v)
        return None

    @staticmethod
    def as_f64(tv):
        t, v = tv
        return float(v) if t in (T_F32, T_F64) else None

    def meta_u64(self, key):
        tv = self.metadata.get(key)
        return None if tv is None else self.as_u64(tv)

    def meta_f64(self, key):
        tv = self.metadata.get(key)
        return None if tv is None else self.as_f64(tv)

    def meta_str(self, key):
        tv = self.metadata.get(key)
        return tv[1] if tv is not None and tv[0] == T_STR else None

    def meta_array_len(self, key):
        tv = self.metadata.get(key)
        if tv is None or tv[0] != T_ARR:
            return None
        return len(tv[1][1])

    # -- payload ----------------------------------------------------------------------
    def data_view(self) -> memoryview:
        """The tensor-data section [data_offset, EOF): the device arena's byte image."""
        return memoryview(self._mm)[self.data_offset:]

    def tensor_bytes(self, name) -> np.ndarray:
        t = self.tensors[name]
        nb = t.nbytes()
        if nb is None:
            raise GgufError(f"Unsupported GGML tensor type for payload read: {name}")
        start = self.data_offset + t.offset
        return np.frombuffer(self._mm, dtype=np.uint8, count=nb, offset=start)

    def read_f32(self, name) -> np.ndarray:
        t = self.tensors[name]
        if t.type != GGML_F32:
            raise GgufError(f"Expected F32 tensor: {name}")
        return self.tensor_bytes(name).view(np.float32).copy()

    def close(self):
        """Unmaps the file; arrays still viewing the payload keep the map alive until they go."""
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass
            self._mm = None


class GgufWriter:
    """Streams a GGUF v3 file: metadata, tensor directory, then aligned payloads."""

    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self.kv = []          # (key, type, value)
        self.tensors = []     # (name, dims, type, nbytes, producer)

    def add(self, key, t, value):
        self.kv.append((key, t, value))

    def add_tensor(self, name, dims, ttype, nbytes, producer):
        """producer() returns the payload when written: bytes, a numpy array, or an iterable of them."""
        self.tensors.append((name, list(dims), ttype, nbytes, producer))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _value(self, t, v) -> bytes:
        if t in _SCALAR_FMT:
            return struct.pack(_SCALAR_FMT[t], v)
        if t == T_BOOL:
            return struct.pack("<B", 1 if v else 0)
        if t == T_STR:
            return self._str(v)
        if t == T_ARR:
            et, items = v
            head = struct.pack("<IQ", et, len(items))
            if et in _SCALAR_FMT:
                return head + np.asarray(items, dtype=np.dtype(_SCALAR_FMT[et])).tobytes()
            return head + b"".join(self._value(et, x) for x in items)
        raise GgufError(f"bad metadata type {t}")

    def write(self, path):
        al = self.alignment
        offsets, cur = [], 0
        for (_, _, _, nbytes, _) in self.tensors:
            offsets.append(cur)
            cur = (cur + nbytes + al - 1) // al * al
        head = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kv)))
        for key, t, v in self.kv:
            head += self._str(key) + struct.pack("<I", t) + self._value(t, v)
        for (name, dims, ttype, _, _), off in zip(self.tensors, offsets):
            head += self._str(name) + struct.pack("<I", len(dims))
            head += b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", ttype, off)
        pad = (-len(head)) % al
        tmp = str(path) + ".tmp"
        with open(tmp, "wb") as fp:
            fp.write(head)
            fp.write(b"\0" * pad)
            pos = 0
            for (name, _, _, nbytes, producer), off in zip(self.tensors, offsets):
                if off > pos:
                    fp.write(b"\0" * (off - pos))
                    pos = off
                payload = producer()
                parts = payload if not isinstance(payload, (np.ndarray, bytes, bytearray)) else [payload]
                written = 0
                for part in parts:
                    b = part.tobytes() if isinstance(part, np.ndarray) else bytes(part)
                    fp.write(b)
                    written += len(b)
                if written != nbytes:
                    raise GgufError(f"tensor {name}: {written} bytes, expected {nbytes}")
                pos += nbytes
        os.replace(tmp, path)
