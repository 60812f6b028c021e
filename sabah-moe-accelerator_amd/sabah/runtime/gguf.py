"""
Sabah / runtime / gguf

A GGUF (v2/v3) reader and writer: the header, the typed key/value metadata,
the tensor table (name, dims with ne[0] fastest, ggml type, offset into the
aligned data section), and absolute byte ranges of every tensor in the file.
The file is memory-mapped read-only and never modified.

Format (gguf.h / gguf.cpp of the pinned llama.cpp; the reference reads it
through gguf-py, sabah/core/model_inspector.py:146-199): little-endian
"GGUF", u32 version, u64 tensor count, u64 kv count; each kv is a string key,
a u32 value type and the value (arrays carry a u32 element type and a u64
count); each tensor info is a string name, u32 n_dims, n_dims u64 extents,
u32 ggml type and a u64 offset relative to the data section, which starts at
the next multiple of general.alignment (default 32) after the tensor table.
Strings are a u64 length and that many UTF-8 bytes.
"""
from __future__ import annotations

import mmap
import os
import re
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}

# ggml type code -> (name, elements per block, bytes per block)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 42: ("Q2_0", 64, 18),
}
GGML_TYPE_CODE = {v[0]: k for k, v in GGML_TYPES.items()}


class GgufError(Exception):
    """The file is not a GGUF this reader understands."""


@dataclass
class TensorInfo:
    name: str
    shape: tuple            # ne[0] (fastest) first, as GGUF stores it
    ggml_type: int
    offset: int             # relative to the data section
    data_offset: int = 0    # absolute file offset
    n_bytes: int = 0

    @property
    def type_name(self) -> str:
        return GGML_TYPES.get(self.ggml_type, ("type%d" % self.ggml_type,))[0]

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


def tensor_bytes(ggml_type: int, shape) -> int:
    """Bytes of a tensor of `shape` (ne[0] first); rows must be whole blocks."""
    if ggml_type not in GGML_TYPES:
        raise GgufError("unknown ggml type %d" % ggml_type)
    _, be, bb = GGML_TYPES[ggml_type]
    if shape[0] % be:
        raise GgufError("ne[0] = %d is not a whole number of %d-element blocks" % (shape[0], be))
    n = shape[0] // be * bb
    for d in shape[1:]:
        n *= d
    return n


class _Cursor:
    def __init__(self, buf, pos=0):
        self.buf, self.pos = buf, pos

    def take(self, fmt):
        if self.pos + struct.calcsize(fmt) > len(self.buf):
            raise GgufError("the header runs past the end of the file at byte %d" % self.pos)
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        if n > len(self.buf) - self.pos:
            raise GgufError("string of %d bytes runs past the end of the file" % n)
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vt):
        if vt in _SCALAR:
            return self.take(_SCALAR[vt])
        if vt == STR:
            return self.string()
        if vt == ARR:
            et, n = self.take("<I"), self.take("<Q")
            if et in _SCALAR and et != BOOL:
                dt = np.dtype(_SCALAR[et])
                a = np.frombuffer(self.buf, dtype=dt, count=n, offset=self.pos).copy()
                self.pos += n * dt.itemsize
                return a
            return [self.value(et) for _ in range(n)]
        raise GgufError("unknown value type %d" % vt)


class GgufFile:
    """One GGUF file, memory-mapped read-only: .version, .kv (key -> value),
    .kv_types (key -> value type), .tensors (name -> TensorInfo in file order),
    .alignment, .data_start."""

    def __init__(self, path: str):
        self.path = os.path.abspath(path)
        self._f = open(path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if size < 24:
            self._f.close()
            raise GgufError("%s: too short for a GGUF header" % path)
        self.mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse(path, size)
        except Exception:
            self.close()
            raise

    def _parse(self, path: str, size: int) -> None:
        c = _Cursor(self.mm)
        if bytes(self.mm[:4]) != GGUF_MAGIC:
            raise GgufError("%s: bad magic %r" % (path, bytes(self.mm[:4])))
        c.pos = 4
        self.version = c.take("<I")
        if self.version not in (2, 3):
            raise GgufError("%s: GGUF version %d is not supported (2 and 3 are)" % (path, self.version))
        n_tensors, n_kv = c.take("<Q"), c.take("<Q")
        self.kv, self.kv_types = {}, {}
        for _ in range(n_kv):
            k = c.string()
            vt = c.take("<I")
            self.kv[k] = c.value(vt)
            self.kv_types[k] = vt
        self.tensors = {}
        for _ in range(n_tensors):
            name = c.string()
            nd = c.take("<I")
            shape = tuple(c.take("<Q") for _ in range(nd))
            t = TensorInfo(name, shape, c.take("<I"), c.take("<Q"))
            self.tensors[name] = t
        self.alignment = int(self.kv.get("general.alignment", DEFAULT_ALIGNMENT))
        self.data_start = (c.pos + self.alignment - 1) // self.alignment * self.alignment
        for t in self.tensors.values():
            t.data_offset = self.data_start + t.offset
            t.n_bytes = tensor_bytes(t.ggml_type, t.shape) if t.ggml_type in GGML_TYPES else 0
            if t.n_bytes and t.data_offset + t.n_bytes > size:
                raise GgufError("%s: tensor %s runs past the end of the file" % (path, t.name))

    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        t = self.tensors[name]
        return np.frombuffer(self.mm, dtype=np.uint8, count=t.n_bytes, offset=t.data_offset)

    def base_address(self) -> int:
        """Host address of the mapping's first byte (a tensor's bytes start at
        base_address() + data_offset, as llama.cpp's mmap'd src0->data does)."""
        return np.frombuffer(self.mm, dtype=np.uint8, count=1).ctypes.data

    def close(self) -> None:
        try:
            self.mm.close()
        except BufferError:
            pass                # a view is still alive; the mapping closes with it
        self._f.close()


def shard_paths(path: str) -> list:
    """All shards of a split GGUF (...-00001-of-000NN.gguf), or [path]."""
    m = re.search(r"-(\d{5})-of-(\d{5})\.gguf$", path)
    if not m:
        return [path]
    n = int(m.group(2))
    base = path[:m.start()]
    return ["%s-%05d-of-%05d.gguf" % (base, i, n) for i in range(1, n + 1)]


# ---------------------------------------------------------------------------
# writer (synthetic model files for tests and tools)
# ---------------------------------------------------------------------------
def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(vt: int, v) -> bytes:
    if vt in _SCALAR:
        return struct.pack(_SCALAR[vt], v)
    if vt == STR:
        return _pack_string(v)
    raise GgufError("write: value type %d needs write_gguf's (type, values) form" % vt)


@dataclass
class WriterTensor:
    name: str
    shape: tuple            # ne[0] first
    ggml_type: int
    data: np.ndarray        # raw bytes, tensor_bytes(ggml_type, shape) of them


def write_gguf(path: str, kv: list, tensors: list, alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """kv: list of (key, value type, value); an array value is (ARR, (elem type, list)).
    tensors: list of WriterTensor, laid out in order at aligned offsets."""
    out = bytearray(GGUF_MAGIC)
    out += struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vt, v in kv:
        out += _pack_string(key) + struct.pack("<I", vt)
        if vt == ARR:
            et, items = v
            out += struct.pack("<IQ", et, len(items))
            for it in items:
                out += _pack_value(et, it)
        else:
            out += _pack_value(vt, v)
    offs, off = [], 0
    for t in tensors:
        n = tensor_bytes(t.ggml_type, t.shape)
        if np.asarray(t.data).nbytes != n:
            raise GgufError("tensor %s: %d bytes given, %d expected" % (t.name, np.asarray(t.data).nbytes, n))
        offs.append(off)
        off = (off + n + alignment - 1) // alignment * alignment
    for t, o in zip(tensors, offs):
        out += _pack_string(t.name) + struct.pack("<I", len(t.shape))
        out += b"".join(struct.pack("<Q", d) for d in t.shape)
        out += struct.pack("<IQ", t.ggml_type, o)
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    with open(path, "wb") as f:
        f.write(out)
        pos = 0
        for t, o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            b = np.ascontiguousarray(t.data).view(np.uint8).tobytes()
            f.write(b)
            pos = o + len(b)
