"""Writes hand_built_v3.gguf, a GGUF file assembled byte by byte from the layout
that integration/llama.cpp/ggml/include/gguf.h:1-30 documents (magic, version,
int64 tensor and KV counts, KV pairs with u32 value types, tensor infos with
int64 extents, the data blob aligned to general.alignment), with struct.pack
only: no GGUF writer is involved, so the reader under test is checked against
the format, not against its own writer.

    python make_gguf_fixture.py      rewrite the fixture beside this script
"""
from __future__ import annotations

import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "hand_built_v3.gguf")

# gguf_type (gguf.h:53-67)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
ALIGN = 64


def s(text: str) -> bytes:                      # u64 length, bytes, no terminator
    b = text.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def kv(key: str, vt: int, payload: bytes) -> bytes:
    return s(key) + struct.pack("<I", vt) + payload


def arr(et: int, items: list, fmt: str | None) -> bytes:
    body = b"".join(s(x) for x in items) if et == STR else b"".join(struct.pack(fmt, x) for x in items)
    return struct.pack("<IQ", et, len(items)) + body


KVS = [
    kv("general.architecture", STR, s("qwen4exp")),
    kv("general.alignment", U32, struct.pack("<I", ALIGN)),
    kv("t.u8", U8, struct.pack("<B", 250)),
    kv("t.i8", I8, struct.pack("<b", -7)),
    kv("t.u16", U16, struct.pack("<H", 65000)),
    kv("t.i16", I16, struct.pack("<h", -30000)),
    kv("t.i32", I32, struct.pack("<i", -123456789)),
    kv("t.f32", F32, struct.pack("<f", 0.15625)),
    kv("t.bool", BOOL, struct.pack("<b", 1)),
    kv("t.u64", U64, struct.pack("<Q", 2 ** 40 + 3)),
    kv("t.i64", I64, struct.pack("<q", -(2 ** 40))),
    kv("t.f64", F64, struct.pack("<d", -2.5e-300)),
    kv("t.utf8", STR, s("Schlüssel ✓")),
    kv("t.arr_u8", ARR, arr(U8, [1, 2, 255], "<B")),
    kv("t.arr_i64", ARR, arr(I64, [-1, 2 ** 62], "<q")),
    kv("t.arr_f64", ARR, arr(F64, [0.5, -0.25], "<d")),
    kv("t.arr_str", ARR, arr(STR, ["a", "", "blk.0"], None)),
    kv("t.arr_bool", ARR, arr(BOOL, [1, 0, 1], "<b")),
    kv("t.arr_empty", ARR, arr(U32, [], "<I")),
]

# (name, ne, ggml_type, bytes, offset in the blob): listed out of offset order,
# each offset a multiple of ALIGN, the IQ3_S tensor 2 x 3 rows of one block,
# the Q2_0 tensor 2 rows of two 64-element blocks, the f32 tensor 5 values
TENSORS = [
    ("blk.0.ffn_down_exps.weight", (128, 2), 42, 2 * 2 * 18, 2 * ALIGN * 11),
    ("blk.0.ffn_gate_exps.weight", (256, 2, 3), 21, 6 * 110, 0),
    ("blk.0.ffn_gate_inp.weight", (5,), 0, 20, ALIGN * 11),
]


def tensor_bytes(i: int, n: int) -> bytes:
    return bytes((37 * i + 11 * j + 5) % 256 for j in range(n))


def build() -> bytes:
    head = b"GGUF" + struct.pack("<Iqq", 3, len(TENSORS), len(KVS)) + b"".join(KVS)
    for name, ne, gt, _, off in TENSORS:
        head += s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<q", d) for d in ne)
        head += struct.pack("<IQ", gt, off)
    data_start = (len(head) + ALIGN - 1) // ALIGN * ALIGN
    end = max(off + n for _, _, _, n, off in TENSORS)
    blob = bytearray(b"\xee" * end)               # padding bytes no tensor owns
    for i, (_, _, _, n, off) in enumerate(TENSORS):
        blob[off:off + n] = tensor_bytes(i, n)
    return head + b"\x00" * (data_start - len(head)) + bytes(blob)


if __name__ == "__main__":
    with open(PATH, "wb") as f:
        f.write(build())
