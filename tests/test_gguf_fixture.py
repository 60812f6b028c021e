"""The GGUF reader (sabah/runtime/gguf.py) against tests/golden/hand_built_v3.gguf,
a file assembled with struct.pack from gguf.h's documented layout
(tests/golden/make_gguf_fixture.py), not by the package's writer: every value
type, arrays of each kind, UTF-8 text, a non-default alignment, tensor infos
listed out of offset order, and padding bytes no tensor owns."""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import pytest

from sabah.runtime import gguf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURE = os.path.join(GOLDEN, "hand_built_v3.gguf")


def fixture_module():
    sys.path.insert(0, GOLDEN)
    try:
        import make_gguf_fixture
        return make_gguf_fixture
    finally:
        sys.path.remove(GOLDEN)


def test_fixture_is_what_its_script_writes():
    assert open(FIXTURE, "rb").read() == fixture_module().build()


def test_header_and_every_value_type():
    f = gguf.GgufFile(FIXTURE)
    try:
        assert f.version == 3 and f.alignment == 64
        kv = f.kv
        assert kv["general.architecture"] == "qwen4exp"
        assert kv["t.u8"] == 250 and kv["t.i8"] == -7 and kv["t.u16"] == 65000 and kv["t.i16"] == -30000
        assert kv["t.i32"] == -123456789 and kv["t.f32"] == 0.15625 and kv["t.bool"] in (1, True)
        assert kv["t.u64"] == 2 ** 40 + 3 and kv["t.i64"] == -(2 ** 40) and kv["t.f64"] == -2.5e-300
        assert kv["t.utf8"] == "Schlüssel ✓"
        assert list(kv["t.arr_u8"]) == [1, 2, 255]
        assert list(kv["t.arr_i64"]) == [-1, 2 ** 62]
        assert list(kv["t.arr_f64"]) == [0.5, -0.25]
        assert list(kv["t.arr_str"]) == ["a", "", "blk.0"]
        assert [bool(v) for v in kv["t.arr_bool"]] == [True, False, True]
        assert len(kv["t.arr_empty"]) == 0
        assert f.kv_types["t.f64"] == 12 and f.kv_types["t.arr_str"] == 9
        assert list(f.kv) == [k for k in f.kv]                       # file order kept
    finally:
        f.close()


def test_tensor_infos_offsets_and_bytes():
    mod = fixture_module()
    f = gguf.GgufFile(FIXTURE)
    try:
        assert list(f.tensors) == [t[0] for t in mod.TENSORS]
        size = os.path.getsize(FIXTURE)
        assert f.data_start % 64 == 0 and f.data_start < size
        for i, (name, ne, gt, nbytes, off) in enumerate(mod.TENSORS):
            t = f.tensors[name]
            assert t.shape == ne and t.ggml_type == gt and t.offset == off
            assert t.n_bytes == nbytes == gguf.tensor_bytes(gt, ne)
            assert t.data_offset == f.data_start + off
            assert bytes(f.data(name)) == mod.tensor_bytes(i, nbytes)
        assert f.tensors["blk.0.ffn_down_exps.weight"].type_name == "Q2_0"
        assert f.tensors["blk.0.ffn_gate_exps.weight"].type_name == "IQ3_S"
    finally:
        f.close()


def test_fixture_sha256_is_pinned():
    digest = hashlib.sha256(open(FIXTURE, "rb").read()).hexdigest()
    assert digest == "b804fd2e758071a137c700a69bc9d889361579ae8ba3faa236849cacc745353b"


@pytest.mark.parametrize("cut,needle", [(3, "too short"), (200, "header runs past the end"),
                                        (-10, "runs past the end of the file")])
def test_truncated_files_are_refused(tmp_path, cut, needle):
    data = open(FIXTURE, "rb").read()
    p = str(tmp_path / "t.gguf")
    open(p, "wb").write(data[:cut] if cut > 0 else data[:len(data) + cut])
    with pytest.raises(gguf.GgufError, match=needle):
        gguf.GgufFile(p).close()


def test_bad_magic_and_version_are_refused(tmp_path):
    data = bytearray(open(FIXTURE, "rb").read())
    p = str(tmp_path / "m.gguf")
    open(p, "wb").write(b"GGUX" + bytes(data[4:]))
    with pytest.raises(gguf.GgufError, match="bad magic"):
        gguf.GgufFile(p)
    data[4:8] = (1).to_bytes(4, "little")
    open(p, "wb").write(bytes(data))
    with pytest.raises(gguf.GgufError, match="version 1"):
        gguf.GgufFile(p)
