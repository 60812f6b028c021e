"""GGUF reading and the model inspector (no GPU): round trips through the
package's writer, the expert-layout proof and every refusal."""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from gguf_models import ARCH, write_model
from sabah.runtime import gguf, model


def test_round_trip_of_metadata_and_tensors(tmp_path):
    p = str(tmp_path / "m.gguf")
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.arange(34 * 3, dtype=np.uint8)                         # three Q8_0 blocks
    kv = [("general.architecture", gguf.STR, "x"), ("u", gguf.U32, 7), ("f", gguf.F32, 1.5),
          ("flag", gguf.BOOL, True), ("big", gguf.U64, 1 << 40), ("neg", gguf.I64, -5), ("d", gguf.F64, 0.25),
          ("arr", gguf.ARR, (gguf.I32, [1, -2, 3])), ("names", gguf.ARR, (gguf.STR, ["a", "bc"]))]
    gguf.write_gguf(p, kv, [gguf.WriterTensor("t.a", (4, 3), 0, a), gguf.WriterTensor("t.b", (96,), 8, b)])
    f = gguf.GgufFile(p)
    try:
        assert f.version == 3 and f.alignment == 32
        assert f.kv["u"] == 7 and f.kv["f"] == 1.5 and f.kv["flag"] is True and f.kv["big"] == 1 << 40
        assert f.kv["neg"] == -5 and f.kv["d"] == 0.25 and f.kv["names"] == ["a", "bc"]
        assert f.kv["arr"].tolist() == [1, -2, 3] and f.kv_types["arr"] == gguf.ARR
        ta, tb = f.tensors["t.a"], f.tensors["t.b"]
        assert ta.shape == (4, 3) and ta.ggml_type == 0 and ta.n_bytes == 48 and ta.data_offset % 32 == 0
        assert tb.type_name == "Q8_0" and tb.n_bytes == 102 and tb.offset % 32 == 0
        assert np.array_equal(f.data("t.a").view(np.float32).reshape(3, 4), a)
        assert np.array_equal(f.data("t.b"), b)
    finally:
        f.close()


def test_rejects_what_is_not_a_gguf(tmp_path):
    p = str(tmp_path / "bad.gguf")
    with open(p, "wb") as fh:
        fh.write(b"GGML" + b"\0" * 40)
    with pytest.raises(gguf.GgufError, match="magic"):
        gguf.GgufFile(p)
    with open(p, "wb") as fh:
        fh.write(b"GGUF" + struct.pack("<IQQ", 9, 0, 0))
    with pytest.raises(gguf.GgufError, match="version"):
        gguf.GgufFile(p)
    # a tensor table that points past the end of the file
    q = str(tmp_path / "short.gguf")
    gguf.write_gguf(q, [], [gguf.WriterTensor("t", (64,), 0, np.zeros(64, np.float32))])
    with open(q, "r+b") as fh:
        fh.truncate(os.path.getsize(q) - 8)
    with pytest.raises(gguf.GgufError, match="past the end"):
        gguf.GgufFile(q)


def test_inspector_accepts_the_shipped_iq_mix(tmp_path, orc):
    """IQ3_XXS gate/up with IQ4_NL down (the reference's shipped blocks), IQ4_XS
    and IQ2_S layers are decodable; the per-expert sizes follow their blocks
    (98 B per 256, 18 B per 32, 136 B per 256, 82 B per 256)."""
    p = str(tmp_path / "iq.gguf")
    rng = np.random.default_rng(3)
    write_model(p, orc, rng, n_layers=3, E=4, D=512, F=256, layer_types=[(18, 18, 20), (23, 23, 23), (22, 22, 21)])
    prof = model.inspect_model(p)
    assert prof.supported, prof.notes
    assert prof.experts[(2, "gate")].per_expert_bytes == 256 * 2 * 82
    assert prof.experts[(0, "gate")].per_expert_bytes == 256 * 2 * 98
    assert prof.experts[(0, "down")].per_expert_bytes == 512 * 8 * 18
    assert prof.experts[(1, "up")].per_expert_bytes == 256 * 2 * 136


def test_inspector_profiles_a_supported_model(tmp_path, orc):
    p = str(tmp_path / "m.gguf")
    rng = np.random.default_rng(1)
    write_model(p, orc, rng, n_layers=2, E=8, D=512, F=256, layer_types=[(21, 21, 21), (12, 12, 14)], Fs=256,
                gate_inp_shexp=True)
    prof = model.inspect_model(p)
    assert prof.supported, prof.notes
    assert (prof.architecture, prof.n_layers, prof.d_model, prof.n_experts, prof.n_used, prof.expert_ff) == \
        (ARCH, 2, 512, 8, 4, 256)
    assert prof.layers == [0, 1]
    g0, d1 = prof.experts[(0, "gate")], prof.experts[(1, "down")]
    assert g0.ggml_type == 21 and g0.shape == (512, 256, 8) and g0.per_expert_bytes == 256 * 2 * 110
    assert d1.ggml_type == 14 and d1.per_expert_bytes == 512 * 210
    assert prof.expert_bank_bytes == sum(t.per_expert_bytes * 8 for t in prof.experts.values())
    assert prof.per_token_expert_bytes() == sum(t.per_expert_bytes for t in prof.experts.values()) * 4
    assert set(prof.shared) == {(l, r) for l in (0, 1) for r in ("gate", "up", "down")}
    assert set(prof.router) == {0, 1} and set(prof.shared_gate_inp) == {0, 1}
    f = gguf.GgufFile(p)
    try:       # the recorded byte range is the tensor's bytes in the file
        assert f.tensors[g0.name].data_offset == g0.data_offset and f.tensors[g0.name].n_bytes == g0.n_bytes
    finally:
        f.close()


def test_inspector_finds_layers_across_shards(tmp_path, orc):
    rng = np.random.default_rng(2)
    base = str(tmp_path / "m")
    for i, layers in enumerate(([0], [1, 2])):
        write_model("%s-%05d-of-00002.gguf" % (base, i + 1), orc, rng, n_layers=3, E=4, D=256, F=256, layers=layers)
    prof = model.inspect_model(base + "-00001-of-00002.gguf")
    assert prof.supported, prof.notes
    assert prof.layers == [0, 1, 2] and len(prof.shards) == 2
    assert prof.experts[(0, "up")].shard == 0 and prof.experts[(2, "down")].shard == 1


@pytest.mark.parametrize("case,needle", [("arch", "not registered"), ("geometry", "geometry"),
                                          ("type", "not decoded"), ("mixed", "differ in type"),
                                          ("missing", "has no down"), ("axis", "slowest")])
def test_inspector_refuses(tmp_path, orc, case, needle):
    p = str(tmp_path / "m.gguf")
    rng = np.random.default_rng(3)
    E, D, F = 4, 256, 256
    if case == "arch":
        gguf.write_gguf(p, [("general.architecture", gguf.STR, "llama")], [])
    elif case == "geometry":
        gguf.write_gguf(p, [("general.architecture", gguf.STR, ARCH)], [])
    elif case == "mixed":
        write_model(p, orc, rng, n_layers=1, E=E, D=D, F=F, layer_types=[(21, 12, 21)])
    else:
        kv = [("general.architecture", gguf.STR, ARCH), ("%s.block_count" % ARCH, gguf.U32, 1),
              ("%s.embedding_length" % ARCH, gguf.U32, D), ("%s.expert_count" % ARCH, gguf.U32, E),
              ("%s.expert_used_count" % ARCH, gguf.U32, 2), ("%s.expert_feed_forward_length" % ARCH, gguf.U32, F)]
        def t(role, qt, shape):
            n = gguf.tensor_bytes(qt, shape)
            return gguf.WriterTensor("blk.0.ffn_%s_exps.weight" % role, shape, qt, np.zeros(n, np.uint8))
        ts = [t("gate", 21, (D, F, E)), t("up", 21, (D, F, E))]
        if case == "type":
            ts.append(t("down", 6, (F, D, E)))              # Q5_0: a GGUF type the kernels do not decode
        elif case == "axis":
            ts.append(t("down", 21, (F, E, D)))             # experts not the slowest axis
        gguf.write_gguf(p, kv, ts)
    prof = model.inspect_model(p)
    assert not prof.supported
    assert any(needle in n for n in prof.notes), prof.notes
    with pytest.raises(model.UnsupportedModel):
        model.load_expert_bank(prof, device="cpu")


def test_inspector_accepts_q2_0_experts(tmp_path, orc):
    """The artifact's Q2_0 experts (ggml type 42, 64-element blocks of 18 B)
    inspect as supported, with their per-expert bytes from the type's geometry."""
    p = str(tmp_path / "m.gguf")
    rng = np.random.default_rng(4)
    E, D, F = 4, 256, 192
    write_model(p, orc, rng, n_layers=1, E=E, D=D, F=F, layer_types=[(42, 42, 42)])
    prof = model.inspect_model(p)
    assert prof.supported, prof.notes
    assert prof.experts[(0, "gate")].ggml_type == 42
    assert prof.experts[(0, "down")].per_expert_bytes == D * (F // 64) * 18
