"""A GGUF model file into HBM and through the runtime (needs an MI355X): the
loaded bank is the file's bytes, its layers match the oracle on those bytes,
and the drop-in entry point accepts the host mmap addresses llama.cpp would
pass as src0->data."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gguf_models import write_model
from helpers import assert_parity

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(scope="module")
def gguf_model(tmp_path_factory, orc):
    p = str(tmp_path_factory.mktemp("gguf") / "m.gguf")
    rng = np.random.default_rng(41)
    # layer 2: the quant mix of the reference's shipped blocks (IQ3_XXS gate/up, IQ4_NL down);
    # layer 3: IQ2_S gate/up (another of the artifact's expert types) with IQ4_XS down;
    # layer 4: Q2_0 (ggml type 42), the artifact's last expert type
    raws, shared = write_model(p, orc, rng, n_layers=5, E=16, D=1024, F=512, n_used=4,
                               layer_types=[(21, 21, 21), (12, 12, 14), (18, 18, 20), (22, 22, 23), (42, 42, 42)],
                               Fs=256,
                               gate_inp_shexp=True)
    return p, raws, shared


def test_loaded_bank_is_the_file_and_runs_its_layers(hip_rt, orc, gguf_model):
    from sabah.runtime import model, routing
    from sabah.runtime.executor import MoEExecutor
    path, raws, shared = gguf_model
    prof = model.inspect_model(path)
    assert prof.supported, prof.notes
    bank = model.load_expert_bank(prof, "cuda:0", verify=True)
    rng = np.random.default_rng(42)
    for l in (0, 1, 2, 3, 4):
        for r in ("gate", "up", "down"):
            assert np.array_equal(bank.tensor(l, r).cpu().numpy().reshape(raws[(l, r)].shape), raws[(l, r)])
        sh = model.load_shared_expert(prof, l)
        ex = MoEExecutor(bank, max_used=4, shared=sh)
        ids, w = routing.uniform_routing(rng, 5, 16, 4)
        x = rng.standard_normal((5, 1024)).astype(np.float32)
        got = ex.run_layer(l, T(x), T(ids), T(w)).cpu().numpy()
        qts = tuple(prof.experts[(l, r)].ggml_type for r in ("gate", "up", "down"))
        want = orc.moe_layer(raws[(l, "gate")], raws[(l, "up")], raws[(l, "down")], qts, x, ids, w,
                             shared=(shared[(l, "gate")], shared[(l, "up")], shared[(l, "down")], (8, 8, 8),
                                     shared[(l, "gate_inp")]))
        assert_parity(got, want, "GGUF layer %d" % l)


def test_drop_in_call_with_the_file_mapping_address(hip_rt, orc, gguf_model):
    from sabah.runtime import model, routing
    from sabah.runtime.executor import MoEExecutor
    path, raws, _ = gguf_model
    prof = model.inspect_model(path)
    bank = model.load_expert_bank(prof, "cuda:0")
    files = model.register_file_keys(bank, prof)
    try:
        ex = MoEExecutor(bank, max_used=4)
        rng = np.random.default_rng(43)
        ids, _ = routing.uniform_routing(rng, 3, 16, 4)
        x = rng.standard_normal((3, 1, 1024)).astype(np.float32)
        for l in (0, 1, 2, 3, 4):
            ref = prof.experts[(l, "gate")]
            key = files[ref.shard].base_address() + ref.data_offset
            via_key = ex.mul_mat_id(l, "gate", T(x), T(ids), source=key)
            direct = ex.mul_mat_id(l, "gate", T(x), T(ids))
            torch.cuda.synchronize()
            assert torch.equal(via_key, direct)
            want = orc.mul_mat_id(raws[(l, "gate")], x, ids, 512, 1024, ref.ggml_type)
            assert_parity(via_key.cpu().numpy(), want, "MUL_MAT_ID through the file key, layer %d" % l)
    finally:
        bank.unregister()
        for f in files:
            f.close()


def test_verify_checksum_sees_a_flipped_bit(hip_rt, gguf_model):
    from sabah.runtime import gguf, model
    path, _, _ = gguf_model
    prof = model.inspect_model(path)
    bank = model.load_expert_bank(prof, "cuda:0", layers=[1])
    ref = prof.experts[(1, "down")]
    f = gguf.GgufFile(path)
    try:
        src = f.data(ref.name)
        n4 = src.size // 4 * 4
        host = model._checksum(src[:n4].view(np.int32))
        dst = bank.tensor(0, "down").view(-1)
        assert model._checksum_dev(dst[:n4]) == host
        dst[12345] ^= 1
        assert model._checksum_dev(dst[:n4]) != host
    finally:
        f.close()
