"""sabah_moe_layer_noalloc: the MoE layer with all of its device scratch in the
library's static array.  It allocates nothing, so its results must equal
sabah_moe_layer's bit for bit (the same kernels on the same inputs), on
consecutive calls that reuse the array with different sizes; the library's
grow-only scratch stays untouched; a call too large for the array fails
before enqueuing anything; and the call can be captured in a HIP graph at a
size no call has used before."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_parity

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K, IQ3_S = 8, 12, 14, 21
DEV = torch.device("cuda:0")


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def vp(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def layer_call(hip_rt, name, desc, x, ids, w, out, resid=None):
    fn = getattr(hip_rt.lib(), name)
    return fn(ctypes.byref(desc), vp(x), vp(ids), vp(w), ids.shape[1], ids.shape[0], vp(out), vp(resid),
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def make_layer(orc, rng, qts, E, D, F, Fs):
    from sabah.runtime.bank import DenseExpert, ExpertBank
    bank = ExpertBank(1, E, D, F, {"gate": qts[0], "up": qts[1], "down": qts[2]}, device="cuda:0")
    raws = {}
    for role, (rows, cols) in {"gate": (F, D), "up": (F, D), "down": (D, F)}.items():
        qt = qts[0] if role != "down" else qts[2]
        raws[role] = orc.quantize_weights(qt, (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32))
        bank.load(0, role, raws[role])
    shared = None
    if Fs:
        shared = DenseExpert(D, Fs, Q8_0, device="cuda:0")
        for role, (rows, cols) in {"gate": (Fs, D), "up": (Fs, D), "down": (D, Fs)}.items():
            raws["s_" + role] = orc.quantize_weights(Q8_0, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
            shared.load(role, raws["s_" + role])
    return bank, shared, raws


def inputs(rng, E, D, K, Tn):
    from sabah.runtime import routing
    ids, w = routing.zipf_routing(rng, Tn, E, K)
    return rng.standard_normal((Tn, D)).astype(np.float32), ids, w


@pytest.mark.parametrize("qts,Fs", [((IQ3_S, IQ3_S, IQ3_S), 512), ((Q4_K, Q4_K, Q6_K), 512), ((IQ3_S, IQ3_S, IQ3_S), 0)])
def test_noalloc_layer_equals_the_allocating_layer_on_two_calls(hip_rt, orc, qts, Fs):
    """Two calls in a row, the second smaller (8 tokens, then 1): each equals
    sabah_moe_layer on the same inputs bit for bit, and the library's
    grow-only scratch does not change while the no-alloc calls run."""
    rng = np.random.default_rng(sum(qts) + Fs)
    E, D, F, K = 48, 2048, 768, 10
    bank, shared, raws = make_layer(orc, rng, qts, E, D, F, Fs)
    desc = bank.layer_desc(0, shared)
    for Tn in (8, 1):
        x, ids, w = inputs(rng, E, D, K, Tn)
        xd, idd, wd = T(x), T(ids), T(w)
        resid = T(rng.standard_normal((Tn, D)).astype(np.float32))
        got = torch.full((Tn, D), float("nan"), dtype=torch.float32, device=DEV)
        before = hip_rt.snapshot()["scratch_bytes"]
        assert layer_call(hip_rt, "sabah_moe_layer_noalloc", desc, xd, idd, wd, got, resid) == 0, hip_rt.last_error()
        torch.cuda.synchronize()
        assert hip_rt.snapshot()["scratch_bytes"] == before
        want = torch.full((Tn, D), float("nan"), dtype=torch.float32, device=DEV)
        hip_rt.check(layer_call(hip_rt, "sabah_moe_layer", desc, xd, idd, wd, want, resid), "moe_layer")
        torch.cuda.synchronize()
        g, r = got.cpu().numpy(), want.cpu().numpy()
        assert np.isfinite(g).all()
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), "tokens=%d" % Tn
        if qts[0] == IQ3_S and Fs == 0:
            ref = orc.moe_layer(raws["gate"], raws["up"], raws["down"], qts, x, ids, w) + resid.cpu().numpy()
            assert_parity(g, ref, "noalloc layer vs oracle, tokens=%d" % Tn)


def test_noalloc_layer_larger_than_any_earlier_call_leaves_library_scratch_alone(hip_rt, orc):
    """64 tokens x top-10 with a shared expert (about 3.2 MB of scratch): the
    no-alloc call runs without growing the library's scratch; the allocating
    layer, run afterwards for the comparison, may grow it."""
    rng = np.random.default_rng(64)
    E, D, F, K, Tn = 64, 2048, 768, 10, 64
    bank, shared, _ = make_layer(orc, rng, (IQ3_S,) * 3, E, D, F, 512)
    desc = bank.layer_desc(0, shared)
    x, ids, w = inputs(rng, E, D, K, Tn)
    xd, idd, wd = T(x), T(ids), T(w)
    got = torch.empty((Tn, D), dtype=torch.float32, device=DEV)
    before = hip_rt.snapshot()["scratch_bytes"]
    assert layer_call(hip_rt, "sabah_moe_layer_noalloc", desc, xd, idd, wd, got) == 0, hip_rt.last_error()
    torch.cuda.synchronize()
    assert hip_rt.snapshot()["scratch_bytes"] == before
    want = torch.empty_like(got)
    hip_rt.check(layer_call(hip_rt, "sabah_moe_layer", desc, xd, idd, wd, want), "moe_layer")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_noalloc_layer_rejects_a_call_beyond_its_static_scratch(hip_rt, orc):
    """400 tokens x top-10 at d_ff 768 needs 12.3 MB of h: more than the 8 MiB
    array.  The call fails with a message naming the sizes and enqueues nothing."""
    rng = np.random.default_rng(400)
    E, D, F, K, Tn = 16, 512, 768, 10, 400
    bank, _, _ = make_layer(orc, rng, (IQ3_S,) * 3, E, D, F, 0)
    desc = bank.layer_desc(0, None)
    x, ids, w = inputs(rng, E, D, K, Tn)
    out = torch.full((Tn, D), 3.0, dtype=torch.float32, device=DEV)
    assert layer_call(hip_rt, "sabah_moe_layer_noalloc", desc, T(x), T(ids), T(w), out) == -1
    msg = hip_rt.last_error()
    assert "static scratch" in msg and str(8 << 20) in msg
    torch.cuda.synchronize()
    assert bool((out == 3.0).all().item())


def test_noalloc_layer_captured_in_a_graph(hip_rt, orc):
    """Captured at a token count no call has used before (5), the graph's
    replays equal the eager no-alloc call, with eager work in between."""
    rng = np.random.default_rng(5)
    E, D, F, K, Tn = 32, 1024, 512, 6, 5
    bank, shared, _ = make_layer(orc, rng, (IQ3_S,) * 3, E, D, F, 256)
    desc = bank.layer_desc(0, shared)
    xs = T(np.zeros((Tn, D), np.float32))
    ids_s = T(np.zeros((Tn, K), np.int32))
    ws_s = T(np.zeros((Tn, K), np.float32))
    out_s = torch.empty((Tn, D), dtype=torch.float32, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = layer_call(hip_rt, "sabah_moe_layer_noalloc", desc, xs, ids_s, ws_s, out_s)
    assert rc == 0, hip_rt.last_error()
    for rep in range(3):
        x, ids, w = inputs(rng, E, D, K, Tn)
        xd, idd, wd = T(x), T(ids), T(w)
        eager = torch.empty_like(out_s)
        hip_rt.check(layer_call(hip_rt, "sabah_moe_layer_noalloc", desc, xd, idd, wd, eager), "noalloc eager")
        torch.cuda.synchronize()
        xs.copy_(xd)
        ids_s.copy_(idd)
        ws_s.copy_(wd)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager), "replay %d" % rep
        (xd * 2.0).sum().item()
