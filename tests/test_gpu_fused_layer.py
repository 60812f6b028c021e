"""The one-launch decode layer (k_layer_decode; sabah_rt_set_layer_fusion(0)
switches back to the two-kernel form): one-token IQ3_S layers run
their gate/up and down workgroups in one grid, the down workgroups waiting
for h through per-workgroup flags that advance once per launch.

The bar is bit-identity with the two-kernel form of the same layer (the same
decoders and fp32 steps) and with the oracle (ggml's CPU path), on single
layers, with a shared expert and residual, in chains whose consecutive
launches differ in shape (so the flags' lockstep must hold across them), in
HIP-graph replays, with a bad expert id, and through the timeout path forced
from the host."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_parity

pytestmark = pytest.mark.gpu

Q8_0, IQ3_S = 8, 21
DEV = torch.device("cuda:0")


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture
def fusion(hip_rt):
    lib = hip_rt.lib()

    def set_mode(mode):
        hip_rt.check(lib.sabah_rt_set_layer_fusion(mode), "set fusion")

    yield set_mode
    set_mode(1)                                 # the library's default


def launches(hip_rt, kind):
    return hip_rt.kernel_timing(kind)[1]


def make_bank(orc, rng, E, D, F, n_layers=1, qt=IQ3_S):
    from sabah.runtime.bank import ExpertBank
    bank = ExpertBank(n_layers, E, D, F, {"gate": qt, "up": qt, "down": qt}, device="cuda:0")
    raws = {}
    for l in range(n_layers):
        for role, (rows, cols) in {"gate": (F, D), "up": (F, D), "down": (D, F)}.items():
            raws[(l, role)] = orc.quantize_weights(qt, (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32))
            bank.load(l, role, raws[(l, role)])
    return bank, raws


def run_both(hip_rt, fusion, fn):
    """fn() under fusion on (checking that the fused kernel ran) and off."""
    lib = hip_rt.lib()
    lib.sabah_rt_set_kernel_timing(1)
    try:
        hip_rt.kernel_timing("layer", reset=True)
        fusion(1)
        fused = fn()
        torch.cuda.synchronize()
        n_fused = launches(hip_rt, "layer")
        fusion(0)
        plain = fn()
        torch.cuda.synchronize()
        assert launches(hip_rt, "layer") == n_fused
    finally:
        lib.sabah_rt_set_kernel_timing(0)
        fusion(1)
    return fused, plain, n_fused


# (E, d_model, d_ff, top-k): the shipped shape's layer, smaller ones, a
# d_model of one unit per row and a deep d_ff
SHAPES = [(24, 2048, 768, 10), (32, 1024, 512, 6), (16, 512, 256, 2), (24, 256, 1024, 8), (12, 4096, 512, 4)]


@pytest.mark.parametrize("E,D,F,K", SHAPES)
def test_fused_layer_equals_two_kernel_layer_and_oracle(hip_rt, orc, fusion, E, D, F, K):
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(E + D + F + K)
    bank, raws = make_bank(orc, rng, E, D, F)
    ids, w = routing.zipf_routing(rng, 1, E, K)
    x = rng.standard_normal((1, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    xd, idd, wd = T(x), T(ids), T(w)
    fused, plain, n = run_both(hip_rt, fusion, lambda: ex.run_layer(0, xd, idd, wd).cpu().numpy())
    assert n == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], (IQ3_S,) * 3, x, ids, w)
    assert_parity(fused, want, "fused layer E=%d D=%d F=%d K=%d" % (E, D, F, K))
    assert np.array_equal(fused.view(np.uint32), want.view(np.uint32))


def test_fused_layer_with_shared_expert_and_residual(hip_rt, orc, fusion):
    from sabah.runtime import routing
    from sabah.runtime.bank import DenseExpert
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(77)
    E, D, F, K, Fs = 48, 2048, 768, 10, 512
    bank, _ = make_bank(orc, rng, E, D, F)
    shared = DenseExpert(D, Fs, Q8_0, device="cuda:0")
    shared.fill_synthetic(seed=78)
    shared.set_gate((rng.standard_normal(D) * 0.03).astype(np.float32))
    ids, w = routing.zipf_routing(rng, 1, E, K)
    x = T(rng.standard_normal((1, D)).astype(np.float32))
    resid = T(rng.standard_normal((1, D)).astype(np.float32))
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    fused, plain, n = run_both(hip_rt, fusion, lambda: ex.run_layer(0, x, T(ids), T(w), resid=resid).cpu().numpy())
    assert n == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))


def test_fused_chain_of_changing_shapes_keeps_the_flags_in_step(hip_rt, orc, fusion):
    """Eight chains of 6 layers, alternating top-k (10 and 3: different
    gate/up and down grid sizes between consecutive launches) and between the
    allocating and the no-alloc layer entry points; every layer bit-identical
    to the two-kernel form."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(6)
    E, D, F, L = 32, 1024, 512, 6
    bank, _ = make_bank(orc, rng, E, D, F, n_layers=L)
    lib = hip_rt.lib()
    for rep in range(8):
        K = 10 if rep % 2 == 0 else 3
        ex = MoEExecutor(bank, max_used=K)
        ids, w = routing.zipf_routing(rng, 1, E, K, n_layers=L)
        x0 = rng.standard_normal((1, D)).astype(np.float32)

        idd, wd = T(ids), T(w)                  # held for the whole chain: the kernels read them later

        def chain():
            x = T(x0)
            for l in range(L):
                desc = bank.layer_desc(l, None)
                fn = lib.sabah_moe_layer_noalloc if (rep + l) % 2 else lib.sabah_moe_layer
                hip_rt.check(fn(ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(idd[l].data_ptr()),
                                ctypes.c_void_p(wd[l].data_ptr()), K, 1, ctypes.c_void_p(x.data_ptr()),
                                ctypes.c_void_p(x.data_ptr()),
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "layer")
            return x.cpu().numpy()

        fused, plain, n = run_both(hip_rt, fusion, chain)
        assert n == sum(1 for l in range(L) if (rep + l) % 2 == 0)    # no-alloc launches are not timed
        assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32)), "rep %d" % rep


def test_fused_chain_graph_replays_match_eager(hip_rt, orc, fusion):
    """The 48-launch chain captured as one HIP graph (the kernels' arguments
    frozen): replays with different inputs, eager chains in between, each
    replay bit-identical to the eager chain."""
    from sabah.runtime import routing
    from sabah.runtime.executor import ChainGraph, MoEExecutor
    rng = np.random.default_rng(48)
    E, D, F, K, L = 16, 512, 256, 4, 48
    from sabah.runtime.bank import ExpertBank
    bank = ExpertBank(L, E, D, F, {"gate": IQ3_S, "up": IQ3_S, "down": IQ3_S}, device="cuda:0")
    bank.fill_synthetic(seed=49)
    ex = MoEExecutor(bank, max_used=K)
    fusion(1)
    cg = ChainGraph(ex, 1, K)
    for rep in range(4):
        ids, w = routing.zipf_routing(rng, 1, E, K, n_layers=L)
        x0 = T(rng.standard_normal((1, D)).astype(np.float32))
        xe = x0.clone()
        ex.run_chain(xe, T(ids), T(w))
        torch.cuda.synchronize()
        got = cg.replay(x0, T(ids), T(w))
        torch.cuda.synchronize()
        assert torch.equal(got, xe), "replay %d" % rep
        fusion(0)
        xp = x0.clone()
        ex.run_chain(xp, T(ids), T(w))
        torch.cuda.synchronize()
        fusion(1)
        assert torch.equal(xp, xe), "two-kernel chain, replay %d" % rep


@pytest.mark.parametrize("groups", [1, 3, 8])
def test_fused_layer_under_forced_down_workgroup_placements(hip_rt, orc, fusion, groups):
    """The down workgroups grouped as if placed j % groups (1: every one on a
    single XCD, so one leader for all; 3: five XCDs without any): one leader
    per group is elected on the device, and the layer stays bit-identical to
    the two-kernel form and the oracle, across consecutive launches."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(300 + groups)
    E, D, F, K = 24, 2048, 768, 10
    bank, raws = make_bank(orc, rng, E, D, F)
    ids, w = routing.zipf_routing(rng, 1, E, K)
    x = rng.standard_normal((1, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    xd, idd, wd = T(x), T(ids), T(w)
    lib = hip_rt.lib()
    hip_rt.check(lib.sabah_rt_set_layer_placement_test(groups), "placement test")
    try:
        fused, plain, n = run_both(hip_rt, fusion, lambda: ex.run_layer(0, xd, idd, wd).cpu().numpy())
        fusion(1)
        again = [ex.run_layer(0, xd, idd, wd).cpu().numpy() for _ in range(3)]
    finally:
        hip_rt.check(lib.sabah_rt_set_layer_placement_test(0), "placement test")
    assert n == 1
    assert lib.sabah_rt_check_errors() == 0, hip_rt.last_error()
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    for a in again:
        assert np.array_equal(a.view(np.uint32), fused.view(np.uint32))
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], (IQ3_S,) * 3, x, ids, w)
    assert np.array_equal(fused.view(np.uint32), want.view(np.uint32))


def test_layer_placement_test_groups_are_validated(hip_rt):
    lib = hip_rt.lib()
    assert lib.sabah_rt_set_layer_placement_test(9) == -1
    assert lib.sabah_rt_set_layer_placement_test(-1) == -1
    assert lib.sabah_rt_set_layer_placement_test(0) == 0


def test_fused_layer_bad_id_poisons_and_fails_the_next_call(hip_rt, orc, fusion):
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(9)
    E, D, F, K = 16, 512, 256, 4
    bank, _ = make_bank(orc, rng, E, D, F)
    ids, w = routing.zipf_routing(rng, 1, E, K)
    ids[0, 2] = E + 5
    x = T(rng.standard_normal((1, D)).astype(np.float32))
    ex = MoEExecutor(bank, max_used=K)
    fusion(1)
    out = ex.run_layer(0, x, T(ids), T(w))
    torch.cuda.synchronize()
    assert np.isnan(out.cpu().numpy()).all()
    lib = hip_rt.lib()
    assert lib.sabah_rt_check_errors() == -1
    assert "outside" in hip_rt.last_error()
    ids[0, 2] = 1
    good = ex.run_layer(0, x, T(ids), T(w)).cpu().numpy()
    assert np.isfinite(good).all()


def test_fused_layer_timeout_path_reports_and_recovers(hip_rt, orc, fusion):
    """Forced from the host (mode 2): the down workgroups of one launch wait
    for a flag value that is never written; their wait sees no progress for
    2 ms (the test's bound) and runs out,
    every wave exits, their rows are NaN, the next call fails naming the wait,
    and the launches after it are correct again."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(10)
    E, D, F, K = 16, 512, 256, 4
    bank, _ = make_bank(orc, rng, E, D, F)
    ids, w = routing.zipf_routing(rng, 1, E, K)
    x = T(rng.standard_normal((1, D)).astype(np.float32))
    ex = MoEExecutor(bank, max_used=K)
    fusion(1)
    want = ex.run_layer(0, x, T(ids), T(w)).cpu().numpy()
    fusion(2)
    out = ex.run_layer(0, x, T(ids), T(w))
    torch.cuda.synchronize()
    assert np.isnan(out.cpu().numpy()).all()
    lib = hip_rt.lib()
    assert lib.sabah_rt_check_errors() == -1
    assert "waited too long" in hip_rt.last_error()
    fusion(1)
    for _ in range(3):
        again = ex.run_layer(0, x, T(ids), T(w)).cpu().numpy()
        assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
    assert lib.sabah_rt_check_errors() == 0


def test_layer_fusion_mode_is_validated(hip_rt):
    lib = hip_rt.lib()
    assert lib.sabah_rt_set_layer_fusion(3) == -1
    assert lib.sabah_rt_set_layer_fusion(-1) == -1
    assert lib.sabah_rt_set_layer_fusion(1) == 0


@pytest.mark.parametrize("off", [2, 6])
def test_layers_with_banks_off_the_16_byte_grid(hip_rt, orc, fusion, off):
    """Gate, up and down banks that start `off` bytes past a 16-byte boundary
    (each inside a larger allocation, so the 16-byte chunks staged around
    their ends stay in bounds): the fused one-token layer and the two-kernel
    form stage regions with a lead and stay bit-identical to each other and
    to the oracle; the group-major batch layer stays bit-identical to the
    token-major batch layer on the same banks, and within tolerance of the
    oracle (the bar of every batch layer)."""
    from sabah.runtime import routing, rt
    rng = np.random.default_rng(70 + off)
    E, D, F, K = 16, 2048, 768, 8
    shapes = {"gate": (F, D), "up": (F, D), "down": (D, F)}
    raws = {r: orc.quantize_weights(IQ3_S, (rng.standard_normal((E,) + s) * 0.02).astype(np.float32))
            for r, s in shapes.items()}
    bufs, ptrs = {}, {}
    for r, raw in raws.items():
        buf = torch.zeros(raw.nbytes + 64, dtype=torch.uint8, device=DEV)
        buf[16 + off:16 + off + raw.nbytes] = T(raw.reshape(-1))
        bufs[r], ptrs[r] = buf, buf.data_ptr() + 16 + off
        assert ptrs[r] % 16 == off
    d = rt.MoeLayerDesc()
    d.gate, d.up, d.down = ptrs["gate"], ptrs["up"], ptrs["down"]
    d.qt_gate = d.qt_up = d.qt_down = IQ3_S
    d.d_model, d.d_ff, d.n_experts = D, F, E
    lib = hip_rt.lib()

    def layer(x, ids, w, prefill=False):
        out = torch.empty_like(x)
        fn = lib.sabah_moe_prefill_layer if prefill else lib.sabah_moe_layer
        hip_rt.check(fn(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(ids.data_ptr()),
                        ctypes.c_void_p(w.data_ptr()), ids.shape[1], ids.shape[0], ctypes.c_void_p(out.data_ptr()),
                        None, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "layer")
        return out

    def want(x, ids, w):
        return orc.moe_layer(raws["gate"], raws["up"], raws["down"], (IQ3_S,) * 3, x, ids, w)

    ids, w = routing.zipf_routing(rng, 1, E, K)
    x = rng.standard_normal((1, D)).astype(np.float32)
    xd, idd, wd = T(x), T(ids), T(w)
    fused, plain, n = run_both(hip_rt, fusion, lambda: layer(xd, idd, wd).cpu().numpy())
    assert n == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    ref = want(x, ids, w)
    assert_parity(fused, ref, "fused layer, banks at +%d" % off)
    assert np.array_equal(fused.view(np.uint32), ref.view(np.uint32))

    ids, w = routing.zipf_routing(rng, 48, E, K)
    x = rng.standard_normal((48, D)).astype(np.float32)
    got = layer(T(x), T(ids), T(w), prefill=True).cpu().numpy()
    tok = layer(T(x), T(ids), T(w)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), tok.view(np.uint32))
    assert_parity(got, want(x, ids, w), "group-major layer, banks at +%d" % off)
