"""Group-major (prefill) MoE layer, through the C ABI (needs an MI355X).

sabah_moe_prefill_layer groups the (token, slot) pairs by expert on the
device and applies each expert's rows to all of its pairs with int8 MFMA
(IQ3_S, Q4_K and Q6_K weights; the K formats' bsum side terms on fp32 MFMA).
Bar: bit-identical to the token-major sabah_moe_layer on the same inputs
(same integer block sums, same fp32 order), and within max_rel <= 1e-3,
cosine >= 0.99999 of the oracle's layer.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from helpers import assert_parity, random_blocks

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K, IQ3_S = 8, 12, 14, 21
DEV = torch.device("cuda:0")


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def iq3s_bank(orc, rng, E, D, F):
    from sabah.runtime.bank import ExpertBank
    bank = ExpertBank(1, E, D, F, {"gate": IQ3_S, "up": IQ3_S, "down": IQ3_S}, device="cuda:0")
    raws = {}
    for role, (rows, cols) in (("gate", (F, D)), ("up", (F, D)), ("down", (D, F))):
        raws[role] = orc.quantize_weights(IQ3_S, (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32))
        bank.load(0, role, raws[role])
    return bank, raws


def typed_bank(orc, rng, E, D, F, qg, qd, random_bytes=False):
    """gate/up of type qg, down of type qd: quantised N(0, 0.02) weights, or
    random valid blocks (every scale, min and quant value across its range)."""
    from sabah.runtime.bank import ExpertBank
    types = {"gate": qg, "up": qg, "down": qd}
    bank = ExpertBank(1, E, D, F, types, device="cuda:0")
    raws = {}
    for role, (rows, cols) in (("gate", (F, D)), ("up", (F, D)), ("down", (D, F))):
        qt = types[role]
        if random_bytes:
            raws[role] = random_blocks(rng, qt, E * rows, cols).reshape(E, rows, -1)
        else:
            raws[role] = orc.quantize_weights(qt, (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32))
        bank.load(0, role, raws[role])
    return bank, raws


def routing_case(rng, case, Tn, E, K):
    from sabah.runtime import routing
    if case == "zipf":
        return routing.zipf_routing(rng, Tn, E, K)
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    if case == "heavy":
        ids[:, 0] = 5                      # every token's first slot on one expert: 3+ pair tiles
        ids[3, 1] = ids[3, 0]              # a duplicate id inside one token
        ids[7, :] = ids[7, 0]              # a token whose slots all hit one expert
    return ids, w


@pytest.mark.parametrize("case,E,D,F,Tn,K", [("zipf", 64, 2048, 768, 40, 10), ("heavy", 48, 1024, 512, 37, 8),
                                             ("uniform", 32, 512, 256, 5, 4)])
def test_prefill_layer_is_the_token_major_layer(hip_rt, orc, case, E, D, F, Tn, K):
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(zlib.crc32(case.encode()) % 1000)
    bank, raws = iq3s_bank(orc, rng, E, D, F)
    ids, w = routing_case(rng, case, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    got = ex.run_prefill_layer(0, T(x), T(ids), T(w))
    ref = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    assert torch.equal(got, ref), "grouped layer differs from the token-major layer (%s)" % case
    want = orc.moe_layer(raws["gate"], raws["up"], raws["down"], (IQ3_S,) * 3, x, ids, w)
    assert_parity(got.cpu().numpy(), want, "prefill %s" % case)


@pytest.mark.parametrize("gated", [False, True])
def test_prefill_layer_with_shared_expert_and_residual(hip_rt, orc, gated):
    from sabah.runtime import routing
    from sabah.runtime.bank import DenseExpert
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(811)
    E, D, F, K, Tn, Fs = 40, 1024, 512, 6, 24, 512
    bank, raws = iq3s_bank(orc, rng, E, D, F)
    shared = DenseExpert(D, Fs, Q8_0, device="cuda:0")
    sh_raw = {}
    for role, (rows, cols) in {"gate": (Fs, D), "up": (Fs, D), "down": (D, Fs)}.items():
        sh_raw[role] = orc.quantize_weights(Q8_0, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        shared.load(role, sh_raw[role])
    ids, w = routing.zipf_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    row = (rng.standard_normal(D) * 0.03).astype(np.float32) if gated else None
    shared.set_gate(row)
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    xd = T(x)
    got = ex.run_prefill_layer(0, xd, T(ids), T(w), resid=xd)
    ref = ex.run_layer(0, xd, T(ids), T(w), resid=xd)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    y = orc.moe_layer(raws["gate"], raws["up"], raws["down"], (IQ3_S,) * 3, x, ids, w,
                      shared=(sh_raw["gate"], sh_raw["up"], sh_raw["down"], (Q8_0,) * 3, row))
    assert_parity(got.cpu().numpy(), x + y, "prefill + shared%s + residual" % (" (gated)" if gated else ""))


def test_prefill_layer_in_place_on_the_residual_stream(hip_rt, orc):
    """out aliasing resid (x <- x + layer(x)) gives what a separate output gives."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(812)
    E, D, F, K, Tn = 16, 512, 256, 4, 9
    bank, _ = iq3s_bank(orc, rng, E, D, F)
    ids, w = routing.zipf_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    sep = ex.run_prefill_layer(0, T(x), T(ids), T(w), resid=T(x))
    xd = T(x)
    ex.run_prefill_layer(0, xd, T(ids), T(w), out=xd, resid=xd)
    torch.cuda.synchronize()
    assert torch.equal(sep, xd)


def test_prefill_layer_poisons_a_token_with_a_bad_id(hip_rt, orc):
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(813)
    E, D, F, K, Tn = 16, 512, 256, 4, 6
    bank, _ = iq3s_bank(orc, rng, E, D, F)
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    ids[2, 1] = E + 3
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    got = ex.run_prefill_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    assert np.all(np.isnan(g[2]))
    assert np.all(np.isfinite(np.delete(g, 2, axis=0)))
    assert hip_rt.lib().sabah_rt_check_errors() == -1
    assert hip_rt.lib().sabah_rt_check_errors() == 0
    ok = ids.copy()
    ok[2, 1] = 0
    ref = ex.run_layer(0, T(x), T(ok), T(w))
    torch.cuda.synchronize()
    r = ref.cpu().numpy()
    keep = [t for t in range(Tn) if t != 2]
    assert np.array_equal(g[keep].view(np.uint32), r[keep].view(np.uint32))


def test_prefill_layer_full_size_matches_token_major(hip_rt, orc):
    """512 tokens x top-10 over 512 IQ3_S experts (2048 / 768) on the
    device-generated bank, Zipf routing: bit-identical to the token-major layer."""
    from sabah.runtime import routing
    from sabah.runtime.bank import ExpertBank
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(814)
    E, D, F, K, Tn = 512, 2048, 768, 10, 512
    bank = ExpertBank(1, E, D, F, {"gate": IQ3_S, "up": IQ3_S, "down": IQ3_S}, device="cuda:0")
    bank.fill_synthetic(seed=11)
    ids, w = routing.zipf_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    got = ex.run_prefill_layer(0, T(x), T(ids), T(w))
    ref = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("qg,qd,case", [(Q4_K, Q6_K, "heavy"), (Q6_K, Q4_K, "zipf"), (Q4_K, IQ3_S, "uniform"),
                                        (IQ3_S, Q6_K, "heavy"), (Q6_K, Q6_K, "uniform"), (Q4_K, Q4_K, "zipf")])
def test_grouped_k_formats_are_the_token_major_layer(hip_rt, orc, qg, qd, case):
    """Q4_K / Q6_K gate/up and down on the grouped kernels: the same bits as the
    token-major layer, and the oracle's layer within tolerance."""
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(900 + 10 * qg + qd)
    E, D, F, Tn, K = 48, 1024, 512, 37, 8
    bank, raws = typed_bank(orc, rng, E, D, F, qg, qd)
    ids, w = routing_case(rng, case, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    got = ex.run_prefill_layer(0, T(x), T(ids), T(w))
    ref = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    assert torch.equal(got, ref), "grouped %d/%d layer differs from the token-major layer (%s)" % (qg, qd, case)
    want = orc.moe_layer(raws["gate"], raws["up"], raws["down"], (qg, qg, qd), x, ids, w)
    assert_parity(got.cpu().numpy(), want, "prefill %d/%d %s" % (qg, qd, case))


@pytest.mark.parametrize("qg,qd", [(Q4_K, Q6_K), (Q6_K, Q4_K)])
def test_grouped_k_formats_random_blocks(hip_rt, orc, qg, qd):
    """Random valid blocks (6-bit scales and mins up to 63, Q6_K int8 scales to
    +-128, every quant value), 2048 / 768 as in the model: the grouped side terms
    are exact, so the result is bit-identical to the token-major layer."""
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(950 + qg)
    E, D, F, Tn, K = 24, 2048, 768, 21, 6
    bank, _ = typed_bank(orc, rng, E, D, F, qg, qd, random_bytes=True)
    ids, w = routing_case(rng, "heavy", Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    got = ex.run_prefill_layer(0, T(x), T(ids), T(w))
    ref = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref)


def test_grouped_mixed_layer_full_size_matches_token_major(hip_rt, orc):
    """32 tokens x top-10 of 512 experts, Q4_K gate/up and Q6_K down (2048 / 768)
    with a Q8_0 shared expert (d_ff 512) and the residual, device-generated bank,
    uniform routing: bit-identical to the token-major layer."""
    from sabah.runtime import routing
    from sabah.runtime.bank import DenseExpert, ExpertBank
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(960)
    E, D, F, K, Tn = 512, 2048, 768, 10, 32
    bank = ExpertBank(1, E, D, F, {"gate": Q4_K, "up": Q4_K, "down": Q6_K}, device="cuda:0")
    bank.fill_synthetic(seed=12)
    shared = DenseExpert(D, 512, Q8_0, device="cuda:0")
    shared.fill_synthetic(seed=13)
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    xd = T(x)
    got = ex.run_prefill_layer(0, xd, T(ids), T(w), resid=xd)
    ref = ex.run_layer(0, xd, T(ids), T(w), resid=xd)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref)
