"""Router gating on the device (sabah_moe_route), through the C ABI (needs an MI355X).

Bar: the selected ids equal the oracle's exactly (ties broken to the lower index on
both sides); the weights, which go through the device's and the host's expf, within
max_rel <= 2e-6 of the oracle's.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_parity, max_rel

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
IQ3_S = 21


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def route(hip_rt, logits, k, norm_w=True, w_scale=1.0):
    import ctypes
    Tn, E = logits.shape
    d_l = T(logits)
    ids = torch.empty((Tn, k), dtype=torch.int32, device=DEV)
    w = torch.empty((Tn, k), dtype=torch.float32, device=DEV)
    vp = ctypes.c_void_p
    hip_rt.check(hip_rt.lib().sabah_moe_route(vp(d_l.data_ptr()), Tn, E, k, int(norm_w), ctypes.c_float(w_scale),
                                              vp(ids.data_ptr()), vp(w.data_ptr()),
                                              vp(torch.cuda.current_stream().cuda_stream)), "route")
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("Tn,E,k,norm_w,w_scale", [(64, 512, 10, True, 1.0), (7, 128, 8, True, 1.0),
                                                   (3, 4096, 64, True, 1.0), (5, 7, 7, True, 1.0),
                                                   (9, 300, 1, True, 1.0), (16, 512, 10, False, 1.0),
                                                   (16, 512, 10, True, 2.5)])
def test_route_matches_oracle(hip_rt, orc, Tn, E, k, norm_w, w_scale):
    rng = np.random.default_rng(E * 100 + k)
    logits = (rng.standard_normal((Tn, E)) * 1.5).astype(np.float32)
    ids, w = route(hip_rt, logits, k, norm_w, w_scale)
    rid, rw = orc.moe_route(logits, k, norm_w, w_scale)
    assert np.array_equal(ids, rid)
    assert max_rel(w, rw) <= 2e-6


def test_route_ties_break_to_the_lower_index(hip_rt, orc):
    rng = np.random.default_rng(3)
    logits = np.round(rng.standard_normal((32, 256)), 1).astype(np.float32)     # many equal logits
    ids, w = route(hip_rt, logits, 12)
    rid, rw = orc.moe_route(logits, 12)
    assert np.array_equal(ids, rid)
    assert max_rel(w, rw) <= 2e-6
    ids, w = route(hip_rt, np.zeros((2, 64), np.float32), 8)
    assert np.array_equal(ids, np.tile(np.arange(8), (2, 1)))
    assert np.all(w == np.float32(0.125))


def test_routed_layer_from_device_logits(hip_rt, orc):
    """Logits -> device route -> the fused layer, all on the device: the same as the
    layer driven by the oracle's ids and weights, within the output tolerance."""
    from sabah.runtime.bank import ExpertBank
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(17)
    E, D, F, K, Tn = 64, 1024, 512, 8, 6
    bank = ExpertBank(1, E, D, F, {"gate": IQ3_S, "up": IQ3_S, "down": IQ3_S}, device="cuda:0")
    raws = {}
    for role, (rows, cols) in (("gate", (F, D)), ("up", (F, D)), ("down", (D, F))):
        raws[role] = orc.quantize_weights(IQ3_S, (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32))
        bank.load(0, role, raws[role])
    ex = MoEExecutor(bank, max_used=K)
    logits = rng.standard_normal((Tn, E)).astype(np.float32)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ids, w = ex.route(T(logits))
    got = ex.run_layer(0, T(x), ids, w).cpu().numpy()
    rid, rw = orc.moe_route(logits, K)
    assert np.array_equal(ids.cpu().numpy(), rid)
    want = orc.moe_layer(raws["gate"], raws["up"], raws["down"], (IQ3_S,) * 3, x, rid, rw)
    assert_parity(got, want, "routed layer")
