"""The oracle's router gating (softmax -> top-k -> renormalise, ggml's CPU op
order) pinned against float64 restatements and closed forms."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import max_rel
from sabah.runtime import routing


def f64_route(logits, k, norm_w=True):
    l = logits.astype(np.float64)
    p = np.exp(l - l.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, axis=1)
    if norm_w:
        w = w / w.sum(axis=1, keepdims=True)
    return ids, w


@pytest.mark.parametrize("T,E,k", [(40, 512, 10), (12, 128, 8), (3, 4096, 64), (5, 7, 7)])
def test_route_matches_float64_softmax_topk(orc, T, E, k):
    rng = np.random.default_rng(E + k)
    logits = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
    ids, w = orc.moe_route(logits, k)
    rid, rw = f64_route(logits, k)
    assert np.array_equal(ids, rid)
    assert max_rel(w, rw) < 1e-6
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
    # the renormalised weights are the softmax over the selected logits, which is
    # how the synthetic routing draws them
    gid, gw = routing.topk_from_logits(logits, k)
    assert np.array_equal(ids, gid) and max_rel(w, gw) < 1e-6


def test_route_without_renormalising_keeps_the_softmax_probabilities(orc):
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((6, 64)).astype(np.float32)
    ids, w = orc.moe_route(logits, 6, norm_w=False)
    rid, rw = f64_route(logits, 6, norm_w=False)
    assert np.array_equal(ids, rid) and max_rel(w, rw) < 1e-6
    assert np.all(w.sum(axis=1) < 1.0)
    ids2, w2 = orc.moe_route(logits, 6, norm_w=False, w_scale=2.5)
    assert np.array_equal(ids2, ids) and np.array_equal(w2, w * np.float32(2.5))


def test_route_closed_forms(orc):
    E, k = 64, 8
    # equal logits: every p is the same float, so the lowest indices win and
    # the renormalised weights are p / (float)(k * p) = 1/k to the last bit
    ids, w = orc.moe_route(np.zeros((2, E), np.float32), k)
    assert np.array_equal(ids, np.tile(np.arange(k), (2, 1)))
    p = np.float32(1.0 / E)
    assert np.array_equal(w, np.full((2, k), p / np.float32(np.float64(p) * k), np.float32))
    # ties among equal logits break to the lower index, wherever they sit
    l = np.full((1, E), -3.0, np.float32)
    l[0, [40, 9, 33]] = 2.0
    l[0, [50, 2]] = 1.0
    ids, _ = orc.moe_route(l, 5)
    assert ids[0].tolist() == [9, 33, 40, 2, 50]
    # one dominant logit takes (nearly) all the weight and comes first
    l = np.zeros((1, E), np.float32)
    l[0, 17] = 40.0
    ids, w = orc.moe_route(l, 3, norm_w=False)
    assert ids[0, 0] == 17 and w[0, 0] == np.float32(1.0) and ids[0, 1:].tolist() == [0, 1]


def test_route_rejects_more_slots_than_experts(orc):
    with pytest.raises(ValueError):
        orc.moe_route(np.zeros((1, 4), np.float32), 5)
