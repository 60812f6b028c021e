"""Host-side routing and workload bookkeeping (no GPU)."""
import numpy as np

from sabah.runtime import routing
from sabah.runtime.workloads import WORKLOADS


def test_topk_weights_are_softmax_over_the_selected():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((5, 64))
    ids, w = routing.topk_from_logits(logits, 8)
    for t in range(5):
        assert set(ids[t]) == set(np.argsort(-logits[t])[:8])
        sel = logits[t, ids[t]]
        ref = np.exp(sel - sel.max()) / np.exp(sel - sel.max()).sum()
        assert np.allclose(w[t], ref, rtol=1e-6) and abs(w[t].sum() - 1) < 1e-6
        assert np.all(np.diff(logits[t, ids[t]]) <= 0)     # descending


def test_zipf_prefill_histogram_spans_zero_to_about_a_hundred():
    mx, zeros = [], []
    for seed in range(4):
        ids, _ = routing.zipf_routing(np.random.default_rng(seed), 512, 512, 10)
        c = np.bincount(ids.ravel(), minlength=512)
        assert c.sum() == 5120 and all(len(set(r)) == 10 for r in ids)
        mx.append(c.max())
        zeros.append((c == 0).sum())
    assert 70 <= np.mean(mx) <= 130 and np.mean(zeros) < 10


def test_expected_unique_experts_for_the_mixed_workload():
    # 512 experts, top-10, 32 tokens: 512 * (1 - (502/512)^32) ~= 239.6
    assert abs(routing.expected_unique(512, 10, 32) - 239.6) < 0.1
    rng = np.random.default_rng(7)
    u = [len(np.unique(routing.uniform_routing(rng, 32, 512, 10)[0])) for _ in range(50)]
    assert abs(np.mean(u) - 239.6) < 6


def test_workload_bytes_match_the_specification():
    w3 = WORKLOADS["iq3s_48x512_top10"]
    assert w3.matrix_bytes("gate") == 675840 and w3.matrix_bytes("down") == 675840
    assert w3.expert_bytes() * 10 == 20275200                       # per layer at top-10
    assert w3.expert_bytes() * 10 * 48 == 973209600                 # per token
    assert w3.bank_bytes() == 48 * 512 * 3 * 675840 == 49828331520
    w1 = WORKLOADS["q8_0_e8_top2"]
    assert w1.expert_bytes() * 2 == 13369344
    w2 = WORKLOADS["q4k_e128_top8"]
    assert w2.expert_bytes() * 8 == 21233664
    w5 = WORKLOADS["mixed_t32_q4k_q6k_shared"]
    assert w5.expert_bytes() == 3059712 and w5.shared_bytes() == 3342336
    w4 = WORKLOADS["iq3s_prefill_t512"]
    assert w4.expert_bytes() == 2027520


def test_step_bytes_count_each_expert_once():
    w3 = WORKLOADS["iq3s_48x512_top10"]
    ids = np.zeros((2, 3, 10), np.int32)
    ids[:, :, :] = np.arange(10)
    ids[1, 2, 0] = 11                       # one extra distinct expert in layer 1
    assert w3.step_expert_bytes(ids) == (10 + 11) * w3.expert_bytes()
