"""The reference's routing-trace fixture (tests/data/bench_trace/ffn_moe_topk_L0.i32,
copied into tests/golden): 3000 tokens x top-10 ids over 512 experts of layer 0."""
import hashlib
import os

import numpy as np

from helpers import ROOT

TRACE = os.path.join(ROOT, "tests", "golden", "ffn_moe_topk_L0.i32")
SHA256 = "407deced0eabfe2c96cf98deefc334c4fb6a822eaf9fa402ae04ef50154bfeea"


def load_trace():
    return np.fromfile(TRACE, dtype=np.int32).reshape(-1, 10)


def test_trace_fixture_integrity():
    assert hashlib.sha256(open(TRACE, "rb").read()).hexdigest() == SHA256
    ids = load_trace()
    assert ids.shape == (3000, 10)
    assert ids.min() >= 0 and ids.max() < 512
    dup_rows = sum(len(set(r)) < 10 for r in ids)
    assert dup_rows == 278                  # rows that route one expert twice


def test_duplicate_ids_give_identical_slot_outputs(orc):
    """Each slot computes independently, so a repeated id repeats its row."""
    ids = load_trace()
    row = next(r for r in ids if len(set(r)) < 10)
    rng = np.random.default_rng(0)
    E, rows, k = 512, 8, 256
    bank = np.zeros((E, rows, 110), np.uint8)
    used = np.unique(row)
    w = (rng.standard_normal((len(used), rows, k)) * 0.02).astype(np.float32)
    bank[used] = orc.quantize_weights(21, w)
    x = rng.standard_normal((1, 1, k)).astype(np.float32)
    out = orc.mul_mat_id(bank, x, row[None].astype(np.int32), rows, k, 21)[0]
    for i in range(10):
        for j in range(10):
            if row[i] == row[j]:
                assert np.array_equal(out[i], out[j])
