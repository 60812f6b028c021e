"""Grouped MUL_MAT_ID (IQ3_S, Q4_K, Q6_K over many tokens) through sabah_rt_mul_mat_id_v2.

The grouped path groups the (token, slot) pairs by expert on the device and
reads each expert once per call (int8 MFMA over up to 16 pairs at a time).
Its integer block sums are exact and its fp32 steps are the token-major
kernel's, so the bar is bit-identity with the token-major path; for IQ3_S
also with the oracle (ggml's CPU MUL_MAT_ID), whose fp32 order for IQ3_S is
the same, and for the K formats (ggml sums their blocks in another fp32
order) the oracle within max_rel <= 1e-3, cosine >= 0.99999.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_parity

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, IQ3_S = 12, 14, 21
DEV = torch.device("cuda:0")
AUTO, NEVER, ALWAYS = 0, 1, 2


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.fixture
def grouping(hip_rt):
    lib = hip_rt.lib()

    def set_mode(mode):
        hip_rt.check(lib.sabah_rt_set_mmid_grouping(mode), "set grouping")

    yield set_mode
    set_mode(AUTO)


def v2(hip_rt, bank, rb, rows, k, E, x, ids, out, qt=IQ3_S):
    return hip_rt.lib().sabah_rt_mul_mat_id_v2(
        vp(bank), ctypes.c_size_t(rows * rb), ctypes.c_size_t(rb),
        vp(x), ctypes.c_size_t(x.stride(1) * 4), x.shape[1], ctypes.c_size_t(x.stride(0) * 4),
        vp(ids), ctypes.c_size_t(4), ctypes.c_size_t(ids.stride(0) * 4), ids.shape[1], ids.shape[0],
        vp(out), ctypes.c_size_t(out.stride(1) * 4), ctypes.c_size_t(out.stride(0) * 4), rows, k, E, qt,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), None)


def grouped_calls(hip_rt):
    return hip_rt.snapshot()["grouped_calls"]


def run(hip_rt, bank, rb, rows, k, E, x, ids, grouped=None, qt=IQ3_S):
    """One v2 call; `grouped` (if given) is whether it must take the grouped path."""
    out = torch.full((ids.shape[0], ids.shape[1], rows), float("nan"), dtype=torch.float32, device=DEV)
    before = grouped_calls(hip_rt)
    hip_rt.check(v2(hip_rt, bank, rb, rows, k, E, x, ids, out, qt), "v2")
    torch.cuda.synchronize()
    if grouped is not None:
        assert grouped_calls(hip_rt) == before + int(grouped)
    return out.cpu().numpy()


def case(orc, seed, E, rows, k, Tn, K, x_rows, qt=IQ3_S):
    """E experts (the last one never selected), Tn tokens x K distinct ids, a
    duplicate id in token 3; about Tn * K / (E - 1) pairs per expert, so most
    experts take several 16-pair tiles."""
    rng = np.random.default_rng(seed)
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    ids = np.stack([rng.choice(E - 1, K, replace=False) for _ in range(Tn)]).astype(np.int32)
    ids[3, K - 1] = ids[3, 0]
    x = rng.standard_normal((Tn, x_rows, k)).astype(np.float32)
    return raw, ids, x


# (k, rows): k <= 1024 runs the 64-row down-shaped kernel, k = 1536 / 2048 the
# gate/up-shaped one (two 16-row groups, k split over two waves)
SHAPES = [(768, 2048), (1024, 128), (256, 64), (2048, 768), (1536, 64)]


@pytest.mark.parametrize("k,rows", SHAPES)
@pytest.mark.parametrize("x_rows_is_n_ids", [False, True])
@pytest.mark.parametrize("qt", [IQ3_S, Q4_K, Q6_K])
def test_grouped_mul_mat_id_is_bit_identical(hip_rt, orc, grouping, qt, k, rows, x_rows_is_n_ids):
    E, Tn, K = 12, 40, 6
    raw, ids, x = case(orc, k + rows + x_rows_is_n_ids + qt, E, rows, k, Tn, K, K if x_rows_is_n_ids else 1, qt)
    bank, rb = T(raw), raw.shape[-1]
    xd, idd = T(x), T(ids)
    grouping(ALWAYS)
    got = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=True, qt=qt)
    grouping(NEVER)
    tok = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=False, qt=qt)
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    assert_parity(got, want, "grouped qt=%d k=%d rows=%d" % (qt, k, rows))
    if qt == IQ3_S:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), tok.view(np.uint32))
    if not x_rows_is_n_ids:
        assert np.array_equal(got[3, K - 1], got[3, 0])


def test_grouped_mul_mat_id_at_512_tokens_matches_token_major(hip_rt, orc, grouping):
    """The shipped gate shape (2048 -> 768) over 512 tokens x top-10 of 64
    experts: the automatic choice takes the grouped path (80 pairs per
    expert); bit-identical to the token-major path and to the oracle."""
    E, Tn, K, k, rows = 64, 512, 10, 2048, 768
    raw, ids, x = case(orc, 5, E, rows, k, Tn, K, 1)
    bank, rb = T(raw), raw.shape[-1]
    xd, idd = T(x), T(ids)
    grouping(AUTO)
    got = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=True)
    grouping(NEVER)
    tok = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=False)
    assert np.array_equal(got.view(np.uint32), tok.view(np.uint32))
    want = orc.mul_mat_id(raw, x[:64], ids[:64], rows, k, IQ3_S)
    assert np.array_equal(got[:64].view(np.uint32), want.view(np.uint32))


def test_grouped_mul_mat_id_poisons_a_bad_slot_and_fails_the_next_call(hip_rt, orc, grouping):
    E, Tn, K, k, rows = 12, 40, 6, 768, 128
    raw, ids, x = case(orc, 9, E, rows, k, Tn, K, 1)
    ids[7, 2] = E + 3
    bank, rb = T(raw), raw.shape[-1]
    grouping(ALWAYS)
    out = torch.full((Tn, K, rows), 0.0, dtype=torch.float32, device=DEV)
    hip_rt.check(v2(hip_rt, bank, rb, rows, k, E, T(x), T(ids), out), "v2")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isnan(got[7, 2]).all()
    good = np.ones((Tn, K), bool)
    good[7, 2] = False
    assert not np.isnan(got[good]).any()
    ok_ids = ids.copy()
    ok_ids[7, 2] = 0
    want = orc.mul_mat_id(raw, x, ok_ids, rows, k, IQ3_S)
    assert np.array_equal(got[good].view(np.uint32), want[good].view(np.uint32))
    lib = hip_rt.lib()
    assert lib.sabah_rt_check_errors() == -1                # the sticky word reports the bad id once
    assert "outside" in hip_rt.last_error()
    assert lib.sabah_rt_check_errors() == 0


def test_auto_grouping_keeps_few_pairs_per_expert_token_major(hip_rt, orc, grouping):
    """Below the automatic threshold (here 4 tokens x 5 ids over 12 experts,
    1.7 pairs per expert where k = 2048 needs 2) the call stays token-major."""
    E, Tn, K, k, rows = 12, 4, 5, 2048, 64
    raw, ids, x = case(orc, 11, E, rows, k, Tn, K, 1)
    bank, rb = T(raw), raw.shape[-1]
    grouping(AUTO)
    got = run(hip_rt, bank, rb, rows, k, E, T(x), T(ids), grouped=False)
    assert np.array_equal(got.view(np.uint32), orc.mul_mat_id(raw, x, ids, rows, k, IQ3_S).view(np.uint32))


def test_grouped_call_captured_in_a_graph_survives_larger_eager_calls(hip_rt, orc, grouping):
    """A grouped call captured in a HIP graph keeps the scratch it was captured
    with: eager calls that grow the library scratch afterwards retire the old
    buffers instead of freeing them, so the replays stay bit-identical (and
    memory torch allocates meanwhile is not overwritten by them)."""
    E, Tn, K, k, rows = 12, 40, 6, 2048, 64
    raw, ids, x = case(orc, 13, E, rows, k, Tn, K, 1)
    bank, rb = T(raw), raw.shape[-1]
    grouping(ALWAYS)
    xd, idd = T(x), T(ids)
    want = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=True)   # eager: sizes the scratch
    out = torch.full((Tn, K, rows), float("nan"), dtype=torch.float32, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = v2(hip_rt, bank, rb, rows, k, E, xd, idd, out)
    assert rc == 0, hip_rt.last_error()
    # larger eager calls: x with one row per slot over many tokens, so the
    # quantised-x scratch grows well past anything sized before
    rng = np.random.default_rng(14)
    for big_t in (200, 400):
        bid = np.stack([rng.choice(E - 1, K, replace=False) for _ in range(big_t)]).astype(np.int32)
        bx = rng.standard_normal((big_t, K, k)).astype(np.float32)
        run(hip_rt, bank, rb, rows, k, E, T(bx), T(bid), grouped=True)
    fill = torch.full((64 << 20,), 7.0, dtype=torch.float32, device=DEV)
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), "replay %d" % rep
        (fill * 1.0).sum().item()                           # eager work between the replays
    assert bool((fill == 7.0).all().item())


def test_scratch_growth_inside_a_capture_fails_and_says_why(hip_rt, orc, grouping):
    """A call that would have to grow the library scratch during a stream
    capture returns -1 before enqueuing anything, with a message naming the
    capture; the same call made eagerly first then captures fine."""
    E, K, k, rows = 12, 6, 2048, 64
    rng = np.random.default_rng(15)
    raw = orc.quantize_weights(IQ3_S, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    bank, rb = T(raw), raw.shape[-1]
    big_t = 1000                                            # 6000 pairs: more than any call before (5120)
    bid = T(np.stack([rng.choice(E - 1, K, replace=False) for _ in range(big_t)]).astype(np.int32))
    bx = T(rng.standard_normal((big_t, K, k)).astype(np.float32))
    out = torch.empty((big_t, K, rows), dtype=torch.float32, device=DEV)
    grouping(ALWAYS)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = v2(hip_rt, bank, rb, rows, k, E, bx, bid, out)
    assert rc == -1
    assert "capture" in hip_rt.last_error()
    eager = run(hip_rt, bank, rb, rows, k, E, bx, bid, grouped=True)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        rc = v2(hip_rt, bank, rb, rows, k, E, bx, bid, out)
    assert rc == 0, hip_rt.last_error()
    out.zero_()
    g2.replay()
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), eager.view(np.uint32))


def test_grouping_mode_is_validated(hip_rt):
    lib = hip_rt.lib()
    assert lib.sabah_rt_set_mmid_grouping(3) == -1
    assert lib.sabah_rt_set_mmid_grouping(-1) == -1
    assert lib.sabah_rt_set_mmid_grouping(AUTO) == 0


@pytest.mark.parametrize("off", [2, 6])
@pytest.mark.parametrize("k,rows", [(2048, 64), (768, 128)])
@pytest.mark.parametrize("qt", [IQ3_S, Q4_K, Q6_K])
def test_grouped_mul_mat_id_with_a_bank_off_the_16_byte_grid(hip_rt, orc, grouping, qt, k, rows, off):
    """A bank that starts `off` bytes past a 16-byte boundary: every staged
    region then has a lead, which both the grouped staging (gate/up form: one
    lead per matrix region) and the token-major staging carry.  The bank sits
    inside a larger allocation, so the 16-byte chunks read around its ends stay
    in bounds."""
    E, Tn, K = 10, 24, 5
    raw, ids, x = case(orc, 100 + k + qt + off, E, rows, k, Tn, K, 1, qt)
    rb = raw.shape[-1]
    buf = torch.zeros(raw.nbytes + 64, dtype=torch.uint8, device=DEV)
    buf[16 + off:16 + off + raw.nbytes] = T(raw.reshape(-1))
    bank = buf[16 + off:]
    assert bank.data_ptr() % 16 == off
    xd, idd = T(x), T(ids)
    grouping(ALWAYS)
    got = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=True, qt=qt)
    grouping(NEVER)
    tok = run(hip_rt, bank, rb, rows, k, E, xd, idd, grouped=False, qt=qt)
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    assert_parity(got, want, "grouped qt=%d k=%d rows=%d off=%d" % (qt, k, rows, off))
    if qt == IQ3_S:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), tok.view(np.uint32))
