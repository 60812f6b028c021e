"""HIP kernels vs the oracle, through the C ABI (needs an MI355X).

Bar: q8 activation bytes, dequantised weights and routing bit-exact; outputs
within max|y-r|/max|r| <= 1e-3 and cosine >= 0.99999 of the oracle (the
ggml-CPU restatement) on the same seeded inputs.
"""
from __future__ import annotations

import ctypes
import zlib

import numpy as np
import pytest
import torch

from helpers import assert_parity, random_blocks, unfused_rounding_row, assert_bits_equal, q8_1_tie_row

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K, IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, Q2_0 = 8, 12, 14, 18, 20, 21, 22, 23, 42
Q5_1, Q5_K = 7, 13
# formats whose fp32 steps follow ggml's vec_dot order exactly: results bit-identical to the oracle's
BIT_EXACT = (Q8_0, IQ3_S, IQ3_XXS, IQ4_NL, IQ4_XS, IQ2_S, Q2_0, Q5_1)
DEV = torch.device("cuda:0")


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def expert_weights(orc, rng, qt, E, rows, cols):
    """[E, rows, row bytes] of type qt: N(0, 0.02) quantised by the oracle's
    encoder, or (IQ3_XXS and IQ2_S, which have none) random valid blocks with modest scales."""
    if qt in (IQ3_XXS, IQ2_S):
        return random_blocks(rng, qt, E * rows, cols).reshape(E, rows, -1)
    return orc.quantize_weights(qt, (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32))


def make_bank(orc, rng, qts, E, D, F, n_layers=1):
    from sabah.runtime.bank import ExpertBank
    bank = ExpertBank(n_layers, E, D, F, {"gate": qts[0], "up": qts[1], "down": qts[2]}, device="cuda:0")
    raws = {}
    for l in range(n_layers):
        for role, (rows, cols), qt in (("gate", (F, D), qts[0]), ("up", (F, D), qts[1]), ("down", (D, F), qts[2])):
            raw = expert_weights(orc, rng, qt, E, rows, cols)
            bank.load(l, role, raw)
            raws[(l, role)] = raw
    return bank, raws


# ---------------------------------------------------------------------------
# bit-exact pieces
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qt", [Q8_0, IQ3_S, Q5_1])
def test_activation_quantisation_is_bit_exact(hip_rt, orc, qt):
    rng = np.random.default_rng(100 + qt)
    k = 2048
    x = rng.standard_normal((9, k)).astype(np.float32)
    x[1] *= 1e-3
    x[2] = 0.0                                              # zero rows
    x[3, :] = np.round(rng.standard_normal(k) * 40) + 0.5   # many exact ties
    x[3, 0] = -127.0 if qt not in (Q8_0, Q5_1) else 127.0
    x[4, 5] = 7.0
    x[4, 900] = -7.0                                        # equal magnitudes, opposite signs
    x[5] = 0.75                                             # constant row
    x[6, ::2] = 0.0
    x[7] *= 1e4
    x[8] = unfused_rounding_row(k)                          # q8_K bytes that a fused multiply-add changes
    if qt == Q5_1:
        x[8] = q8_1_tie_row(k)                              # q8_1 sums whose fp16 rounding a fused multiply changes
    ab = orc.act_row_bytes(qt, k)
    y = torch.zeros(9, ab, dtype=torch.uint8, device=DEV)
    hip_rt.check(hip_rt.lib().sabah_quantize_act(vp(T(x)), vp(y), qt, 9, k, stream()), "quantize_act")
    torch.cuda.synchronize()
    want = orc.quantize_act(qt, x)
    assert np.array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("qt,k", [(Q8_0, 1024), (Q8_0, 96), (Q4_K, 2048), (Q6_K, 768), (IQ3_S, 2048), (IQ3_S, 768),
                                  (IQ3_XXS, 2048), (IQ3_XXS, 768), (IQ4_NL, 640), (IQ4_NL, 96), (IQ4_XS, 2048),
                                  (IQ4_XS, 768), (IQ2_S, 2048), (IQ2_S, 768), (Q2_0, 2048), (Q2_0, 192),
                                  (Q2_0, 64), (Q5_1, 1024), (Q5_1, 96), (Q5_K, 2048), (Q5_K, 768)])
def test_dequant_is_bit_exact(hip_rt, orc, qt, k):
    rng = np.random.default_rng(qt * 7 + k)
    raw = random_blocks(rng, qt, 37, k)
    src = T(raw)
    dst = torch.empty(37, k, dtype=torch.float32, device=DEV)
    torch.cuda.synchronize()
    hip_rt.check(hip_rt.lib().sabah_dequant(vp(src), vp(dst), qt, 37, k), "dequant")
    got = dst.cpu().numpy()
    want = orc.dequantize(qt, raw, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------------------
# MUL_MAT_ID through sabah_rt_mul_mat_id_v2
# ---------------------------------------------------------------------------
def v2(hip_rt, src, expert_stride, row_bytes, x, ids, out, rows, k, E, qt):
    return hip_rt.lib().sabah_rt_mul_mat_id_v2(
        ctypes.c_void_p(src), expert_stride, row_bytes,
        vp(x), x.stride(1) * 4, x.shape[1], x.stride(0) * 4,
        vp(ids), 4, ids.stride(0) * 4, ids.shape[1], ids.shape[0],
        vp(out), out.stride(1) * 4, out.stride(0) * 4, rows, k, E, qt, stream(), None)


# (Q8_0, 32768): a row (34816 bytes) larger than a workgroup's 32 KB staging
# area, so each row is staged in two passes, with over 64 KB of LDS
# (IQ4_NL, 96): a row of three blocks, one partial four-block unit
CASES = [(Q8_0, 1024, 96), (Q8_0, 2048, 40), (Q8_0, 160, 24), (Q4_K, 2048, 48), (Q4_K, 768, 64),
         (Q6_K, 768, 72), (IQ3_S, 2048, 48), (IQ3_S, 768, 104), (Q8_0, 32768, 6),
         (IQ3_XXS, 2048, 48), (IQ3_XXS, 2560, 40), (IQ4_NL, 640, 64), (IQ4_NL, 96, 24), (IQ4_XS, 2048, 48),
         (IQ4_XS, 768, 72), (IQ2_S, 2048, 48), (IQ2_S, 768, 80), (Q2_0, 2048, 48), (Q2_0, 768, 64),
         (Q2_0, 192, 40), (Q2_0, 64, 24), (Q5_1, 2048, 48), (Q5_1, 96, 24), (Q5_K, 2048, 48), (Q5_K, 768, 64)]


@pytest.mark.parametrize("qt,k,rows", CASES)
@pytest.mark.parametrize("x_rows_is_n_ids", [False, True])
def test_mul_mat_id_matches_oracle(hip_rt, orc, qt, k, rows, x_rows_is_n_ids):
    rng = np.random.default_rng(qt * 1000 + k + rows + x_rows_is_n_ids)
    E, Tn, K = 7, 3, 4
    raw = expert_weights(orc, rng, qt, E, rows, k)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(Tn)]).astype(np.int32)
    ids[2, 3] = ids[2, 1]                                    # duplicate id
    x_rows = K if x_rows_is_n_ids else 1
    x = rng.standard_normal((Tn, x_rows, k)).astype(np.float32)
    bank = T(raw)
    out = torch.full((Tn, K, rows), float("nan"), dtype=torch.float32, device=DEV)
    rb = raw.shape[-1]
    hip_rt.check(v2(hip_rt, bank.data_ptr(), rows * rb, rb, T(x), T(ids), out, rows, k, E, qt), "v2")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    assert_parity(got, want, "qt=%d k=%d" % (qt, k))
    if qt in BIT_EXACT:
        # same int sums, same fp32 scale-and-accumulate order as ggml's vec_dot
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if x_rows == 1:
        assert np.array_equal(got[2, 3], got[2, 1])


# Many tokens: 32 tokens x 10 ids over 1000-2048 rows give 10,000+ single-pass
# row tiles, so the launch grows each workgroup's row tile to several staging
# passes (up to 8) while keeping 1,024+ workgroups.  IQ3_S at k 2048: 32-row
# passes, 256-row tiles.  Q6_K at k 768: 51-row passes, 408-row tiles, the last
# 8 rows long (2048 = 5 x 408 + 8).  Q8_0 at k 1024: 30-row passes, 240-row
# tiles, the last 40 rows long.
@pytest.mark.parametrize("qt,k,rows", [(IQ3_S, 2048, 2048), (Q6_K, 768, 2048), (Q8_0, 1024, 1000)])
def test_mul_mat_id_many_tokens_in_multi_pass_row_tiles(hip_rt, orc, qt, k, rows):
    rng = np.random.default_rng(qt * 7 + rows)
    E, Tn, K = 24, 32, 10
    raw = expert_weights(orc, rng, qt, E, rows, k)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(Tn)]).astype(np.int32)
    x = rng.standard_normal((Tn, 1, k)).astype(np.float32)
    bank = T(raw)
    out = torch.full((Tn, K, rows), float("nan"), dtype=torch.float32, device=DEV)
    rb = raw.shape[-1]
    L = hip_rt.lib()
    hip_rt.check(L.sabah_rt_set_mmid_grouping(1), "grouping")   # the token-major kernel (IQ3_S would group)
    try:
        hip_rt.check(v2(hip_rt, bank.data_ptr(), rows * rb, rb, T(x), T(ids), out, rows, k, E, qt), "v2")
        torch.cuda.synchronize()
    finally:
        hip_rt.check(L.sabah_rt_set_mmid_grouping(0), "grouping")
    got = out.cpu().numpy()
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    assert_parity(got, want, "qt=%d k=%d rows=%d" % (qt, k, rows))
    if qt in BIT_EXACT:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qt,k,rows,pad", [(IQ3_S, 2560, 40, 36), (Q8_0, 1024, 24, 6), (Q4_K, 512, 70, 16)])
def test_mul_mat_id_padded_rows(hip_rt, orc, qt, k, rows, pad):
    """Rows `pad` bytes apart beyond their length (src0->nb[1] > row bytes):
    each row is staged as its own tile; IQ3_S k=2560 rows (1100 bytes) take
    two passes at 25 tiles per workgroup."""
    rng = np.random.default_rng(qt * 7 + k + pad)
    E, Tn, K = 5, 2, 3
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    rb = raw.shape[-1]
    padded = np.full((E, rows, rb + pad), 0xA5, dtype=np.uint8)
    padded[:, :, :rb] = raw
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(Tn)]).astype(np.int32)
    x = rng.standard_normal((Tn, 1, k)).astype(np.float32)
    bank = T(padded)
    out = torch.full((Tn, K, rows), float("nan"), dtype=torch.float32, device=DEV)
    hip_rt.check(v2(hip_rt, bank.data_ptr(), rows * (rb + pad), rb + pad, T(x), T(ids), out, rows, k, E, qt), "v2")
    torch.cuda.synchronize()
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    assert_parity(out.cpu().numpy(), want, "padded qt=%d" % qt)
    if qt in (Q8_0, IQ3_S):
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


# One token of IQ3_S runs the per-wave rounds kernel (k_mmid_rounds): its
# outputs must be bit-identical to the whole-tile kernel's (k_mmid, forced with
# sabah_rt_set_mmid_rounds(0)) and to the oracle.  Shapes: the shipped gate/up
# form (k 2048: 32-row tiles, x one row) and down form (k 768: 85-row tiles, x
# one row per slot); a last tile of 4 rows (100 = 3 x 32 + 4: five of its
# eight waves own no unit); one unit per row (k 256, 256-row tiles, rows 300);
# 16 units per row (k 4096, 16-row tiles); and a padded row stride, which keeps
# the whole-tile kernel.
@pytest.mark.parametrize("k,rows,x_rows_is_n_ids,pad,Tn", [(2048, 768, False, 0, 1), (768, 2048, True, 0, 1),
                                                            (2048, 100, False, 0, 1), (256, 300, True, 0, 1),
                                                            (4096, 40, False, 0, 1), (2048, 64, False, 20, 1),
                                                            (2048, 768, False, 0, 4), (768, 2048, True, 0, 3)])
def test_one_token_iq3s_rounds_kernel_equals_the_tile_kernel(hip_rt, orc, k, rows, x_rows_is_n_ids, pad, Tn):
    """(The last two shapes: 4 and 3 tokens, whose row tiles stay single-pass, so they take
    the rounds kernel too.)"""
    rng = np.random.default_rng(k + rows + pad + 17 * x_rows_is_n_ids + 101 * Tn)
    qt, E, K = IQ3_S, 12, 10
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    rb = raw.shape[-1]
    padded = np.full((E, rows, rb + pad), 0xA5, dtype=np.uint8)
    padded[:, :, :rb] = raw
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(Tn)]).astype(np.int32)
    ids[0, 7] = ids[0, 2]                                   # duplicate id
    x_rows = K if x_rows_is_n_ids else 1
    x = rng.standard_normal((Tn, x_rows, k)).astype(np.float32)
    bank, xd, idd = T(padded), T(x), T(ids)
    L = hip_rt.lib()
    outs = []
    try:
        for mode in (1, 0):
            hip_rt.check(L.sabah_rt_set_mmid_rounds(mode), "rounds mode")
            out = torch.full((Tn, K, rows), float("nan"), dtype=torch.float32, device=DEV)
            hip_rt.check(v2(hip_rt, bank.data_ptr(), rows * (rb + pad), rb + pad, xd, idd, out, rows, k, E, qt), "v2")
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
    finally:
        hip_rt.check(L.sabah_rt_set_mmid_rounds(1), "rounds mode")
    assert_bits_equal(outs[0], outs[1], "rounds vs tile kernel, k=%d rows=%d" % (k, rows))
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    assert np.array_equal(outs[0].view(np.uint32), want.view(np.uint32))
    if x_rows == 1:
        assert np.array_equal(outs[0][0, 7], outs[0][0, 2])


def test_one_token_iq3s_rounds_kernel_poisons_a_bad_id(hip_rt, orc):
    rng = np.random.default_rng(81)
    qt, E, rows, k = IQ3_S, 4, 96, 2048
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    x = T(rng.standard_normal((1, 1, k)).astype(np.float32))
    ids = T(np.array([[3, -1, 0]], np.int32))
    out = torch.zeros(1, 3, rows, dtype=torch.float32, device=DEV)
    assert v2(hip_rt, T(raw).data_ptr(), rows * 880, 880, x, ids, out, rows, k, E, qt) == 0
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isnan(o[0, 1])) and np.all(np.isfinite(o[0, [0, 2]]))
    assert hip_rt.lib().sabah_rt_check_errors() == -1
    assert hip_rt.lib().sabah_rt_check_errors() == 0


def test_mul_mat_id_detects_wrong_expert_and_wrong_row(hip_rt, orc):
    rng = np.random.default_rng(77)
    qt, E, rows, k, K = IQ3_S, 8, 64, 768, 4
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    ids = np.array([[1, 5, 2, 7]], np.int32)
    x = rng.standard_normal((1, K, k)).astype(np.float32)
    out = torch.empty(1, K, rows, dtype=torch.float32, device=DEV)
    hip_rt.check(v2(hip_rt, T(raw).data_ptr(), rows * 330, 330, T(x), T(ids), out, rows, k, E, qt), "v2")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exact = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    wrong_expert = orc.mul_mat_id(raw, x, (ids + 1) % E, rows, k, qt)
    row0 = orc.mul_mat_id(raw, np.repeat(x[:, :1], K, axis=1), ids, rows, k, qt)
    from helpers import rel_l2
    err = rel_l2(got, exact)
    assert rel_l2(wrong_expert, exact) > 1e4 * max(err, 1e-9)
    assert rel_l2(row0, exact) > 1e-1


def test_registered_key_gives_bit_identical_results(hip_rt, orc):
    """A caller-side (host) address registered for the bank selects the same bytes
    as the device pointer itself; moving the bank does not change a bit."""
    rng = np.random.default_rng(78)
    qt, E, rows, k, K = IQ3_S, 6, 48, 2048, 3
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    host_key = np.zeros(raw.size, np.uint8)                 # stands for llama.cpp's mmap address
    dev_a, dev_b = T(raw), T(raw)
    ids = np.array([[4, 0, 4]], np.int32)
    x = rng.standard_normal((1, 1, k)).astype(np.float32)
    L = hip_rt.lib()
    outs = []
    for src in (dev_a.data_ptr(), dev_b.data_ptr(), host_key.ctypes.data):
        if src == host_key.ctypes.data:
            hip_rt.check(L.sabah_rt_register_bank(ctypes.c_void_p(src), vp(dev_b), raw.size, rows * 880, E), "register")
        out = torch.empty(1, K, rows, dtype=torch.float32, device=DEV)
        hip_rt.check(v2(hip_rt, src, rows * 880, 880, T(x), T(ids), out, rows, k, E, qt), "v2")
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    hip_rt.check(L.sabah_rt_unregister_bank(ctypes.c_void_p(host_key.ctypes.data)), "unregister")
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    # an unregistered host address is refused with a message, not read
    out = torch.empty(1, K, rows, dtype=torch.float32, device=DEV)
    assert v2(hip_rt, host_key.ctypes.data, rows * 880, 880, T(x), T(ids), out, rows, k, E, qt) == -1
    assert "register" in hip_rt.last_error()


def test_out_of_range_id_poisons_its_slot_and_fails_the_next_call(hip_rt, orc):
    rng = np.random.default_rng(79)
    qt, E, rows, k = Q8_0, 4, 16, 256
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    bank = T(raw)
    x = T(rng.standard_normal((1, 1, k)).astype(np.float32))
    ids = T(np.array([[1, 9]], np.int32))                    # 9 >= n_experts
    out = torch.zeros(1, 2, rows, dtype=torch.float32, device=DEV)
    assert v2(hip_rt, bank.data_ptr(), rows * 272, 272, x, ids, out, rows, k, E, qt) == 0
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isnan(o[0, 1])) and np.all(np.isfinite(o[0, 0]))
    assert hip_rt.lib().sabah_rt_check_errors() == -1
    assert "outside" in hip_rt.last_error()
    assert hip_rt.lib().sabah_rt_check_errors() == 0       # the word was cleared


def test_metrics_count_every_lookup_as_resident(hip_rt, orc):
    before = hip_rt.metrics()["hits"]
    rng = np.random.default_rng(80)
    raw = orc.quantize_weights(Q8_0, (rng.standard_normal((3, 8, 64)) * 0.02).astype(np.float32))
    out = torch.empty(2, 2, 8, dtype=torch.float32, device=DEV)
    x = T(rng.standard_normal((2, 1, 64)).astype(np.float32))
    hip_rt.check(v2(hip_rt, T(raw).data_ptr(), 8 * 68, 68, x, T(np.array([[0, 1], [2, 2]], np.int32)), out, 8, 64,
                    3, Q8_0), "v2")
    torch.cuda.synchronize()
    m = hip_rt.metrics()
    assert m["hits"] == before + 4 and m["misses"] == 0 and m["evictions"] == 0


# ---------------------------------------------------------------------------
# fused block / layer / chain
# ---------------------------------------------------------------------------
def test_moe_block_single_token_q8_0(hip_rt, orc):
    """sabah_moe_block with the reference's signature, on the Q8_0 / E=8 / top-2 /
    1024<->2048 workload (weights N(0,0.02) -> Q8_0, x ~ N(0,1), 2 distinct ids,
    softmax weights)."""
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(2024)
    E, D, F, K = 8, 1024, 2048, 2
    bank, raws = make_bank(orc, rng, (Q8_0, Q8_0, Q8_0), E, D, F)
    ex = MoEExecutor(bank, max_used=K)
    x = rng.standard_normal(D).astype(np.float32)
    ids = rng.choice(E, K, replace=False).astype(np.int32)
    lg = rng.standard_normal(K)
    w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
    ex.upload_x(x)
    ex.run_block(0, ids, w)
    got = ex.download_out()
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], (Q8_0,) * 3, x[None], ids[None],
                         w[None])[0]
    assert_parity(got, want, "moe_block")
    # accumulate adds onto the previous output
    ex.run_block(0, ids, w, accumulate=True)
    assert_parity(ex.download_out(), 2 * want, "moe_block accumulate")


# iq3xxs_iq4nl_artifact_shape: the quant mix of the reference's shipped block
# (IQ3_XXS gate/up, IQ4_NL down; results/bench_moe_blk0_iq3s.json) at its
# inferred shape, d_model 2560 and expert d_ff 640 (REPORT.md:345-347)
# iq3s_t32: 32 tokens, so gate/up and down run grown multi-pass row tiles and
# down reads h quantised once per (token, slot) row (q8_K rows); q8_0_t4_hq and
# iq4nl_down_t3_hq take that path with q8_0 rows (Q8_0 / IQ4_NL down, d_ff 768)
@pytest.mark.parametrize("name", ["q4k_e128_top8", "mixed_t32_q4k_q6k_shared", "iq3s_small", "iq3s_t32",
                                  "iq3xxs_iq4nl_artifact_shape", "iq4xs_small", "iq2s_iq3s_mix", "q8_0_t4_hq",
                                  "iq4nl_down_t3_hq", "q2_0_decode", "q2_0_down_t3_hq", "q2_0_partial_units",
                                  "q4k_q5_1_block", "q5_1_down_t3_hq", "q5k_decode", "q5k_t4_hq"])
def test_moe_layer_matches_oracle(hip_rt, orc, name):
    from sabah.runtime import routing
    from sabah.runtime.bank import DenseExpert
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(zlib.crc32(name.encode()) % 1000)
    shared = None
    if name == "q4k_e128_top8":
        E, D, F, K, Tn, qts = 128, 2048, 768, 8, 1, (Q4_K, Q4_K, Q4_K)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    elif name == "mixed_t32_q4k_q6k_shared":
        E, D, F, K, Tn, qts = 96, 2048, 768, 10, 32, (Q4_K, Q4_K, Q6_K)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    elif name == "iq3xxs_iq4nl_artifact_shape":
        E, D, F, K, Tn, qts = 64, 2560, 640, 10, 3, (IQ3_XXS, IQ3_XXS, IQ4_NL)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "iq2s_iq3s_mix":
        E, D, F, K, Tn, qts = 48, 2560, 768, 10, 2, (IQ2_S, IQ2_S, IQ3_S)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "iq3s_t32":
        E, D, F, K, Tn, qts = 64, 2048, 768, 10, 32, (IQ3_S, IQ3_S, IQ3_S)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "iq4xs_small":
        E, D, F, K, Tn, qts = 32, 2048, 768, 8, 2, (IQ4_XS, IQ4_XS, IQ4_XS)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    elif name == "q8_0_t4_hq":
        E, D, F, K, Tn, qts = 16, 1024, 768, 4, 4, (Q8_0, Q8_0, Q8_0)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    elif name == "iq4nl_down_t3_hq":
        E, D, F, K, Tn, qts = 24, 2048, 768, 6, 3, (IQ3_XXS, IQ3_XXS, IQ4_NL)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "q2_0_decode":
        E, D, F, K, Tn, qts = 64, 2048, 768, 10, 1, (Q2_0, Q2_0, Q2_0)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "q2_0_down_t3_hq":
        E, D, F, K, Tn, qts = 24, 2048, 768, 6, 3, (IQ3_XXS, IQ3_XXS, Q2_0)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "q4k_q5_1_block":
        # the reference's Q4_K / Q4_K / Q5_1 block (results/bench_moe_blk0.json), one token
        E, D, F, K, Tn, qts = 32, 2048, 768, 8, 1, (Q4_K, Q4_K, Q5_1)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    elif name == "q5_1_down_t3_hq":
        E, D, F, K, Tn, qts = 24, 2048, 768, 6, 3, (Q5_1, Q5_1, Q5_1)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "q5k_decode":
        E, D, F, K, Tn, qts = 64, 2048, 768, 10, 1, (Q5_K, Q5_K, Q5_K)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    elif name == "q5k_t4_hq":
        E, D, F, K, Tn, qts = 32, 2048, 768, 8, 4, (Q5_K, Q5_K, Q5_K)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    elif name == "q2_0_partial_units":
        # d_model 960 = 3 units + 3 blocks, d_ff 576 = 2 units + 1 block
        E, D, F, K, Tn, qts = 16, 960, 576, 4, 2, (Q2_0, Q2_0, Q2_0)
        ids, w = routing.uniform_routing(rng, Tn, E, K)
    else:
        E, D, F, K, Tn, qts = 64, 2048, 768, 10, 4, (IQ3_S, IQ3_S, IQ3_S)
        ids, w = routing.zipf_routing(rng, Tn, E, K)
    bank, raws = make_bank(orc, rng, qts, E, D, F)
    sh_raw = None
    if name.startswith("mixed"):
        Fs = 512
        shared = DenseExpert(D, Fs, Q8_0, device="cuda:0")
        sh_raw = {}
        for role, (rows, cols) in {"gate": (Fs, D), "up": (Fs, D), "down": (D, Fs)}.items():
            sh_raw[role] = orc.quantize_weights(Q8_0, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
            shared.load(role, sh_raw[role])
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    out = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    sh = None if sh_raw is None else (sh_raw["gate"], sh_raw["up"], sh_raw["down"], (Q8_0,) * 3)
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], qts, x, ids, w, shared=sh)
    assert_parity(out.cpu().numpy(), want, name)
    if name.startswith("q2_0") or name.startswith("q5_1"):
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_mixed_layer_at_512_experts_on_a_synthetic_bank(hip_rt, orc):
    """The mixed small-batch decode workload at its full size: 32 tokens x
    top-10 of 512 experts from uniform router logits (about 240 distinct
    experts), Q4_K gate/up, Q6_K down, a Q8_0 shared expert of d_ff 512.  The
    bank is generated on the device; the oracle reads back the routed experts'
    bytes and the shared expert's."""
    from sabah.runtime import routing
    from sabah.runtime.bank import DenseExpert, ExpertBank
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(532)
    E, D, F, K, Tn, Fs = 512, 2048, 768, 10, 32, 512
    qts = (Q4_K, Q4_K, Q6_K)
    bank = ExpertBank(1, E, D, F, {"gate": Q4_K, "up": Q4_K, "down": Q6_K}, device="cuda:0")
    bank.fill_synthetic(seed=532)
    shared = DenseExpert(D, Fs, Q8_0, device="cuda:0")
    shared.fill_synthetic(seed=533)
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    used = np.unique(ids)
    assert 200 <= len(used) <= 280
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    out = MoEExecutor(bank, max_used=K, shared=shared).run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    remap = {int(e): i for i, e in enumerate(used)}
    sub = {r: np.stack([bank.read_expert(0, r, int(e)) for e in used]) for r in ("gate", "up", "down")}
    sh = tuple(shared.read(r) for r in ("gate", "up", "down")) + ((Q8_0,) * 3,)
    want = orc.moe_layer(sub["gate"], sub["up"], sub["down"], qts, x, np.vectorize(remap.get)(ids).astype(np.int32),
                         w, shared=sh)
    assert_parity(out.cpu().numpy(), want, "mixed layer, 512 experts")


def test_moe_layer_with_a_sigmoid_gated_shared_expert(hip_rt, orc):
    """The shared expert's output times sigmoid(gate_inp . x) (qwen4exp.cpp:877-885),
    applied in the shared down launch.  A random gate row: within tolerance of the
    oracle; rows giving g = 1 and g = 0 exactly: bit-identical to the ungated layer
    and to the layer without the shared expert."""
    from sabah.runtime import routing
    from sabah.runtime.bank import DenseExpert
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(71)
    E, D, F, K, Tn, Fs, qts = 48, 2048, 768, 8, 5, 512, (Q4_K, Q4_K, Q6_K)
    bank, raws = make_bank(orc, rng, qts, E, D, F)
    shared = DenseExpert(D, Fs, Q8_0, device="cuda:0")
    sh_raw = {}
    for role, (rows, cols) in {"gate": (Fs, D), "up": (Fs, D), "down": (D, Fs)}.items():
        sh_raw[role] = orc.quantize_weights(Q8_0, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        shared.load(role, sh_raw[role])
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    row = (rng.standard_normal(D) * 0.03).astype(np.float32)
    shared.set_gate(row)
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    got = ex.run_layer(0, T(x), T(ids), T(w)).cpu().numpy()
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], qts, x, ids, w,
                         shared=(sh_raw["gate"], sh_raw["up"], sh_raw["down"], (Q8_0,) * 3, row))
    assert_parity(got, want, "gated shared expert")
    shared.set_gate(None)
    ungated = ex.run_layer(0, T(x), T(ids), T(w)).cpu().numpy()
    routed = MoEExecutor(bank, max_used=K).run_layer(0, T(x), T(ids), T(w)).cpu().numpy()
    for t in range(Tn):
        shared.set_gate(1e4 * x[t])
        assert np.array_equal(ex.run_layer(0, T(x), T(ids), T(w)).cpu().numpy()[t], ungated[t])
        shared.set_gate(-1e4 * x[t])
        assert np.array_equal(ex.run_layer(0, T(x), T(ids), T(w)).cpu().numpy()[t], routed[t])


def _dense_shared_case(orc, rng, qt_routed, qt_shared, E, D, F, Fs, K):
    from sabah.runtime.bank import DenseExpert
    bank, raws = make_bank(orc, rng, (qt_routed,) * 3, E, D, F)
    shared = DenseExpert(D, Fs, qt_shared, device="cuda:0")
    sh_raw = {}
    for role, (rows, cols) in {"gate": (Fs, D), "up": (Fs, D), "down": (D, Fs)}.items():
        sh_raw[role] = orc.quantize_weights(qt_shared, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        shared.load(role, sh_raw[role])
    return bank, raws, shared, sh_raw


def test_shared_expert_over_a_batch_is_bit_exact_with_the_oracle(hip_rt, orc):
    """At four tokens and more the shared expert reads each weight row once
    per launch for all tokens (k_dense_tokens); with Q8_0 throughout the
    layer is bit-exact with the oracle."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(6061)
    E, D, F, Fs, K, Tn = 16, 1024, 512, 768, 4, 6
    bank, raws, shared, sh_raw = _dense_shared_case(orc, rng, Q8_0, Q8_0, E, D, F, Fs, K)
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    got = MoEExecutor(bank, max_used=K, shared=shared).run_layer(0, T(x), T(ids), T(w)).cpu().numpy()
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], (Q8_0,) * 3, x, ids, w,
                         shared=(sh_raw["gate"], sh_raw["up"], sh_raw["down"], (Q8_0,) * 3))
    assert_bits_equal(got, want, "Q8_0 layer with a shared expert over 6 tokens")


@pytest.mark.parametrize("qt_shared,Tn,gated", [(Q8_0, 7, True), (Q4_K, 40, True), (IQ3_S, 5, False)])
def test_shared_expert_over_a_batch_equals_one_token_calls(hip_rt, orc, qt_shared, Tn, gated):
    """The batched shared expert (x and h quantised once, each weight row read
    once per 32 tokens, the gate logits computed in the gate/up launch) gives
    every token the bits of a one-token call of the same layer (the per-token
    launches), with and without the sigmoid gate; 40 tokens take two token
    groups."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(6062 + Tn)
    E, D, F, Fs, K = 16, 1024, 512, 512, 4
    bank, raws, shared, _ = _dense_shared_case(orc, rng, Q8_0, qt_shared, E, D, F, Fs, K)
    if gated:
        shared.set_gate((rng.standard_normal(D) * 0.05).astype(np.float32))
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    batch = ex.run_layer(0, T(x), T(ids), T(w)).cpu().numpy()
    for t in range(Tn):
        one = ex.run_layer(0, T(x[t:t + 1]), T(ids[t:t + 1]), T(w[t:t + 1])).cpu().numpy()
        assert_bits_equal(batch[t:t + 1], one, "token %d of %d" % (t, Tn))


def test_batched_shared_expert_on_its_side_stream_in_a_graph(hip_rt, orc):
    """The batched shared expert runs on the library's side stream, forked
    from the caller's stream and joined before the routed combine.  Captured
    in a HIP graph (the fork and join become graph edges) and replayed with
    new inputs, eager layers in between: every replay equals the eager layer,
    and the eager layer equals the oracle."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(6071)
    E, D, F, Fs, K, Tn = 16, 1024, 512, 512, 4, 8
    bank, raws, shared, sh_raw = _dense_shared_case(orc, rng, Q8_0, Q8_0, E, D, F, Fs, K)
    shared.set_gate((rng.standard_normal(D) * 0.05).astype(np.float32))
    ex = MoEExecutor(bank, max_used=K, shared=shared)
    xs = torch.zeros(Tn, D, dtype=torch.float32, device=DEV)
    ids_s = torch.zeros(Tn, K, dtype=torch.int32, device=DEV)
    w_s = torch.zeros(Tn, K, dtype=torch.float32, device=DEV)
    out = torch.zeros(Tn, D, dtype=torch.float32, device=DEV)
    ex.run_layer(0, xs, ids_s, w_s, out=out)                # sizes the library scratch
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ex.run_layer(0, xs, ids_s, w_s, out=out)
    torch.cuda.synchronize()
    for rep in range(3):
        ids, w = routing.uniform_routing(rng, Tn, E, K)
        x = rng.standard_normal((Tn, D)).astype(np.float32)
        eager = ex.run_layer(0, T(x), T(ids), T(w)).cpu().numpy()
        xs.copy_(T(x))
        ids_s.copy_(T(ids))
        w_s.copy_(T(w))
        g.replay()
        torch.cuda.synchronize()
        assert_bits_equal(out.cpu().numpy(), eager, "replay %d" % rep)
        want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], (Q8_0,) * 3, x, ids, w,
                             shared=(sh_raw["gate"], sh_raw["up"], sh_raw["down"], (Q8_0,) * 3,
                                     shared.gate_inp.cpu().numpy()))
        assert_parity(eager, want, "gated shared expert, replay %d" % rep)


@pytest.mark.parametrize("D,F", [(512, 544), (1024, 800)])
def test_iq3s_gate_up_with_a_partial_last_row_tile(hip_rt, orc, D, F):
    """IQ3_S gate/up runs in two rounds of 256 units per workgroup (R = 256 /
    units per row rows); d_ff here leaves the last workgroup a part of a round
    (and, at 512 / 544, waves with no units at all)."""
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(D + F)
    E, K, Tn, qts = 12, 4, 3, (IQ3_S, IQ3_S, Q8_0)
    bank, raws = make_bank(orc, rng, qts, E, D, F)
    ids, w = routing.uniform_routing(rng, Tn, E, K)
    x = rng.standard_normal((Tn, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    out = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    want = orc.moe_layer(raws[(0, "gate")], raws[(0, "up")], raws[(0, "down")], qts, x, ids, w)
    assert_parity(out.cpu().numpy(), want, "partial row tile D=%d F=%d" % (D, F))


def test_moe_chain_is_the_sequence_of_residual_layers(hip_rt, orc):
    from sabah.runtime import routing
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(31)
    E, D, F, K, L = 32, 1024, 512, 6, 3
    bank, raws = make_bank(orc, rng, (IQ3_S,) * 3, E, D, F, n_layers=L)
    ids, w = routing.zipf_routing(rng, 1, E, K, n_layers=L)
    x0 = rng.standard_normal((1, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    xd = T(x0)
    ex.run_chain(xd, T(ids), T(w))
    torch.cuda.synchronize()
    xr = x0.copy()
    for l in range(L):
        xr = xr + orc.moe_layer(raws[(l, "gate")], raws[(l, "up")], raws[(l, "down")], (IQ3_S,) * 3, xr, ids[l], w[l])
    assert_parity(xd.cpu().numpy(), xr, "chain")


def test_chain_graph_replays_match_eager(hip_rt, orc):
    """The chain captured as a HIP graph: three replays with different
    inputs, eager work and synchronisations in between, each bit-identical to
    the eager chain on the same inputs."""
    from sabah.runtime import routing
    from sabah.runtime.executor import ChainGraph, MoEExecutor
    rng = np.random.default_rng(57)
    E, D, F, K, L = 24, 512, 256, 4, 3
    bank, _ = make_bank(orc, rng, (IQ3_S,) * 3, E, D, F, n_layers=L)
    ex = MoEExecutor(bank, max_used=K)
    cg = ChainGraph(ex, 1, K)
    for rep in range(3):
        ids, w = routing.zipf_routing(rng, 1, E, K, n_layers=L)
        x0 = T(rng.standard_normal((1, D)).astype(np.float32))
        xe = x0.clone()
        ex.run_chain(xe, T(ids), T(w))
        torch.cuda.synchronize()
        got = cg.replay(x0, T(ids), T(w))
        torch.cuda.synchronize()
        assert torch.equal(got, xe), "replay %d" % rep
        (x0 * 2.0).sum().item()                          # unrelated eager work between replays


def test_full_size_iq3s_layer_on_synthetic_bank(hip_rt, orc):
    """One layer of the 512-expert IQ3_S shape with the bank generated on the
    device; the oracle reads back the ten routed experts' bytes."""
    from sabah.runtime import routing
    from sabah.runtime.bank import ExpertBank
    from sabah.runtime.executor import MoEExecutor
    rng = np.random.default_rng(48)
    E, D, F, K = 512, 2048, 768, 10
    bank = ExpertBank(1, E, D, F, {"gate": IQ3_S, "up": IQ3_S, "down": IQ3_S}, device="cuda:0")
    bank.fill_synthetic(seed=7)
    ids, w = routing.zipf_routing(rng, 1, E, K)
    x = rng.standard_normal((1, D)).astype(np.float32)
    ex = MoEExecutor(bank, max_used=K)
    out = ex.run_layer(0, T(x), T(ids), T(w))
    torch.cuda.synchronize()
    used = np.unique(ids)
    remap = {int(e): i for i, e in enumerate(used)}
    sub = {r: np.stack([bank.read_expert(0, r, int(e)) for e in used]) for r in ("gate", "up", "down")}
    # weights look like quantised N(0, 0.02): the decoded spread is in range
    dq = orc.dequantize(IQ3_S, sub["gate"][0], D)
    assert 0.012 < dq.std() < 0.03
    ids_local = np.vectorize(remap.get)(ids).astype(np.int32)
    want = orc.moe_layer(sub["gate"], sub["up"], sub["down"], (IQ3_S,) * 3, x, ids_local, w)
    assert_parity(out.cpu().numpy(), want, "full-size layer")
