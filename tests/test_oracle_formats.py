"""Pins of the CPU oracle (oracle/ggml_cpu_ref.c) - no GPU.

Each check fixes a quantity by something other than the oracle's own formula:
hand-built blocks with closed-form values, numpy's IEEE fp16 conversion,
tie cases that separate rounding modes, exact integer brute force, and
float64 recomputation from independently decoded operands.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from helpers import dequant_act, f16, max_rel, random_blocks, unfused_rounding_row

Q8_0, Q4_K, Q6_K, Q8_K, IQ3_S = 8, 12, 14, 15, 21


# ---------------------------------------------------------------------------
# binary16
# ---------------------------------------------------------------------------
def test_fp32_to_fp16_matches_numpy_round_to_nearest_even(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                  2 ** -14, 2 ** -14 - 2 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.fp32_to_fp16_bits(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_fp16_to_fp32_is_exact_for_every_finite_half(orc):
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    h = h[((h >> 10) & 0x1F) != 0x1F]                     # finite halves
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.fp16_bits_to_fp32(int(b)) for b in h[::7]], np.float32)
    assert np.array_equal(got.view(np.uint32), want[::7].view(np.uint32))


# ---------------------------------------------------------------------------
# decoders: hand-built blocks with closed-form values
# ---------------------------------------------------------------------------
def test_q8_0_known_answer(orc):
    blk = f16(0.5) + bytes(((j - 16) & 0xFF) for j in range(32))
    y = orc.dequantize(Q8_0, np.frombuffer(blk, np.uint8), 32)
    assert np.array_equal(y, (np.arange(32) - 16) * 0.5)


def _q4k_block(d, dmin, sc, mn, q):
    p = bytearray(12)
    for j in range(4):
        p[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        p[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        p[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return f16(d) + f16(dmin) + bytes(p) + bytes(qs)


def test_q4_K_known_answer_scales_and_mins(orc):
    sc = [1, 2, 3, 4, 37, 50, 63, 17]          # sub-blocks 4..7 exercise the split 6-bit packing
    mn = [0, 5, 9, 13, 40, 63, 21, 33]
    q = [(7 * e + 3) % 16 for e in range(256)]
    blk = _q4k_block(0.5, 0.25, sc, mn, q)
    y = orc.dequantize(Q4_K, np.frombuffer(blk, np.uint8), 256)
    want = np.array([0.5 * sc[e // 32] * q[e] - 0.25 * mn[e // 32] for e in range(256)])
    assert np.array_equal(y, want.astype(np.float32))


def test_q6_K_known_answer(orc):
    u = [(5 * e + 11) % 64 for e in range(256)]     # unsigned 6-bit values
    ql, qh = bytearray(128), bytearray(64)
    for half in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (u[128 * half + 32 * s + l] for s in range(4))
            ql[64 * half + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * half + 32 + l] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * half + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    sc = [((-1) ** j) * (j + 1) for j in range(16)]
    blk = bytes(ql) + bytes(qh) + bytes((s & 0xFF) for s in sc) + f16(0.25)
    y = orc.dequantize(Q6_K, np.frombuffer(blk, np.uint8), 256)
    want = np.array([0.25 * sc[e // 16] * (u[e] - 32) for e in range(256)], np.float32)
    assert np.array_equal(y, want)


def _iq3s_block(d, qs, qh, signs, scales):
    b = lambda a: bytes(int(v) & 0xFF for v in a)
    return f16(d) + b(qs) + b(qh) + b(signs) + b(scales)


def test_iq3_S_known_answer_grid_rows(orc):
    from helpers import oracle_iq3s_grid
    grid = oracle_iq3s_grid()
    for start in (0, 64, 448):                       # qh bit selects the upper half of the grid
        idx = [start + i for i in range(64)]
        qs = [i & 0xFF for i in idx]
        qh = [0xFF if start >= 256 else 0] * 8
        blk = _iq3s_block(1.0, qs, qh, [0] * 32, [0] * 4)
        y = orc.dequantize(IQ3_S, np.frombuffer(blk, np.uint8), 256)
        want = [(grid[i] >> (8 * j)) & 0xFF for i in idx for j in range(4)]
        assert np.array_equal(y, np.array(want, np.float32)), start


def test_iq3_S_signs_qh_and_scales(orc):
    from helpers import oracle_iq3s_grid
    grid = oracle_iq3s_grid()
    rng = np.random.default_rng(5)
    qs = rng.integers(0, 256, 64)
    qh = rng.integers(0, 256, 8)
    signs = rng.integers(0, 256, 32)
    scales = rng.integers(0, 256, 4)
    blk = _iq3s_block(0.125, qs, qh, signs, scales)
    y = orc.dequantize(IQ3_S, np.frombuffer(blk, np.uint8), 256)
    want = []
    for ib in range(8):
        s = (scales[ib // 2] >> (4 * (ib % 2))) & 15
        for g in range(8):
            gi = int(qs[8 * ib + g]) | (((int(qh[ib]) >> g) & 1) << 8)
            sg = int(signs[4 * ib + g // 2])
            for j in range(4):
                mag = (grid[gi] >> (8 * j)) & 0xFF
                neg = (sg >> (4 * (g % 2) + j)) & 1
                want.append(0.125 * (1 + 2 * s) * mag * (-1 if neg else 1))
    assert np.array_equal(y, np.array(want, np.float32))


# ---------------------------------------------------------------------------
# activation quantisers: ties and sign conventions
# ---------------------------------------------------------------------------
def test_q8_0_rounds_halves_away_from_zero(orc):
    x = np.zeros(32, np.float32)
    x[0] = 127.0                                     # d = 1 exactly, 1/d = 1
    x[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -3.4999]
    y = orc.quantize_q8_0(x)
    assert y[:2].view(np.float16)[0] == 1.0
    q = y[2:].view(np.int8)
    assert list(q[:9]) == [127, 3, -3, 1, -1, 2, -2, 127, -3]


def test_q8_0_zero_block(orc):
    y = orc.quantize_q8_0(np.zeros(64, np.float32))
    assert not y.any()


def test_q8_K_ties_round_to_even_and_scale_sign(orc):
    x = np.zeros(256, np.float32)
    x[0] = -127.0                                    # signed max -127 -> iscale = +1
    x[1:8] = [2.5, -2.5, 3.5, 0.5, 1.5, -1.5, 126.5]
    y = orc.quantize_q8_K(x)
    assert y[:4].view(np.float32)[0] == 1.0
    q = y[4:260].view(np.int8)
    assert list(q[:8]) == [-127, 2, -2, 4, 0, 2, -2, 126]
    x[0] = 127.0                                     # signed max +127 -> iscale = -1, d = -1
    y = orc.quantize_q8_K(x)
    assert y[:4].view(np.float32)[0] == -1.0
    q = y[4:260].view(np.int8)
    assert list(q[:8]) == [-127, -2, 2, -4, 0, -2, 2, -126]


def test_q8_K_first_maximum_wins_and_clamps_at_127(orc):
    x = np.zeros(256, np.float32)
    x[3], x[10] = 5.0, -5.0                          # equal magnitudes: the first sets the sign
    y = orc.quantize_q8_K(x)
    q = y[4:260].view(np.int8)
    assert q[3] == -127 and q[10] == 127
    d = y[:4].view(np.float32)[0]
    assert d == np.float32(1.0) / (np.float32(-127.0) / np.float32(5.0))


def test_q8_K_constant_zero_block_and_bsums(orc):
    y = orc.quantize_q8_K(np.full(256, 0.75, np.float32))
    assert np.all(y[4:260].view(np.int8) == -127)
    assert np.all(y[260:292].view(np.int16) == -127 * 16)
    assert not orc.quantize_q8_K(np.zeros(512, np.float32)).any()
    rng = np.random.default_rng(2)
    y = orc.quantize_q8_K(rng.standard_normal(256).astype(np.float32))
    q = y[4:260].view(np.int8).astype(np.int64)
    assert np.array_equal(y[260:292].view(np.int16), q.reshape(16, 16).sum(axis=1))
    assert np.abs(q).max() == 127


def test_q8_K_rounds_the_product_before_the_round_to_int_add(orc):
    # ggml's nearest_int(iscale * x): the product is an fp32 value of its own,
    # so values whose exact product rounds the other way stay on the fp32 side.
    x = unfused_rounding_row(256)
    y = orc.quantize_q8_K(x)
    iscale = np.float32(-127.0) / np.float32(3.0)
    q = y[4:260].view(np.int8).astype(np.int64)
    assert np.array_equal(q, np.rint(iscale * x).astype(np.int64))          # fp32 product, RNE
    fused = np.rint(x.astype(np.float64) * float(iscale)).astype(np.int64)  # one rounding
    assert np.all(fused[1:] != q[1:])


# ---------------------------------------------------------------------------
# block dots: exact integers and float64 recomputation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qt,k", [(Q8_0, 256), (Q4_K, 512), (Q6_K, 512), (IQ3_S, 512)])
def test_vec_dot_matches_float64_of_decoded_operands(orc, qt, k):
    rng = np.random.default_rng(qt)
    raw = random_blocks(rng, qt, 8, k)
    w = orc.dequantize(qt, raw, k).astype(np.float64)
    for r in range(8):
        x = rng.standard_normal(k).astype(np.float32)
        a = orc.quantize_act(qt, x[None])[0]
        ref = float(w[r] @ dequant_act(orc, qt, a, k))
        got = orc.vec_dot(qt, raw[r], a, k)
        scale = float(np.abs(w[r]).max() * np.abs(dequant_act(orc, qt, a, k)).sum())
        assert abs(got - ref) <= 1e-6 * scale, (qt, r, got, ref)


def test_iq3_S_dot_is_the_exact_integer_sum(orc):
    from helpers import oracle_iq3s_grid
    grid = oracle_iq3s_grid()
    rng = np.random.default_rng(9)
    qs, qh = rng.integers(0, 256, 64), rng.integers(0, 256, 8)
    signs, scales = rng.integers(0, 256, 32), rng.integers(0, 256, 4)
    blk = np.frombuffer(_iq3s_block(1.0, qs, qh, signs, scales), np.uint8)
    xi = rng.integers(-126, 127, 256).astype(np.float32)
    xi[17] = -127.0                                  # activation scale d = 1 exactly
    a = orc.quantize_q8_K(xi)
    assert a[:4].view(np.float32)[0] == 1.0
    total = 0
    for ib in range(8):
        ls = 2 * ((int(scales[ib // 2]) >> (4 * (ib % 2))) & 15) + 1
        for g in range(8):
            gi = int(qs[8 * ib + g]) | (((int(qh[ib]) >> g) & 1) << 8)
            for j in range(4):
                mag = (grid[gi] >> (8 * j)) & 0xFF
                neg = (int(signs[4 * ib + g // 2]) >> (4 * (g % 2) + j)) & 1
                total += ls * mag * (-1 if neg else 1) * int(xi[32 * ib + 4 * g + j])
    assert orc.vec_dot(IQ3_S, blk, a, 256) == float(total)


def test_q4_K_min_term_uses_bsums(orc):
    """A block whose only content is the min term: every nibble 0, so the dot is
    -dmin*d8*sum_j m_j*bsum(j) exactly."""
    mn = [1, 2, 3, 4, 5, 6, 7, 8]
    blk = np.frombuffer(_q4k_block(1.0, 1.0, [0] * 8, mn, [0] * 256), np.uint8)
    xi = np.arange(256, dtype=np.float32) % 11 - 5
    xi[0] = -127.0
    a = orc.quantize_q8_K(xi)
    want = -sum(mn[e // 32] * int(xi[e]) for e in range(256))
    assert orc.vec_dot(Q4_K, blk, a, 256) == float(want)


# ---------------------------------------------------------------------------
# MUL_MAT_ID semantics and the combine
# ---------------------------------------------------------------------------
def _bank(orc, rng, qt, E, rows, k):
    w = (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32)
    return orc.quantize_weights(qt, w)


@pytest.mark.parametrize("x_rows_is_n_ids", [False, True])
def test_mul_mat_id_brute_force(orc, x_rows_is_n_ids):
    rng = np.random.default_rng(11)
    qt, E, rows, k, T, K = IQ3_S, 6, 24, 512, 3, 4
    bank = _bank(orc, rng, qt, E, rows, k)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    ids[1, 2] = ids[1, 0]                            # a duplicate id inside one token
    x_rows = K if x_rows_is_n_ids else 1
    x = rng.standard_normal((T, x_rows, k)).astype(np.float32)
    got = orc.mul_mat_id(bank, x, ids, rows, k, qt)
    W = orc.dequantize(qt, bank, k).astype(np.float64)
    for t in range(T):
        for i in range(K):
            a = orc.quantize_act(qt, x[t, i % x_rows][None])[0]
            ref = W[ids[t, i]] @ dequant_act(orc, qt, a, k)
            assert max_rel(got[t, i], ref) < 1e-6
    if x_rows == 1:
        assert np.array_equal(got[1, 2], got[1, 0])  # duplicate slots are identical


def test_mul_mat_id_rejects_bad_ids_and_geometry(orc):
    rng = np.random.default_rng(3)
    bank = _bank(orc, rng, Q8_0, 2, 8, 64)
    x = np.zeros((1, 1, 64), np.float32)
    with pytest.raises(ValueError):
        orc.mul_mat_id(bank, x, np.array([[2]], np.int32), 8, 64, Q8_0)
    with pytest.raises(ValueError):
        orc.mul_mat_id(bank, np.zeros((1, 2, 64), np.float32), np.array([[0, 1, 1]], np.int32), 8, 64, Q8_0)


def test_moe_layer_is_the_composition_of_mul_mat_ids(orc):
    """One layer = gate/up MUL_MAT_ID, silu(g)*u, down MUL_MAT_ID on h, weighted serial sum."""
    rng = np.random.default_rng(21)
    qt, E, D, F, T, K = Q4_K, 5, 512, 256, 2, 3
    g, u = _bank(orc, rng, qt, E, F, D), _bank(orc, rng, qt, E, F, D)
    dn = _bank(orc, rng, qt, E, D, F)
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    out, h = orc.moe_layer(g, u, dn, (qt, qt, qt), x, ids, w, return_h=True)
    G = orc.mul_mat_id(g, x[:, None], ids, F, D, qt)
    U = orc.mul_mat_id(u, x[:, None], ids, F, D, qt)
    H = (G / (np.float32(1) + np.exp(-G))) * U
    assert max_rel(h, H) < 1e-6
    Y = orc.mul_mat_id(dn, h, ids, D, F, qt)
    for t in range(T):
        acc = Y[t, 0] * w[t, 0]
        for s in range(1, K):
            acc = acc + Y[t, s] * w[t, s]
        assert np.array_equal(out[t], acc)
    # one-hot weights pick out one slot's down output
    one = np.zeros_like(w)
    one[:, 1] = 1.0
    assert np.array_equal(orc.moe_layer(g, u, dn, (qt, qt, qt), x, ids, one), Y[:, 1])


def test_moe_layer_shared_expert_is_added_last(orc):
    rng = np.random.default_rng(22)
    D, F, Fs, E = 256, 256, 256, 3
    g, u = _bank(orc, rng, Q4_K, E, F, D), _bank(orc, rng, Q4_K, E, F, D)
    dn = _bank(orc, rng, Q6_K, E, D, F)
    sg, su = _bank(orc, rng, Q8_0, 1, Fs, D)[0], _bank(orc, rng, Q8_0, 1, Fs, D)[0]
    sd = _bank(orc, rng, Q8_0, 1, D, Fs)[0]
    x = rng.standard_normal((1, D)).astype(np.float32)
    ids = np.array([[2, 0]], np.int32)
    w = np.array([[0.7, 0.3]], np.float32)
    routed = orc.moe_layer(g, u, dn, (Q4_K, Q4_K, Q6_K), x, ids, w)
    both = orc.moe_layer(g, u, dn, (Q4_K, Q4_K, Q6_K), x, ids, w, shared=(sg, su, sd, (Q8_0, Q8_0, Q8_0)))
    shared_only = orc.moe_layer(sg[None], su[None], sd[None], (Q8_0, Q8_0, Q8_0), x,
                                np.array([[0]], np.int32), np.array([[1.0]], np.float32))
    assert np.array_equal(both, routed + shared_only)


def test_moe_layer_gated_shared_expert_closed_forms(orc):
    """qwen4exp.cpp:877-885: the shared expert's output is multiplied by
    sigmoid(gate_inp . x) and then added.  Rows that make the logit 0, +big and
    -big give g = 0.5, 1 and 0 exactly, so the gated layer is pinned bit for bit
    against the routed part and the ungated shared output; a random row is
    checked against a float64 sigmoid."""
    rng = np.random.default_rng(23)
    D, F, Fs, E, T = 256, 256, 256, 4, 3
    g, u = _bank(orc, rng, Q4_K, E, F, D), _bank(orc, rng, Q4_K, E, F, D)
    dn = _bank(orc, rng, Q6_K, E, D, F)
    sg, su = _bank(orc, rng, Q8_0, 1, Fs, D)[0], _bank(orc, rng, Q8_0, 1, Fs, D)[0]
    sd = _bank(orc, rng, Q8_0, 1, D, Fs)[0]
    x = rng.standard_normal((T, D)).astype(np.float32)
    ids = np.array([[2, 0], [1, 3], [3, 3]], np.int32)
    w = np.array([[0.7, 0.3], [0.5, 0.5], [0.9, 0.1]], np.float32)
    qts, sq = (Q4_K, Q4_K, Q6_K), (Q8_0, Q8_0, Q8_0)
    routed = orc.moe_layer(g, u, dn, qts, x, ids, w)
    ys = np.stack([orc.moe_layer(sg[None], su[None], sd[None], sq, x[t:t + 1], np.array([[0]], np.int32),
                                 np.array([[1.0]], np.float32))[0] for t in range(T)])
    ungated = orc.moe_layer(g, u, dn, qts, x, ids, w, shared=(sg, su, sd, sq))
    assert np.array_equal(ungated, routed + ys)

    def gated(row):
        return orc.moe_layer(g, u, dn, qts, x, ids, w, shared=(sg, su, sd, sq, row))
    assert np.array_equal(gated(np.zeros(D, np.float32)), routed + ys * np.float32(0.5))
    for t in range(T):       # a row along x[t] makes that token's logit +-|x|^2 * 1e4
        up = gated(1e4 * x[t])[t]
        assert np.array_equal(up, ungated[t])
        down = gated(-1e4 * x[t])[t]
        assert np.array_equal(down, routed[t])
    row = (rng.standard_normal(D) * 0.05).astype(np.float32)
    logit = x.astype(np.float64) @ row.astype(np.float64)
    gate = 1.0 / (1.0 + np.exp(-logit))
    want = routed.astype(np.float64) + ys.astype(np.float64) * gate[:, None]
    assert max_rel(gated(row), want) < 1e-6
    with pytest.raises(ValueError):
        gated(np.zeros(D + 1, np.float32))


def test_encoders_round_trip(orc):
    rng = np.random.default_rng(4)
    for qt, k, tol in [(Q8_0, 512, 0.01), (Q4_K, 512, 0.12), (Q6_K, 512, 0.03), (IQ3_S, 512, 0.25)]:
        w = (rng.standard_normal((16, k)) * 0.02).astype(np.float32)
        back = orc.dequantize(qt, orc.quantize_weights(qt, w), k)
        err = np.linalg.norm(back - w) / np.linalg.norm(w)
        assert err < tol, (qt, err)


# ---------------------------------------------------------------------------
# IQ3_XXS, IQ4_NL, IQ4_XS (sabah_rt.cu:2320-2344, 2380-2409; quants.py:1039-1075, 1364-1411)
# ---------------------------------------------------------------------------
IQ3_XXS, IQ4_NL, IQ4_XS = 18, 20, 23
KV = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def test_iq4_nl_known_answer(orc):
    qs = bytes((j | ((15 - j) << 4)) for j in range(16))
    blk = np.frombuffer(f16(1.0) + qs, np.uint8)
    y = orc.dequantize(IQ4_NL, blk, 32)
    assert y[:16].tolist() == KV and y[16:].tolist() == KV[::-1]
    blk = np.frombuffer(f16(0.5) + qs, np.uint8)
    assert np.array_equal(orc.dequantize(IQ4_NL, blk, 32), y * np.float32(0.5))


def test_iq4_xs_known_answer_scales(orc):
    """ls of sub-block ib = scales_l nibble ib | 2 bits ib of scales_h << 4; value d*(ls-32)*kv[q]."""
    ls = [33, 32, 63, 0, 40, 17, 48, 31]
    sh = sum(((v >> 4) & 3) << (2 * i) for i, v in enumerate(ls))
    sl = bytes((ls[2 * i] & 15) | ((ls[2 * i + 1] & 15) << 4) for i in range(4))
    qs = bytes((j % 16) | (((j + 5) % 16) << 4) for j in range(128))
    blk = np.frombuffer(f16(1.0) + struct.pack("<H", sh) + sl + qs, np.uint8)
    y = orc.dequantize(IQ4_XS, blk, 256).reshape(8, 32)
    for ib in range(8):
        q = [j % 16 for j in range(16 * ib, 16 * ib + 16)]
        want = [KV[v] * (ls[ib] - 32) for v in q] + [KV[(v + 5) % 16] * (ls[ib] - 32) for v in q]
        assert y[ib].tolist() == want, ib


def test_iq3_xxs_known_answer_grid_signs_and_scale(orc):
    from helpers import oracle_table
    grid = oracle_table("orc_iq3xxs_grid")
    qs = np.arange(64, dtype=np.uint8) * 3            # grid entries 0, 3, ..., 189
    aux = []
    for ib in range(8):           # sign indices (7 bits each) and the scale nibble
        s7 = [(5 * ib + l) & 127 for l in range(4)]
        aux.append(s7[0] | (s7[1] << 7) | (s7[2] << 14) | (s7[3] << 21) | (ib << 28))
    blk = np.frombuffer(f16(1.0) + qs.tobytes() + struct.pack("<8I", *aux), np.uint8)
    y = orc.dequantize(IQ3_XXS, blk, 256)
    for ib in range(8):
        db = (0.5 + ib) * 0.5
        for l in range(4):
            s7 = (5 * ib + l) & 127
            sg = s7 | ((bin(s7).count("1") & 1) << 7)
            for h in range(2):
                g = grid[int(qs[8 * ib + 2 * l + h])]
                for j in range(4):
                    e = 32 * ib + 8 * l + 4 * h + j
                    sign = -1.0 if (sg >> (4 * h + j)) & 1 else 1.0
                    assert y[e] == np.float32(db * ((g >> (8 * j)) & 0xFF) * sign), (ib, l, h, j)


IQ2_S = 22


def iq2s_block(qs, signs, qh, scales, d=1.0):
    return np.frombuffer(f16(d) + bytes(qs) + bytes(signs) + bytes(qh) + bytes(scales), np.uint8)


def test_iq2_s_known_answer_grid_qh_signs_and_scales(orc):
    """element 32 ib + 8 l + j = db * grid[qs[4 ib + l] | qh bits 2l, 2l+1 << 8][j] * sign bit j;
    db = d * (0.5 + nibble) * 0.25 with the low nibble of scales[ib] for l < 2, the high one after
    (sabah_rt.cu:2293-2318; quants.py:1007-1037)."""
    from helpers import oracle_table
    grid = oracle_table("orc_iq2s_grid")
    qs = [(37 * i + 5) & 255 for i in range(32)]
    signs = [(29 * i + 3) & 255 for i in range(32)]
    qh = [(0x1B * (i + 1)) & 255 for i in range(8)]         # every 2-bit pattern occurs
    scales = [(i | ((15 - 2 * i) << 4)) & 255 for i in range(8)]
    y = orc.dequantize(IQ2_S, iq2s_block(qs, signs, qh, scales), 256)
    for ib in range(8):
        for l in range(4):
            gi = qs[4 * ib + l] | (((qh[ib] >> (2 * l)) & 3) << 8)
            nib = (scales[ib] & 15) if l < 2 else (scales[ib] >> 4)
            db = (0.5 + nib) * 0.25
            for j in range(8):
                sign = -1.0 if (signs[4 * ib + l] >> j) & 1 else 1.0
                e = 32 * ib + 8 * l + j
                assert y[e] == np.float32(db * ((grid[gi] >> (8 * j)) & 0xFF) * sign), (ib, l, j)


def test_iq2_s_dot_is_an_eighth_of_the_exact_integer_sum(orc):
    from helpers import oracle_table
    grid = oracle_table("orc_iq2s_grid")
    rng = np.random.default_rng(14)
    qs, signs = rng.integers(0, 256, 32), rng.integers(0, 256, 32)
    qh, scales = rng.integers(0, 256, 8), rng.integers(0, 256, 8)
    blk = iq2s_block(qs.astype(np.uint8), signs.astype(np.uint8), qh.astype(np.uint8), scales.astype(np.uint8))
    xi = rng.integers(-126, 127, 256).astype(np.float32)
    xi[7] = -127.0                                     # activation scale d = 1 exactly
    a = orc.quantize_q8_K(xi)
    total = 0
    for ib in range(8):
        for l in range(4):
            gi = int(qs[4 * ib + l]) | (((int(qh[ib]) >> (2 * l)) & 3) << 8)
            ls = 2 * ((int(scales[ib]) & 15) if l < 2 else (int(scales[ib]) >> 4)) + 1
            for j in range(8):
                s = -1 if (int(signs[4 * ib + l]) >> j) & 1 else 1
                total += ls * ((grid[gi] >> (8 * j)) & 0xFF) * s * int(xi[32 * ib + 8 * l + j])
    assert orc.vec_dot(IQ2_S, blk, a, 256) == np.float32(0.125) * np.float32(total)


@pytest.mark.parametrize("qt,k", [(IQ3_XXS, 512), (IQ4_NL, 256), (IQ4_XS, 512), (IQ2_S, 512)])
def test_new_iq_dots_match_float64_of_decoded_operands(orc, qt, k):
    rng = np.random.default_rng(qt + 100)
    raw = random_blocks(rng, qt, 8, k)
    w = orc.dequantize(qt, raw, k).astype(np.float64)
    for r in range(8):
        x = rng.standard_normal(k).astype(np.float32)
        a = orc.quantize_act(qt, x[None])[0]
        ref = float(w[r] @ dequant_act(orc, qt, a, k))
        got = orc.vec_dot(qt, raw[r], a, k)
        scale = float(np.abs(w[r]).max() * np.abs(dequant_act(orc, qt, a, k)).sum())
        assert abs(got - ref) <= 1e-6 * scale, (qt, r, got, ref)


def test_iq3_xxs_dot_is_a_quarter_of_the_exact_integer_sum(orc):
    from helpers import oracle_table
    grid = oracle_table("orc_iq3xxs_grid")
    rng = np.random.default_rng(12)
    qs = rng.integers(0, 256, 64).astype(np.uint8)
    aux = rng.integers(0, 2 ** 32, 8, dtype=np.uint64).astype(np.uint32)
    blk = np.frombuffer(f16(1.0) + qs.tobytes() + aux.tobytes(), np.uint8)
    xi = rng.integers(-126, 127, 256).astype(np.float32)
    xi[3] = -127.0                                     # activation scale d = 1 exactly
    a = orc.quantize_q8_K(xi)
    total = 0
    for ib in range(8):
        v = int(aux[ib])
        ls = 2 * (v >> 28) + 1
        for l in range(4):
            s7 = (v >> (7 * l)) & 127
            sg = s7 | ((bin(s7).count("1") & 1) << 7)
            for h in range(2):
                g = grid[int(qs[8 * ib + 2 * l + h])]
                for j in range(4):
                    e = 32 * ib + 8 * l + 4 * h + j
                    total += ls * ((g >> (8 * j)) & 0xFF) * (-1 if (sg >> (4 * h + j)) & 1 else 1) * int(xi[e])
    assert orc.vec_dot(IQ3_XXS, blk, a, 256) == np.float32(0.25) * np.float32(total)


@pytest.mark.parametrize("qt", [IQ4_NL, IQ4_XS])
def test_iq4_encoders_round_trip(orc, qt):
    rng = np.random.default_rng(qt)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    back = orc.dequantize(qt, orc.quantize_weights(qt, w), 512)
    assert np.sqrt(np.mean((back - w) ** 2)) < 0.15 * np.sqrt(np.mean(w ** 2))
