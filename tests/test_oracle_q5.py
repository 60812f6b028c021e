"""Pins of the oracle's Q5_1, Q5_K and q8_1 code (oracle/ggml_cpu_ref.c) - no GPU.

The formats as the reference reads them (sabah_rt.cu:2241-2290, 2487-2541;
gguf-py quants.py:367-409, 559-583): Q5_1 blocks of 32 (fp16 d, fp16 m, u32
qh, 16 nibble bytes: element j < 16 is the low nibble of qs[j] plus bit j of
qh times 16, element j + 16 the high nibble plus bit j + 16; value d q + m);
Q5_K super-blocks of 256 (Q4_K's d, dmin and 6-bit scales and mins, then
qh[32], then qs[128]: element l of sub-block j is the nibble of
qs[32 (j / 2) + l] plus bit j of qh[l] times 16).  ggml pairs Q5_1 with q8_1
activations (q8_0's bytes plus s = fp16(sum q * d)) and Q5_K with q8_K.

Each value is fixed by something other than the oracle's own formula:
hand-built blocks with one bit set at a time, Q5_K with qh = 0 against the
already pinned Q4_K decoder, numpy's fp16 for q8_1's scale and sum, and
float64 recomputation of the dots from independently decoded operands.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from helpers import dequant_act, f16, random_blocks

Q5_1, Q8_1, Q4_K, Q5_K, Q8_K = 7, 9, 12, 13, 15


def _q5_1_block(d, m, qh, qs):
    return f16(d) + f16(m) + struct.pack("<I", qh) + bytes(qs)


def test_q5_1_each_fifth_bit_lands_on_its_element(orc):
    # every nibble 0: only the element whose qh bit is set reads 16
    for bit in (0, 5, 15, 16, 21, 31):
        blk = np.frombuffer(_q5_1_block(1.0, 0.0, 1 << bit, [0] * 16), np.uint8)
        y = orc.dequantize(Q5_1, blk, 32)
        want = np.zeros(32, np.float32)
        want[bit] = 16.0
        assert np.array_equal(y, want), bit


def test_q5_1_nibbles_scale_and_offset(orc):
    # low nibble of qs[j] is element j, high nibble element j + 16
    qs = [(j & 15) | ((15 - j) << 4) for j in range(16)]
    blk = np.frombuffer(_q5_1_block(0.5, -3.0, 0xFFFF0000, qs), np.uint8)
    y = orc.dequantize(Q5_1, blk, 32)
    lo = [0.5 * j - 3.0 for j in range(16)]
    hi = [0.5 * (15 - j + 16) - 3.0 for j in range(16)]
    assert np.array_equal(y, np.array(lo + hi, np.float32))


def _q5k_block(d, dmin, sc, mn, q):
    p = bytearray(12)
    for j in range(4):
        p[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        p[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        p[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    qh, qs = bytearray(32), bytearray(128)
    for j in range(8):
        for l in range(32):
            v = q[32 * j + l]
            qs[32 * (j // 2) + l] |= (v & 15) << (4 * (j & 1))
            qh[l] |= (v >> 4) << j
    return f16(d) + f16(dmin) + bytes(p) + bytes(qh) + bytes(qs)


def test_q5_K_without_fifth_bits_is_q4_K(orc):
    rng = np.random.default_rng(51)
    for _ in range(4):
        q4 = random_blocks(rng, Q4_K, 1, 256)[0]
        # the same d, dmin, scales and nibbles with qh = 0
        q5 = np.concatenate([q4[:16], np.zeros(32, np.uint8), q4[16:]])
        assert np.array_equal(orc.dequantize(Q5_K, q5, 256), orc.dequantize(Q4_K, q4, 256))


def test_q5_K_known_answer_fifth_bits_scales_and_mins(orc):
    sc = [1, 2, 3, 4, 37, 50, 63, 17]
    mn = [0, 5, 9, 13, 40, 63, 21, 33]
    q = [(11 * e + 5) % 32 for e in range(256)]
    blk = np.frombuffer(_q5k_block(0.5, 0.25, sc, mn, q), np.uint8)
    y = orc.dequantize(Q5_K, blk, 256)
    want = np.array([0.5 * sc[e // 32] * q[e] - 0.25 * mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_q5_K_qh_bit_j_of_byte_l_is_element_32j_plus_l(orc):
    for j, l in ((0, 0), (2, 7), (5, 31), (7, 19)):
        q = [0] * 256
        q[32 * j + l] = 16
        blk = np.frombuffer(_q5k_block(1.0, 0.0, [1] * 8, [0] * 8, q), np.uint8)
        assert bin(int(blk[16 + l])).count("1") == 1 and (blk[16 + l] >> j) & 1
        y = orc.dequantize(Q5_K, blk, 256)
        want = np.zeros(256, np.float32)
        want[32 * j + l] = 16.0
        assert np.array_equal(y, want), (j, l)


def test_q8_1_is_q8_0_plus_the_scaled_sum(orc):
    rng = np.random.default_rng(81)
    x = rng.standard_normal(256).astype(np.float32) * 3
    x[:32] = 0.0                                   # a zero block: d = s = 0
    a = orc.quantize_q8_1(x).reshape(-1, 36)
    a0 = orc.quantize_q8_0(x).reshape(-1, 34)
    assert np.array_equal(a[:, :2], a0[:, :2]) and np.array_equal(a[:, 4:], a0[:, 2:])
    for b in range(8):
        blk = x[32 * b:32 * b + 32]
        d = np.float32(np.abs(blk).max()) / np.float32(127.0)     # fp32 d, before its fp16 rounding
        qsum = int(a[b, 4:].view(np.int8).astype(np.int64).sum())
        want = np.float16(np.float32(qsum) * d) if d else np.float16(0)
        assert a[b, 2:4].copy().view(np.float16)[0] == want, b
    assert not a[0].any()


def test_q8_1_hand_block(orc):
    x = np.arange(32, dtype=np.float32) - 15.0     # amax 16: d = 16/127, q = round(x * 127/16)
    a = orc.quantize_q8_1(x)
    d = np.float32(16.0) / np.float32(127.0)
    q = np.array([np.sign(v) * np.floor(abs(v) * (np.float32(1.0) / d) + 0.5) for v in x], np.int64)
    assert np.array_equal(a[4:].view(np.int8).astype(np.int64), q)
    assert a[:2].copy().view(np.float16)[0] == np.float16(d)
    assert a[2:4].copy().view(np.float16)[0] == np.float16(np.float32(q.sum()) * d)


@pytest.mark.parametrize("qt,k", [(Q5_1, 256), (Q5_1, 96), (Q5_K, 512)])
def test_q5_dots_match_float64_of_decoded_operands(orc, qt, k):
    rng = np.random.default_rng(qt + k)
    raw = random_blocks(rng, qt, 8, k)
    w = orc.dequantize(qt, raw, k).astype(np.float64)
    for r in range(8):
        x = rng.standard_normal(k).astype(np.float32)
        a = orc.quantize_act(qt, x[None])[0]
        xa = dequant_act(orc, qt, a, k)
        if qt == Q5_1:
            # d_x sum(q_w q_x) d_w + m_w s_x per block, with s_x the stored fp16 value
            blk = a.reshape(-1, 36)
            s = blk[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1)
            m = raw[r].reshape(-1, 24)[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1)
            qw = (w[r].reshape(-1, 32) - m[:, None])              # d_w q_w
            ref = float((qw * xa.reshape(-1, 32)).sum() + (m * s).sum())
        else:
            ref = float(w[r] @ xa)
        got = orc.vec_dot(qt, raw[r], a, k)
        scale = float(np.abs(w[r]).max() * np.abs(xa).sum())
        assert abs(got - ref) <= 2e-6 * scale, (qt, r, got, ref)


def test_q5_1_dot_sums_blocks_in_order(orc):
    """Per block, (d_w d_x) sumi + m_w s_x, added to the running fp32 sum in
    block order: two blocks whose terms cancel only in that order."""
    xq = np.zeros(64, np.float32)
    xq[0], xq[32] = 127.0, 127.0                   # d_x = 1, s_x = 127 in both blocks
    a = orc.quantize_q8_1(xq)
    assert a[:2].copy().view(np.float16)[0] == 1.0 and a[2:4].copy().view(np.float16)[0] == 127.0
    b0 = _q5_1_block(1.0, 0.0, 0, [31 & 15] + [0] * 15)    # q_w[0] = 15: term 15 * 127
    b1 = _q5_1_block(2.0 ** -11, 0.0, 0, [1] + [0] * 15)     # tiny term, lost after a large sum
    w = np.frombuffer(b0 + b1, np.uint8)
    t0 = np.float32(np.float32(1.0) * np.float32(15 * 127)) + np.float32(0.0)
    t1 = np.float32(np.float32(2.0 ** -11) * np.float32(127)) + np.float32(0.0)
    want = np.float32(np.float32(np.float32(0.0) + t0) + t1)
    assert orc.vec_dot(Q5_1, w, a, 64) == float(want)


def test_q5_encoders_round_trip(orc):
    rng = np.random.default_rng(55)
    for qt, k, tol in [(Q5_1, 512, 0.06), (Q5_K, 512, 0.06)]:
        w = (rng.standard_normal((16, k)) * 0.02).astype(np.float32)
        back = orc.dequantize(qt, orc.quantize_weights(qt, w), k)
        err = np.linalg.norm(back - w) / np.linalg.norm(w)
        assert err < tol, (qt, err)


def test_the_q8_1_tie_row_separates_one_rounding_from_two(orc):
    """The GPU test's regression row (helpers.q8_1_tie_row): every block's
    fl32(sum(q) * d) is an exact fp16 tie, and for many blocks rounding the
    exact product to fp16 once gives the other half than the oracle's s."""
    from helpers import q8_1_tie_row
    row = q8_1_tie_row(2048)
    a = orc.quantize_q8_1(row).reshape(-1, 36)
    differ = 0
    for b in range(64):
        blk = row[32 * b:32 * b + 32]
        d = np.float32(np.abs(blk).max()) / np.float32(127.0)
        qsum = int(a[b, 4:].view(np.int8).astype(np.int64).sum())
        p32 = np.float32(np.float32(qsum) * d)
        lo = np.float16(p32)
        assert a[b, 2:4].copy().view(np.float16)[0] == lo
        assert float(p32) != float(qsum) * float(d)
        differ += np.float16(float(qsum) * float(d)) != lo
    assert differ >= 16
