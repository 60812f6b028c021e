"""Pins of the oracle's Q2_0 (ggml type 42): 64-element blocks of 18 bytes,
fp16 d then 16 bytes of 2-bit codes, element j = (code j - 1) * d with code j
at bits 2*(j % 4) of byte j / 4 (sabah_rt.cu:2411-2419 host, 2547-2557
device; gguf-py quants.py:224-235).

The decoder is pinned by hand-built blocks whose values follow from that
closed form.  The dot is pinned as an exact integer sum (weights and
activations chosen so every scale is 1.0), and against float64 sums of the
independently decoded operands.  What no check here can pin is the
activation type and the float order of ggml's own Q2_0 dot, whose CPU source
is not in the reference: the oracle pairs Q2_0 with q8_0 activations and adds
one term per 32 elements in element order (parity unpinned for that choice).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import dequant_act, f16, random_blocks

Q2_0 = 42


def block(d: float, codes) -> bytes:
    """A Q2_0 block from 64 codes (0..3), packed as the format defines."""
    codes = list(codes)
    assert len(codes) == 64
    qs = bytes(sum(codes[4 * b + i] << (2 * i) for i in range(4)) for b in range(16))
    return f16(d) + qs


def test_geometry(orc):
    assert orc.BLOCK[Q2_0] == (64, 18)
    assert orc.row_bytes(Q2_0, 128) == 36 and orc.row_bytes(Q2_0, 96) == 0
    assert orc.act_row_bytes(Q2_0, 128) == 4 * 34            # q8_0 activations


def test_dequant_known_answer_code_order_and_offset(orc):
    # byte 0xE4 = codes 0, 1, 2, 3 from the low bits up; 0x1B the reverse
    qs = bytes([0xE4] * 8 + [0x1B] * 8)
    y = orc.dequantize(Q2_0, np.frombuffer(f16(1.0) + qs, np.uint8), 64)
    assert y[:32].tolist() == [-1.0, 0.0, 1.0, 2.0] * 8
    assert y[32:].tolist() == [2.0, 1.0, 0.0, -1.0] * 8


def test_dequant_scales_blocks_independently(orc):
    raw = block(0.5, [0] * 64) + block(-2.0, [3] * 64) + block(0.0, [2] * 64) + block(2 ** -14, [2, 3] * 32)
    y = orc.dequantize(Q2_0, np.frombuffer(raw, np.uint8), 256)
    assert (y[:64] == -0.5).all()
    assert (y[64:128] == -4.0).all()
    assert (y[128:192] == 0.0).all()
    assert y[192:].tolist() == [2 ** -14, 2 ** -13] * 32


def test_dot_is_the_exact_integer_sum(orc):
    """d_w = 1 and activations that quantise exactly (each 32-block holds
    +-127, so its q8_0 scale is 1.0): the dot is sum((code - 1) * x), an
    integer computed here from the codes by numpy's own bit unpacking."""
    rng = np.random.default_rng(42)
    k = 512
    codes = rng.integers(0, 4, k)
    raw = np.frombuffer(b"".join(block(1.0, codes[64 * b:64 * b + 64]) for b in range(k // 64)), np.uint8)
    x = rng.integers(-127, 128, k).astype(np.float32)
    x[::32] = 127.0
    a = orc.quantize_act(Q2_0, x[None])[0]
    assert np.array_equal(dequant_act(orc, Q2_0, a, k), x)    # exact q8_0 round trip
    qs = raw.reshape(-1, 18)[:, 2:]
    unpacked = np.unpackbits(qs, axis=1, bitorder="little").reshape(-1, 64, 2)
    got_codes = (unpacked[:, :, 0] + 2 * unpacked[:, :, 1]).reshape(-1)
    assert np.array_equal(got_codes, codes)
    want = int(((codes - 1) * x.astype(np.int64)).sum())
    assert orc.vec_dot(Q2_0, raw, a, k) == float(want)


def test_dot_halves_pair_with_their_own_activation_scales(orc):
    """Two 32-element halves of one block, activations of different scales:
    the dot is d_w * (d_a0 * S0 + d_a1 * S1) exactly (small powers of two)."""
    codes = [3] * 32 + [0] * 32                              # +2 on the first half, -1 on the second
    raw = np.frombuffer(block(0.25, codes), np.uint8)
    x = np.concatenate([np.full(32, 127 * 0.5), np.full(32, 127 * 4.0)]).astype(np.float32)
    a = orc.quantize_act(Q2_0, x[None])[0]
    assert orc.vec_dot(Q2_0, raw, a, 64) == 0.25 * (0.5 * 32 * 2 * 127 + 4.0 * 32 * -1 * 127)


@pytest.mark.parametrize("k", [64, 192, 1024])
def test_dot_matches_float64_of_decoded_operands(orc, k):
    rng = np.random.default_rng(k)
    raw = random_blocks(rng, Q2_0, 8, k)
    w = orc.dequantize(Q2_0, raw, k).astype(np.float64)
    for r in range(8):
        x = rng.standard_normal(k).astype(np.float32)
        a = orc.quantize_act(Q2_0, x[None])[0]
        av = dequant_act(orc, Q2_0, a, k)
        ref = float(w[r] @ av)
        got = orc.vec_dot(Q2_0, raw[r], a, k)
        assert abs(got - ref) <= 1e-6 * float(np.abs(w[r]).max() * np.abs(av).sum()), (r, got, ref)


def test_encoder_round_trip(orc):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    raw = orc.quantize_weights(Q2_0, w)
    y = orc.dequantize(Q2_0, raw, 256).reshape(4, 4, 64)
    wb = w.reshape(4, 4, 64)
    amax = np.abs(wb).max(axis=2, keepdims=True)
    # levels -d, 0, d, 2d with d = amax / 2: error at most d / 2 above -d, clipped below it
    d = amax / 2
    err = np.abs(y - wb)
    inside = wb >= -d
    assert (err[inside] <= (d / 2 * 1.01 + 1e-9).repeat(64, axis=2)[inside]).all()
