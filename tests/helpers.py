"""Shared test helpers: parity metrics, hand-built quant blocks, decoded activations."""
from __future__ import annotations

import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"

MAX_REL_TOL = 1e-3      # max|y - r| / max|r|
COS_TOL = 0.99999


def max_rel(y, r) -> float:
    y, r = np.asarray(y, np.float64), np.asarray(r, np.float64)
    return float(np.abs(y - r).max() / max(np.abs(r).max(), 1e-30))


def rel_l2(y, r) -> float:
    y, r = np.asarray(y, np.float64), np.asarray(r, np.float64)
    return float(np.linalg.norm(y - r) / max(np.linalg.norm(r), 1e-30))


def cosine(y, r) -> float:
    y, r = np.asarray(y, np.float64).ravel(), np.asarray(r, np.float64).ravel()
    return float(y @ r / max(np.sqrt((y @ y) * (r @ r)), 1e-300))


def assert_parity(y, r, what=""):
    mr, c = max_rel(y, r), cosine(y, r)
    assert mr <= MAX_REL_TOL and c >= COS_TOL, "%s: max_rel=%.3e (tol %.0e) cos=%.8f (tol %.5f) rel_l2=%.3e" % (
        what, mr, MAX_REL_TOL, c, COS_TOL, rel_l2(y, r))
    return mr, c


def assert_bits_equal(got, want, what=""):
    """Bitwise equality of two float arrays; on failure the message gives the
    number of differing 32-bit words, the first positions, and how many of
    them are 0xFFFFFFFF (an output fill that was not overwritten, or that
    landed after the kernel's store)."""
    g = np.ascontiguousarray(got).view(np.uint32)
    w = np.ascontiguousarray(want).view(np.uint32)
    assert g.shape == w.shape, "%s: shapes %s vs %s" % (what, g.shape, w.shape)
    bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
    if bad.size:
        gf, wf = g.reshape(-1), w.reshape(-1)
        first = [(tuple(int(i) for i in np.unravel_index(j, g.shape)), "%08x" % gf[j], "%08x" % wf[j])
                 for j in bad[:8]]
        raise AssertionError("%s: %d of %d words differ (%d of them 0xffffffff in got, %d in want); first %s" % (
            what, bad.size, g.size, int((gf[bad] == 0xFFFFFFFF).sum()), int((wf[bad] == 0xFFFFFFFF).sum()), first))


def f16(x: float) -> bytes:
    return np.array([x], np.float16).tobytes()


def dequant_act(O, qt: int, act: np.ndarray, k: int) -> np.ndarray:
    """float64 values of a quantised activation row (as its vec_dot partner sees them)."""
    act = np.ascontiguousarray(act, np.uint8).reshape(-1)
    if qt in (O.Q8_0, O.IQ4_NL, O.Q2_0):             # q8_0 activations
        blk = act.reshape(-1, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)
        return (blk[:, 2:].view(np.int8).astype(np.float64) * d).reshape(-1)[:k]
    if qt == O.Q5_1:                                  # q8_1 activations: d, s, 32 values
        blk = act.reshape(-1, 36)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)
        return (blk[:, 4:].view(np.int8).astype(np.float64) * d).reshape(-1)[:k]
    blk = act.reshape(-1, 292)
    d = blk[:, :4].copy().view(np.float32).astype(np.float64)
    return (blk[:, 4:260].view(np.int8).astype(np.float64) * d).reshape(-1)[:k]


def reference_iq3s_grid() -> list[int] | None:
    """The 512-entry IQ3_S grid as the reference's table header spells it (text parse)."""
    p = os.path.join(REF, "sabah/runtime/cuda/sabah_iq_tables.h")
    if not os.path.exists(p):
        return None
    t = open(p).read()
    i = t.index("static const uint32_t iq3s_grid[512]")
    body = t[i:t.index("};", i)]
    return [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{8})", body)]


def oracle_iq3s_grid() -> list[int]:
    t = open(os.path.join(ROOT, "oracle", "iq3s_grid_u32.h")).read()
    return [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{8})", t)]


def product_iq3s_grid() -> list[int]:
    """Expand the product's packed level table (csrc/iq3s_grid.h) to the byte form."""
    t = open(os.path.join(ROOT, "sabah-moe-accelerator_amd", "csrc", "iq3s_grid.h")).read()
    body = t[t.index("kIq3sGridLevels"):]
    lv = [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{3})", body)]
    return [sum((2 * ((v >> (3 * j)) & 7) + 1) << (8 * j) for j in range(4)) for v in lv]


def random_blocks(rng, qt: int, n_rows: int, k: int) -> np.ndarray:
    """Random bytes that form valid blocks: every field random, fp16 scales finite and modest."""
    from oracle import BLOCK
    qb, bb = BLOCK[qt]
    nb = k // qb
    raw = rng.integers(0, 256, size=(n_rows, nb, bb), dtype=np.uint8)

    def scales(n):
        return (rng.uniform(0.25, 2.0, size=n) * rng.choice([-1, 1], size=n) * 1e-2).astype(np.float16)

    if qt in (8, 18, 20, 21, 22, 23, 42):   # Q8_0, IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, Q2_0: fp16 d at 0
        raw[:, :, 0:2] = scales(n_rows * nb).view(np.uint8).reshape(n_rows, nb, 2)
    elif qt == 7:                           # Q5_1: d, m at 0, 2
        raw[:, :, 0:2] = np.abs(scales(n_rows * nb)).view(np.uint8).reshape(n_rows, nb, 2)
        raw[:, :, 2:4] = scales(n_rows * nb).view(np.uint8).reshape(n_rows, nb, 2)
    elif qt in (12, 13):                    # Q4_K, Q5_K: d, dmin at 0, 2 (non-negative in real data)
        raw[:, :, 0:2] = np.abs(scales(n_rows * nb)).view(np.uint8).reshape(n_rows, nb, 2)
        raw[:, :, 2:4] = np.abs(scales(n_rows * nb)).view(np.uint8).reshape(n_rows, nb, 2)
    elif qt == 14:                          # Q6_K: d at 208
        raw[:, :, 208:210] = scales(n_rows * nb).view(np.uint8).reshape(n_rows, nb, 2)
    return raw.reshape(n_rows, nb * bb)


def q8_1_tie_row(k: int, seed: int = 0) -> np.ndarray:
    """A row of k fp32 values (k a multiple of 32) whose every 32-block has a
    q8_1 scaled sum at an fp16 tie: fl32(sum(q) * d) lies exactly halfway
    between two halves while the exact product does not, so rounding the
    product once to fp16 (a fused mixed-precision multiply) gives the other
    half than rounding it to fp32 first, as ggml does.  Built per block: a
    tie value v and a sum S, a scale d with fl32(S * d) = v != S * d, the
    block's largest magnitude 127 d, and the other values multiples of d
    whose quantised sum makes S."""
    rng = np.random.default_rng(seed)
    f32 = np.float32
    out = []
    while len(out) < k // 32:
        S = int(rng.integers(-600, 600))
        if abs(S) < 150:
            continue
        # an fp16 tie: a half h and its successor, midpoint v (exact in fp32)
        h = np.float16(rng.uniform(0.05, 20.0) * (1 if S > 0 else -1))
        v = f32((float(h) + float(np.nextafter(h, np.float16(np.inf if S > 0 else -np.inf)))) / 2)
        d0 = f32(float(v) / S)
        for dd in (d0, np.nextafter(d0, f32(1)), np.nextafter(d0, f32(-1))):
            amax = f32(float(dd) * 127)
            if not (f32(amax / f32(127)) == dd and f32(f32(S) * dd) == v and float(S) * float(dd) != float(v)):
                continue
            q = np.zeros(32, np.int64)
            q[0] = 127
            rest = S - 127
            for j in range(1, 32):             # spread the rest over the other 31, each within [-126, 126]
                share = int(np.clip(round(rest / (32 - j)), -126, 126))
                q[j] = share
                rest -= share
            if rest != 0:
                break
            blk = (q.astype(np.float64) * float(dd)).astype(np.float32)
            idv = f32(1) / dd
            back = np.array([np.sign(x) * np.floor(abs(float(x * idv)) + 0.5) for x in blk])
            if np.array_equal(back, q) and f32(np.abs(blk).max()) == amax:
                out.append(blk)
            break
    return np.concatenate(out)


def unfused_rounding_row(k: int, amax: float = 3.0) -> np.ndarray:
    """A row of k fp32 values (k a multiple of 256) whose q8_K bytes depend on
    rounding the product iscale*x before ggml's round-to-int add: each 256-block
    opens with +amax (so iscale = fl(-127/amax)), then holds values x for which
    rint(fl(iscale*x)) != rint(iscale*x) (exact).  A fused multiply-add gets
    every one of them wrong by one."""
    iscale = np.float32(-127.0) / np.float32(amax)
    hits = []
    for h in np.arange(-126.5, 127.0, 1.0):
        c0 = np.float32(h / float(iscale))
        for c in (np.nextafter(c0, np.float32(-9), dtype=np.float32), c0, np.nextafter(c0, np.float32(9), dtype=np.float32)):
            if not abs(c) < amax:
                continue
            exact = float(iscale) * float(c)          # 24 x 24 bits: exact in float64
            if np.rint(np.float32(iscale * c)) != np.rint(exact):
                hits.append(c)
    assert len(hits) >= 32, len(hits)
    per = 255
    row = np.empty(k, np.float32)
    for b in range(k // 256):
        row[256 * b] = amax
        row[256 * b + 1:256 * (b + 1)] = [hits[(b * per + i) % len(hits)] for i in range(per)]
    return row


def reference_table(name: str, n: int, width: int) -> list[int] | None:
    """A table of the reference's sabah_iq_tables.h (text parse), or None if it is not mounted."""
    p = os.path.join(REF, "sabah/runtime/cuda/sabah_iq_tables.h")
    if not os.path.exists(p):
        return None
    t = open(p).read()
    i = t.index(name + "[%d]" % n)
    body = t[t.index("{", i):t.index("};", i)]
    if width == 0:
        return [int(x) for x in re.findall(r"-?\d+", body)]
    return [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{%d})" % width, body)]


def oracle_table(name: str) -> list[int]:
    """A table of oracle/iq_tables_u32.h."""
    t = open(os.path.join(ROOT, "oracle", "iq_tables_u32.h")).read()
    i = t.index(name + "[")
    body = t[t.index("{", i):t.index("};", i)]
    return [int(x, 0) for x in re.findall(r"-?0x[0-9a-fA-F]+|-?\d+", body)]

