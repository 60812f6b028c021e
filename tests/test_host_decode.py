"""The library's own host decoders (host_decode.h), through
sabah_rt_host_dequant, which runs on the CPU without a GPU or sabah_rt_init
(as the reference's host routine, sabah_rt.cu:3845-3849): every format,
random valid blocks, bit-identical to the oracle's dequantisation (the device
decoders are held to the same bits by the GPU tests)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from helpers import random_blocks

FORMATS = [(8, 1024), (7, 1024), (12, 2048), (13, 2048), (14, 768), (21, 2048), (18, 768), (22, 768), (20, 640),
           (23, 768), (42, 960)]


@pytest.mark.parametrize("qt,k", FORMATS)
def test_host_dequant_is_bit_identical_to_the_oracle(hip_rt_cpu, orc, qt, k):
    rng = np.random.default_rng(qt * 31 + k)
    raw = random_blocks(rng, qt, 5, k)
    want = orc.dequantize(qt, raw, k)
    L = hip_rt_cpu.lib()
    for r in range(5):
        src = np.ascontiguousarray(raw[r])
        dst = np.full(k, np.nan, np.float32)
        rc = L.sabah_rt_host_dequant(ctypes.c_void_p(src.ctypes.data), ctypes.c_void_p(dst.ctypes.data), qt, k)
        assert rc == 0, hip_rt_cpu.last_error()
        assert np.array_equal(dst.view(np.uint32), want[r].view(np.uint32)), (qt, r)


def test_host_dequant_rejects_unknown_types_and_partial_blocks(hip_rt_cpu):
    L = hip_rt_cpu.lib()
    src = np.zeros(1024, np.uint8)
    dst = np.zeros(256, np.float32)
    p, q = ctypes.c_void_p(src.ctypes.data), ctypes.c_void_p(dst.ctypes.data)
    assert L.sabah_rt_host_dequant(p, q, 2, 256) == -1                  # Q4_0: not decoded
    assert "unsupported" in hip_rt_cpu.last_error()
    assert L.sabah_rt_host_dequant(p, q, 12, 250) == -1                 # not whole Q4_K blocks
    assert L.sabah_rt_host_dequant(None, q, 8, 32) == -1
