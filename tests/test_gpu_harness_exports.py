"""The memory, copy, event and slab exports the reference harness binds
(sabah/runtime/rt.py:70-107; semantics sabah_rt.cu:3240-3353, 3889-3903), and
sabah_rt_host_dequant (sabah_rt.cu:3845-3847), through the C ABI."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from helpers import random_blocks

pytestmark = pytest.mark.gpu


def test_device_memory_copies_and_memset(hip_rt):
    L = hip_rt.lib()
    n = 1 << 16
    src = np.arange(n, dtype=np.uint8)
    d = L.sabah_dev_alloc(n)
    assert d
    try:
        hip_rt.check(L.sabah_memcpy_h2d(d, src.ctypes.data, n), "h2d")
        back = np.empty_like(src)
        hip_rt.check(L.sabah_memcpy_d2h(back.ctypes.data, d, n), "d2h")
        assert np.array_equal(back, src)
        hip_rt.check(L.sabah_memset_d(d, 0x5A, n // 2), "memset")
        hip_rt.check(L.sabah_memcpy_d2h(back.ctypes.data, d, n), "d2h")
        assert (back[:n // 2] == 0x5A).all() and np.array_equal(back[n // 2:], src[n // 2:])
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        hip_rt.check(L.sabah_dev_mem(ctypes.byref(free), ctypes.byref(total)), "dev_mem")
        assert 0 < free.value <= total.value
    finally:
        L.sabah_dev_free(d)


def test_async_copy_events_and_stream_order(hip_rt):
    """A pinned buffer copied on the copy stream, the compute stream made to
    wait for it through an event, a host dequant on the compute stream's data:
    the events report completion and a non-negative elapsed time."""
    L = hip_rt.lib()
    n = 1 << 20
    h = L.sabah_host_alloc(n)
    d = L.sabah_dev_alloc(n)
    e0, e1 = L.sabah_event_create(), L.sabah_event_create()
    assert h and d and e0 and e1
    try:
        hv = (ctypes.c_uint8 * n).from_address(h)
        np.frombuffer(hv, np.uint8)[:] = np.arange(n, dtype=np.uint64).astype(np.uint8)
        hip_rt.check(L.sabah_event_record_copy(e0), "record copy")
        hip_rt.check(L.sabah_h2d_async(d, h, n), "h2d async")
        hip_rt.check(L.sabah_event_record_copy(e1), "record copy")
        hip_rt.check(L.sabah_compute_wait_event(e1), "compute wait")
        hip_rt.check(L.sabah_sync_copy(), "sync copy")
        assert L.sabah_event_query(e1) == 1
        ms = L.sabah_event_elapsed_ms(e0, e1)
        assert ms >= 0.0
        hip_rt.check(L.sabah_event_sync(e1), "event sync")
        hip_rt.check(L.sabah_event_record_compute(e0), "record compute")
        hip_rt.check(L.sabah_copy_wait_event(e0), "copy wait")
        hip_rt.check(L.sabah_sync_compute(), "sync compute")
        back = np.empty(n, np.uint8)
        hip_rt.check(L.sabah_memcpy_d2h(back.ctypes.data, d, n), "d2h")
        assert np.array_equal(back, np.arange(n, dtype=np.uint64).astype(np.uint8))
    finally:
        L.sabah_event_destroy(e0)
        L.sabah_event_destroy(e1)
        L.sabah_dev_free(d)
        L.sabah_host_free(h)


def test_slab_hands_out_aligned_ranges_and_merges_freed_ones(hip_rt):
    L = hip_rt.lib()
    cap = 1 << 20
    hip_rt.check(L.sabah_slab_init(cap), "slab init")
    try:
        hip_rt.check(L.sabah_slab_init(cap // 2), "slab init again")     # no-op on an existing slab
        a = L.sabah_slab_alloc(1000)
        b = L.sabah_slab_alloc(300000)
        c = L.sabah_slab_alloc(300000)
        assert a and b and c and len({a, b, c}) == 3
        assert all(p % 256 == 0 for p in (a, b, c))
        assert b - a >= 1000 and c - b >= 300000
        assert L.sabah_slab_alloc(cap) is None                          # too large for what is left
        L.sabah_slab_free(b)
        L.sabah_slab_free(a)
        L.sabah_slab_free(c)
        whole = L.sabah_slab_alloc(cap)                                  # the merged free ranges are whole again
        assert whole == a
        L.sabah_slab_free(whole)
        L.sabah_slab_free(whole + 256)                                   # not handed out: ignored
        assert L.sabah_slab_alloc(cap) == a
    finally:
        L.sabah_slab_destroy()
    assert L.sabah_slab_alloc(256) is None


@pytest.mark.parametrize("qt,k", [(8, 96), (12, 512), (14, 256), (21, 768), (18, 256), (20, 160), (23, 512), (22, 256)])
def test_host_dequant_matches_the_oracle(hip_rt, orc, qt, k):
    rng = np.random.default_rng(qt * 1000 + k)
    raw = random_blocks(rng, qt, 1, k)[0]
    out = np.empty(k, np.float32)
    hip_rt.check(hip_rt.lib().sabah_rt_host_dequant(raw.ctypes.data, out.ctypes.data, qt, k), "host dequant")
    want = orc.dequantize(qt, raw[None], k)[0]
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_host_dequant_rejects_a_partial_block(hip_rt):
    L = hip_rt.lib()
    raw = np.zeros(110, np.uint8)
    out = np.empty(100, np.float32)
    assert L.sabah_rt_host_dequant(raw.ctypes.data, out.ctypes.data, 21, 100) == -1
    assert "host dequant" in hip_rt.last_error()
