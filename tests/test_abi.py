"""The C-ABI library without a GPU: it loads, exports every symbol the public
header declares, and rejects invalid MUL_MAT_ID arguments before touching the
device (the host-side checks of sabah_rt.cu:3516-3547)."""
import ctypes
import os
import re

import pytest

from helpers import ROOT

HEADER = os.path.join(ROOT, "include", "sabah_rt.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sabah_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from sabah.runtime import rt
    L = rt.lib()
    names = declared_functions()
    assert len(names) >= 17
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    from sabah.runtime import rt
    assert set(declared_functions()) == set(rt.SIGNATURES)


def test_grouping_mode_setter_validates_without_a_device():
    from sabah.runtime import rt
    L = rt.lib()
    assert L.sabah_rt_set_mmid_grouping(3) == -1
    assert "grouping mode" in rt.last_error()
    for mode in (1, 2, 0):
        assert L.sabah_rt_set_mmid_grouping(mode) == 0


def test_build_info_and_row_bytes():
    from sabah.runtime import rt
    L = rt.lib()
    assert rt.build_info().startswith("sabah_rt abi=v2 sentinel=0")
    assert L.sabah_row_bytes(21, 2048) == 880 and L.sabah_row_bytes(21, 768) == 330
    assert L.sabah_row_bytes(12, 768) == 432 and L.sabah_row_bytes(14, 768) == 630
    assert L.sabah_row_bytes(8, 1024) == 1088
    assert L.sabah_row_bytes(2, 1024) == 0           # unsupported type
    assert L.sabah_row_bytes(21, 100) == 0           # not a whole number of blocks


def _v2(L, **kw):
    a = dict(source=1, expert_stride=880 * 768, row_stride=880, d_x=1, x_id_stride=8192, x_rows=1,
             x_token_stride=8192, d_ids=1, ids_id_stride=4, ids_token_stride=40, n_ids=10, n_tokens=1,
             d_dst=1, dst_id_stride=3072, dst_token_stride=30720, rows=768, k=2048, n_experts=512, qt=21)
    a.update(kw)
    vp = ctypes.c_void_p
    return L.sabah_rt_mul_mat_id_v2(vp(a["source"]), a["expert_stride"], a["row_stride"], vp(a["d_x"]),
                                    a["x_id_stride"], a["x_rows"], a["x_token_stride"], vp(a["d_ids"]),
                                    a["ids_id_stride"], a["ids_token_stride"], a["n_ids"], a["n_tokens"],
                                    vp(a["d_dst"]), a["dst_id_stride"], a["dst_token_stride"], a["rows"], a["k"],
                                    a["n_experts"], a["qt"], None, None)


@pytest.mark.parametrize("bad,msg", [
    (dict(k=2047), "geometry"),
    (dict(k=2016), "whole number"),
    (dict(x_rows=3), "input rows"),
    (dict(qt=2), "unsupported quant type"),
    (dict(row_stride=879), "row stride"),
    (dict(source=0), "null pointer"),
    (dict(n_experts=0), "geometry"),
])
def test_v2_rejects_invalid_arguments_without_a_device(bad, msg):
    from sabah.runtime import rt
    L = rt.lib()
    assert _v2(L, **bad) == -1
    assert msg in rt.last_error()


def test_v2_zero_tokens_is_a_counted_noop():
    from sabah.runtime import rt
    L = rt.lib()
    before = rt.snapshot()["empty_calls"]
    assert _v2(L, n_tokens=0) == 0
    assert rt.snapshot()["empty_calls"] == before + 1


def test_v2_requires_init():
    from sabah.runtime import rt
    if rt._initialised is not None:
        pytest.skip("runtime already initialised in this process")
    assert _v2(rt.lib()) == -1
    assert "sabah_rt_init" in rt.last_error()


def test_metrics_before_any_call():
    from sabah.runtime import rt
    m = rt.metrics()
    assert m["misses"] == 0 and m["evictions"] == 0 and m["bytes_fetched"] == 0


def _desc(qt_gate=21, qt_up=21, qt_down=21, d_model=2048, d_ff=768, n_experts=512):
    from sabah.runtime import rt
    d = rt.MoeLayerDesc()
    d.gate, d.up, d.down = 1, 1, 1                     # never dereferenced: the checks come first
    d.qt_gate, d.qt_up, d.qt_down = qt_gate, qt_up, qt_down
    d.d_model, d.d_ff, d.n_experts = d_model, d_ff, n_experts
    return d


@pytest.mark.parametrize("kw", [dict(qt_gate=12, qt_up=14, qt_down=14), dict(qt_gate=8, qt_up=8, qt_down=8),
                                dict(qt_down=8), dict(d_model=2560), dict(d_model=4096),
                                dict(d_ff=1280), dict(n_experts=8192)])
def test_prefill_layer_rejects_shapes_it_does_not_group_without_a_device(kw):
    """The grouped layer takes gate/up of one type and down, each IQ3_S, Q4_K or
    Q6_K, d_model a multiple of 512 up to 2048, d_ff a multiple of 256 up to 1024
    and n_experts <= 4096; anything else is refused before the device is touched."""
    from sabah.runtime import rt
    L = rt.lib()
    d = _desc(**kw)
    vp = ctypes.c_void_p
    rc = L.sabah_moe_prefill_layer(ctypes.byref(d), vp(1), vp(1), vp(1), 10, 4, vp(1), None, None)
    assert rc == -1
    assert "grouped MoE layer" in rt.last_error() or "unsupported type mix" in rt.last_error()


@pytest.mark.parametrize("args,msg", [((0, 10), "n_experts"), ((5000, 10), "n_experts"), ((512, 0), "n_used"),
                                      ((8, 9), "n_used"), ((512, 65), "n_used")])
def test_route_rejects_invalid_shapes_without_a_device(args, msg):
    """sabah_moe_route takes 1 <= n_experts <= 4096 and 1 <= n_used <= min(n_experts, 64);
    anything else is refused before the device is touched."""
    from sabah.runtime import rt
    L = rt.lib()
    vp = ctypes.c_void_p
    E, k = args
    assert L.sabah_moe_route(vp(1), 3, E, k, 1, 1.0, vp(1), vp(1), None) == -1
    assert msg in rt.last_error()
    assert L.sabah_moe_route(vp(1), 3, 512, 10, 1, 0.0, vp(1), vp(1), None) == -1
    assert "w_scale" in rt.last_error()


# The names the reference harness's rt.lib() binds with getattr (its
# sabah/runtime/rt.py:70-107 signature table) and the five the llama.cpp bridge
# resolves with dlsym (patch 0001:158-165, plus the bank registration this
# library adds): loading either caller fails on the first name missing.
REFERENCE_HARNESS_NAMES = [
    "sabah_rt_last_error", "sabah_rt_init", "sabah_rt_shutdown", "sabah_rt_device_count",
    "sabah_dev_alloc", "sabah_dev_free", "sabah_host_alloc", "sabah_host_free", "sabah_dev_mem",
    "sabah_memcpy_h2d", "sabah_memcpy_d2h", "sabah_memset_d", "sabah_h2d_async",
    "sabah_event_create", "sabah_event_destroy", "sabah_event_record_copy", "sabah_event_record_compute",
    "sabah_compute_wait_event", "sabah_copy_wait_event", "sabah_event_elapsed_ms", "sabah_event_sync",
    "sabah_event_query", "sabah_sync_copy", "sabah_sync_compute", "sabah_sync_all", "sabah_moe_block",
    "sabah_dequant", "sabah_row_bytes", "sabah_slab_init", "sabah_slab_alloc", "sabah_slab_free",
    "sabah_slab_destroy",
]
BRIDGE_NAMES = ["sabah_rt_init", "sabah_rt_mul_mat_id_v2", "sabah_rt_last_error", "sabah_rt_get_metrics",
                "sabah_rt_register_bank"]


def test_library_exports_every_name_the_reference_harness_and_bridge_bind():
    from sabah.runtime import rt
    L = rt.lib()
    missing = [n for n in REFERENCE_HARNESS_NAMES + BRIDGE_NAMES if not hasattr(L, n)]
    assert not missing, missing
    assert set(REFERENCE_HARNESS_NAMES) <= set(rt.SIGNATURES)


def test_slab_and_events_fail_cleanly_without_init():
    """Calls that need the library's streams fail with a message before
    sabah_rt_init instead of touching a null stream."""
    from sabah.runtime import rt
    L = rt.lib()
    if rt._initialised is not None:
        pytest.skip("the library is already initialised in this process")
    assert L.sabah_sync_copy() == -1 and "sabah_rt_init" in rt.last_error()
    assert L.sabah_h2d_async(None, None, 0) == -1
    assert L.sabah_slab_alloc(256) is None                  # no slab yet
