"""
Sabah / runtime / rt

ctypes binding to libsabah_rt.so, the MI355X build of the runtime.  Same
shape as the reference binding (sabah/runtime/rt.py:20-142): quant codes and
block geometry, a `lib()` loader with argument types, `check()` turning a -1
into an exception that carries the runtime's message, `row_bytes()`.

Device memory and streams come from PyTorch-ROCm; this module only moves
pointers and sizes.  There is no CPU fallback: if the library is missing,
every entry point raises RuntimeUnavailable.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(os.path.dirname(HERE))          # sabah-moe-accelerator_amd/
CSRC = os.path.join(PKG_ROOT, "csrc")

# ggml type codes, so a runtime trace and a llama.cpp trace mean the same thing
QTYPE = {"Q5_1": 7, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ3_XXS": 18, "IQ4_NL": 20, "IQ3_S": 21,
         "IQ2_S": 22, "IQ4_XS": 23, "Q2_0": 42}
QTYPE_NAME = {v: k for k, v in QTYPE.items()}

# (elements per block, bytes per block)
QBLOCK = {7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 18: (256, 98), 20: (32, 18),
          21: (256, 110), 22: (256, 82), 23: (256, 136), 42: (64, 18)}


class RuntimeUnavailable(Exception):
    """The HIP runtime library is missing or could not be loaded."""


class SabahRuntimeError(Exception):
    """A runtime entry point returned -1; the message is the runtime's."""


# the reference's name for the same exception (rt.py:37-38)
SabahCudaError = SabahRuntimeError


def library_path() -> str:
    return os.environ.get("SABAH_RT_LIB") or os.path.join(CSRC, "libsabah_rt.so")


c_vp, c_sz, c_i, c_u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_ulonglong


class MoeLayerDesc(ctypes.Structure):
    """sabah_moe_layer_desc (include/sabah_rt.h)."""
    _fields_ = [("gate", c_vp), ("up", c_vp), ("down", c_vp),
                ("qt_gate", c_i), ("qt_up", c_i), ("qt_down", c_i),
                ("d_model", c_i), ("d_ff", c_i), ("n_experts", c_i),
                ("shared_gate", c_vp), ("shared_up", c_vp), ("shared_down", c_vp),
                ("qt_shared_gate", c_i), ("qt_shared_up", c_i), ("qt_shared_down", c_i),
                ("d_ff_shared", c_i), ("shared_gate_inp", c_vp)]


# every symbol include/sabah_rt.h declares, with its ctypes signature
SIGNATURES = {
    "sabah_rt_init": ([c_i], c_i),
    "sabah_rt_shutdown": ([], c_i),
    "sabah_rt_last_error": ([], ctypes.c_char_p),
    "sabah_rt_build_info": ([], ctypes.c_char_p),
    "sabah_rt_device_count": ([], c_i),
    "sabah_rt_mul_mat_id_v2": ([c_vp, c_sz, c_sz, c_vp, c_sz, c_i, c_sz, c_vp, c_sz, c_sz, c_i, c_i,
                                c_vp, c_sz, c_sz, c_i, c_i, c_i, c_i, c_vp, c_vp], c_i),
    "sabah_rt_register_bank": ([c_vp, c_vp, c_sz, c_sz, c_i], c_i),
    "sabah_rt_unregister_bank": ([c_vp], c_i),
    "sabah_rt_check_errors": ([], c_i),
    "sabah_rt_get_metrics": ([ctypes.POINTER(c_u64)] * 5, c_i),
    "sabah_rt_get_diag": ([ctypes.POINTER(c_u64)] * 5, c_i),
    "sabah_rt_snapshot": ([ctypes.c_char_p, c_sz], c_i),
    "sabah_row_bytes": ([c_i, c_i], c_sz),
    "sabah_dequant": ([c_vp, c_vp, c_i, c_i, c_i], c_i),
    "sabah_quantize_act": ([c_vp, c_vp, c_i, c_i, c_i, c_vp], c_i),
    "sabah_moe_block": ([c_vp, c_vp, c_vp, c_vp, c_vp, c_i, c_i, c_i, c_i, c_i, c_i, c_i], c_i),
    "sabah_moe_layer": ([ctypes.POINTER(MoeLayerDesc), c_vp, c_vp, c_vp, c_i, c_i, c_vp, c_vp, c_vp], c_i),
    "sabah_moe_layer_noalloc": ([ctypes.POINTER(MoeLayerDesc), c_vp, c_vp, c_vp, c_i, c_i, c_vp, c_vp, c_vp], c_i),
    "sabah_moe_chain": ([ctypes.POINTER(MoeLayerDesc), c_i, c_vp, c_vp, c_vp, c_i, c_i, c_vp], c_i),
    "sabah_moe_prefill_layer": ([ctypes.POINTER(MoeLayerDesc), c_vp, c_vp, c_vp, c_i, c_i, c_vp, c_vp, c_vp], c_i),
    "sabah_moe_route": ([c_vp, c_i, c_i, c_i, c_i, ctypes.c_float, c_vp, c_vp, c_vp], c_i),
    "sabah_rt_set_mmid_grouping": ([c_i], c_i),
    # memory, copies, events and streams for the harness (the reference binds them, rt.py:70-107)
    "sabah_dev_alloc": ([c_sz], c_vp),
    "sabah_dev_free": ([c_vp], None),
    "sabah_host_alloc": ([c_sz], c_vp),
    "sabah_host_free": ([c_vp], None),
    "sabah_dev_mem": ([ctypes.POINTER(c_sz), ctypes.POINTER(c_sz)], c_i),
    "sabah_memcpy_h2d": ([c_vp, c_vp, c_sz], c_i),
    "sabah_memcpy_d2h": ([c_vp, c_vp, c_sz], c_i),
    "sabah_memset_d": ([c_vp, c_i, c_sz], c_i),
    "sabah_h2d_async": ([c_vp, c_vp, c_sz], c_i),
    "sabah_event_create": ([], c_vp),
    "sabah_event_destroy": ([c_vp], None),
    "sabah_event_record_copy": ([c_vp], c_i),
    "sabah_event_record_compute": ([c_vp], c_i),
    "sabah_compute_wait_event": ([c_vp], c_i),
    "sabah_copy_wait_event": ([c_vp], c_i),
    "sabah_event_elapsed_ms": ([c_vp, c_vp], ctypes.c_float),
    "sabah_event_sync": ([c_vp], c_i),
    "sabah_event_query": ([c_vp], c_i),
    "sabah_sync_copy": ([], c_i),
    "sabah_sync_compute": ([], c_i),
    "sabah_sync_all": ([], c_i),
    "sabah_slab_init": ([c_sz], c_i),
    "sabah_slab_alloc": ([c_sz], c_vp),
    "sabah_slab_free": ([c_vp], None),
    "sabah_slab_destroy": ([], None),
    "sabah_rt_host_dequant": ([c_vp, c_vp, c_i, c_i], c_i),
}

# harness-only exports (not part of the drop-in header)
EXTRA_SIGNATURES = {
    "sabah_synth_weights": ([c_vp, c_i, ctypes.c_longlong, c_i, ctypes.c_ulonglong, ctypes.c_float, c_vp], c_i),
    "sabah_rt_set_kernel_timing": ([c_i], c_i),
    "sabah_rt_set_layer_fusion": ([c_i], c_i),
    "sabah_rt_set_mmid_rounds": ([c_i], c_i),
    "sabah_rt_set_layer_placement_test": ([c_i], c_i),
    "sabah_rt_set_selfcheck": ([c_i, ctypes.c_double, c_i], c_i),
    "sabah_rt_get_kernel_timing": ([c_i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_u64), c_i], c_i),
}

KERNEL_KINDS = {"mmid": 0, "gate_up": 1, "down": 2, "chain": 3, "grouped_gate_up": 4, "grouped_down": 5, "layer": 6}


def kernel_timing(kind: str, reset: bool = False) -> tuple[float, int]:
    """(total ms, launches) of one kernel kind since timing was switched on."""
    ms, n = ctypes.c_double(), c_u64()
    check(lib().sabah_rt_get_kernel_timing(KERNEL_KINDS[kind], ctypes.byref(ms), ctypes.byref(n), int(reset)),
          "kernel timing")
    return ms.value, n.value


class _Handle:
    """The library, opened on first use and bound to SIGNATURES then.

    There is exactly one handle per process: every module goes through
    `lib()`, so argument types are set once and a missing build surfaces as
    RuntimeUnavailable at the first call that needs the GPU path (never as a
    silent fallback)."""

    cdll = None

    @classmethod
    def open(cls):
        if cls.cdll is None:
            path = library_path()
            if not os.path.isfile(path):
                raise RuntimeUnavailable(
                    "%s does not exist; build the HIP library first "
                    "(__graft_entry__.build(), or make -C %s)" % (path, CSRC))
            try:
                handle = ctypes.CDLL(path)
            except OSError as exc:
                raise RuntimeUnavailable("%s did not load: %s" % (path, exc)) from exc
            for name, (argtypes, restype) in {**SIGNATURES, **EXTRA_SIGNATURES}.items():
                entry = getattr(handle, name)
                entry.argtypes, entry.restype = argtypes, restype
            cls.cdll = handle
        return cls.cdll


def lib():
    """The bound libsabah_rt.so (raises RuntimeUnavailable when it cannot be opened)."""
    return _Handle.open()


def last_error() -> str:
    """The library's message for its most recent failure ("" when there is none
    or the library is not loaded)."""
    if _Handle.cdll is None:
        return ""
    raw = _Handle.cdll.sabah_rt_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def check(rc, what="runtime call"):
    """Pass a 0 return code through; turn anything else (-1, or None from a
    missing return) into SabahRuntimeError carrying the library's message."""
    if rc == 0:
        return rc
    raise SabahRuntimeError("%s returned %r: %s" % (what, rc, last_error() or "no message from the library"))


def row_bytes(qt: int, n: int) -> int:
    """GGUF bytes of one row of n elements of type qt; n must fill whole blocks."""
    elems, nbytes = QBLOCK[qt]
    blocks, rest = divmod(n, elems)
    if rest:
        raise ValueError("%d elements leave %d over a whole number of %d-element %s blocks"
                         % (n, rest, elems, QTYPE_NAME.get(qt, str(qt))))
    return blocks * nbytes


def available() -> bool:
    """True when the HIP library can be opened (a GPU is not required)."""
    try:
        _Handle.open()
    except RuntimeUnavailable:
        return False
    return True


def device_count() -> int:
    """GPUs the library sees (0 without the library or without a GPU)."""
    return int(_Handle.open().sabah_rt_device_count()) if available() else 0


_initialised = None


def init(device: int = 0) -> None:
    """sabah_rt_init once per process (idempotent for the same device)."""
    global _initialised
    if _initialised == device:
        return
    check(lib().sabah_rt_init(device), "sabah_rt_init")
    _initialised = device


def metrics() -> dict:
    v = [c_u64() for _ in range(5)]
    check(lib().sabah_rt_get_metrics(*[ctypes.byref(z) for z in v]), "get_metrics")
    return dict(zip(("hits", "misses", "evictions", "bytes_fetched", "resident_bytes"), (z.value for z in v)))


def diag() -> dict:
    v = [c_u64() for _ in range(5)]
    check(lib().sabah_rt_get_diag(*[ctypes.byref(z) for z in v]), "get_diag")
    return dict(zip(("calls", "tokens", "overflow", "verify_ok", "verify_fail"), (z.value for z in v)))


def snapshot() -> dict:
    import json
    buf = ctypes.create_string_buffer(2048)
    check(lib().sabah_rt_snapshot(buf, 2048), "snapshot")
    return json.loads(buf.value.decode())


def build_info() -> str:
    return lib().sabah_rt_build_info().decode()
