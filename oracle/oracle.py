"""ORACLE - test infrastructure only.

ctypes wrapper around oracle/libsabah_oracle.so, the C restatement of ggml's
CPU MUL_MAT_ID path (ggml_cpu_ref.c).  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module; the product package never
does.  All arrays are numpy; nothing here touches a GPU.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsabah_oracle.so")

Q8_0, Q4_K, Q6_K, Q8_K, IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, Q2_0 = 8, 12, 14, 15, 18, 20, 21, 22, 23, 42
Q5_1, Q8_1, Q5_K = 7, 9, 13
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292), IQ3_S: (256, 110),
         Q5_1: (32, 24), Q8_1: (32, 36), Q5_K: (256, 176),
         IQ3_XXS: (256, 98), IQ4_NL: (32, 18), IQ4_XS: (256, 136),
         IQ2_S: (256, 82), Q2_0: (64, 18)}

_lib = None


def build() -> None:
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, ci, cf = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
    L.orc_fp16_to_fp32.argtypes, L.orc_fp16_to_fp32.restype = [ctypes.c_uint16], cf
    L.orc_fp32_to_fp16.argtypes, L.orc_fp32_to_fp16.restype = [cf], ctypes.c_uint16
    for n in ("orc_quantize_q8_0", "orc_quantize_q8_1", "orc_quantize_q8_K"):
        getattr(L, n).argtypes, getattr(L, n).restype = [vp, vp, ci], None
    L.orc_quantize_act.argtypes, L.orc_quantize_act.restype = [ci, vp, vp, ci], ci
    L.orc_quantize_weights.argtypes, L.orc_quantize_weights.restype = [ci, vp, vp, ci], ci
    L.orc_dequantize_row.argtypes, L.orc_dequantize_row.restype = [ci, vp, vp, ci], ci
    L.orc_vec_dot.argtypes, L.orc_vec_dot.restype = [ci, vp, vp, ci], cf
    L.orc_row_bytes.argtypes, L.orc_row_bytes.restype = [ci, ci], sz
    L.orc_act_row_bytes.argtypes, L.orc_act_row_bytes.restype = [ci, ci], sz
    L.orc_mul_mat_id.argtypes = [vp, sz, sz, vp, sz, ci, sz, vp, sz, sz, ci, ci,
                                 vp, sz, sz, ci, ci, ci, ci, ci]
    L.orc_mul_mat_id.restype = ci
    L.orc_moe_layer.argtypes = [ctypes.POINTER(MoeLayerDesc), vp, vp, vp, ci, ci, vp, vp, ci]
    L.orc_moe_layer.restype = ci
    L.orc_moe_route.argtypes = [vp, ci, ci, ci, ci, cf, vp, vp]
    L.orc_moe_route.restype = ci
    _lib = L
    return L


class MoeLayerDesc(ctypes.Structure):
    _fields_ = [("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("qt_gate", ctypes.c_int), ("qt_up", ctypes.c_int), ("qt_down", ctypes.c_int),
                ("d_model", ctypes.c_int), ("d_ff", ctypes.c_int), ("n_experts", ctypes.c_int),
                ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p),
                ("shared_down", ctypes.c_void_p),
                ("qt_shared_gate", ctypes.c_int), ("qt_shared_up", ctypes.c_int),
                ("qt_shared_down", ctypes.c_int), ("d_ff_shared", ctypes.c_int),
                ("shared_gate_inp", ctypes.c_void_p)]


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def row_bytes(qt: int, k: int) -> int:
    return int(lib().orc_row_bytes(qt, k))


def act_row_bytes(qt: int, k: int) -> int:
    return int(lib().orc_act_row_bytes(qt, k))


def fp32_to_fp16_bits(x: float) -> int:
    return int(lib().orc_fp32_to_fp16(float(x)))


def fp16_bits_to_fp32(h: int) -> float:
    return float(lib().orc_fp16_to_fp32(int(h)))


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.zeros(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0(_p(x), _p(y), x.size)
    return y


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.zeros(x.size // 32 * 36, np.uint8)
    lib().orc_quantize_q8_1(_p(x), _p(y), x.size)
    return y


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.zeros(x.size // 256 * 292, np.uint8)
    lib().orc_quantize_q8_K(_p(x), _p(y), x.size)
    return y


def quantize_act(qt: int, x: np.ndarray) -> np.ndarray:
    """Quantise each row of x into the activation format ggml pairs with qt."""
    x = np.ascontiguousarray(x, np.float32)
    k = x.shape[-1]
    rows = x.reshape(-1, k)
    ab = act_row_bytes(qt, k)
    y = np.zeros((rows.shape[0], ab), np.uint8)
    for r in range(rows.shape[0]):
        rr = np.ascontiguousarray(rows[r])
        assert lib().orc_quantize_act(qt, _p(rr), _p(y[r]), k) == 0
    return y.reshape(*x.shape[:-1], ab)


def quantize_weights(qt: int, w: np.ndarray) -> np.ndarray:
    """Encode each row of w (last axis = k) into qt blocks."""
    w = np.ascontiguousarray(w, np.float32)
    k = w.shape[-1]
    rows = w.reshape(-1, k)
    rb = row_bytes(qt, k)
    y = np.zeros((rows.shape[0], rb), np.uint8)
    L = lib()
    for r in range(rows.shape[0]):
        assert L.orc_quantize_weights(qt, _p(rows[r]), _p(y[r]), k) == 0
    return y.reshape(*w.shape[:-1], rb)


def dequantize(qt: int, raw: np.ndarray, k: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    rb = row_bytes(qt, k)
    rows = raw.reshape(-1, rb)
    out = np.zeros((rows.shape[0], k), np.float32)
    L = lib()
    for r in range(rows.shape[0]):
        assert L.orc_dequantize_row(qt, _p(rows[r]), _p(out[r]), k) == 0
    return out.reshape(*raw.shape[:-1], k)


def vec_dot(qt: int, w_row: np.ndarray, act_row: np.ndarray, k: int) -> float:
    w_row = np.ascontiguousarray(w_row, np.uint8)
    act_row = np.ascontiguousarray(act_row, np.uint8)
    return float(lib().orc_vec_dot(qt, _p(w_row), _p(act_row), k))


def mul_mat_id(bank: np.ndarray, x: np.ndarray, ids: np.ndarray, rows: int, k: int, qt: int,
               n_threads: int = 0) -> np.ndarray:
    """bank [E, rows, row_bytes] u8; x [T, x_rows, k] f32; ids [T, n_ids] i32 -> [T, n_ids, rows]."""
    bank = np.ascontiguousarray(bank, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    E = bank.shape[0]
    rb = bank.shape[-1]
    T, n_ids = ids.shape
    x_rows = x.shape[1]
    dst = np.zeros((T, n_ids, rows), np.float32)
    rc = lib().orc_mul_mat_id(_p(bank), rows * rb, rb,
                              _p(x), k * 4, x_rows, x_rows * k * 4,
                              _p(ids), 4, n_ids * 4, n_ids, T,
                              _p(dst), rows * 4, n_ids * rows * 4,
                              rows, k, E, qt, n_threads)
    if rc != 0:
        raise ValueError("oracle mul_mat_id rejected its arguments")
    return dst


def moe_layer(gate, up, down, qts, x, ids, w, shared=None, n_threads: int = 0,
              return_h: bool = False):
    """Gated expert FFN + combine for T tokens.

    gate/up: [E, d_ff, rb] u8, down: [E, d_model, rb] u8, qts = (qt_gate, qt_up, qt_down),
    x [T, d_model] f32, ids/w [T, n_used]; shared = (gate_s, up_s, down_s, qts_s) or
    (gate_s, up_s, down_s, qts_s, gate_inp) with gate_inp the [d_model] f32 gate row, or None.
    """
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    T, n_used = ids.shape
    D = x.shape[1]
    F = gate.shape[1]
    desc = MoeLayerDesc()
    desc.gate, desc.up, desc.down = gate.ctypes.data, up.ctypes.data, down.ctypes.data
    desc.qt_gate, desc.qt_up, desc.qt_down = qts
    desc.d_model, desc.d_ff, desc.n_experts = D, F, gate.shape[0]
    keep = []
    if shared is not None:
        sg, su, sd, sq = shared[:4]
        sg, su, sd = (np.ascontiguousarray(a, np.uint8) for a in (sg, su, sd))
        keep = [sg, su, sd]
        desc.shared_gate, desc.shared_up, desc.shared_down = sg.ctypes.data, su.ctypes.data, sd.ctypes.data
        desc.qt_shared_gate, desc.qt_shared_up, desc.qt_shared_down = sq
        desc.d_ff_shared = sg.shape[0]
        if len(shared) > 4 and shared[4] is not None:
            gi = np.ascontiguousarray(shared[4], np.float32).reshape(-1)
            if gi.size != D:
                raise ValueError("shared gate row has %d values, d_model is %d" % (gi.size, D))
            keep.append(gi)
            desc.shared_gate_inp = gi.ctypes.data
    out = np.zeros((T, D), np.float32)
    h = np.zeros((T, n_used, F), np.float32)
    rc = lib().orc_moe_layer(ctypes.byref(desc), _p(x), _p(ids), _p(w), n_used, T, _p(out), _p(h),
                             n_threads)
    del keep
    if rc != 0:
        raise ValueError("oracle moe_layer rejected its arguments")
    return (out, h) if return_h else out


def moe_route(logits: np.ndarray, n_used: int, norm_w: bool = True, w_scale: float = 1.0):
    """(ids [T, n_used] int32, w [T, n_used] f32) of ggml's softmax -> top-k -> renormalise."""
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    ids = np.zeros((T, n_used), np.int32)
    w = np.zeros((T, n_used), np.float32)
    if lib().orc_moe_route(_p(logits), T, E, n_used, int(norm_w), w_scale, _p(ids), _p(w)) != 0:
        raise ValueError("oracle moe_route rejected its arguments")
    return ids, w
