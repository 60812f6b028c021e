"""
Sabah / runtime / bank

The HBM-resident expert bank.  The reference streams experts from disk into
a VRAM LRU tier keyed by (source tensor, expert) (sabah_rt.cu:97-106,
748-800; sabah/runtime/hot_tier.py:148-578); with 288 GB of HBM3E the whole
bank of the shipped model shape (48 layers x 3 roles x 512 IQ3_S experts,
49.8 GB) is resident, so residency reduces to one device allocation and an
address table: expert e of (layer, role) is at base[layer][role] + e * expert_stride.

Layout in HBM: one allocation; inside it, per layer, the gate, up and down
tensors back to back, each in GGUF layout [n_experts][rows][row_bytes]
(rows contiguous, experts contiguous), every tensor 256-byte aligned.  This is
exactly the layout llama.cpp hands MUL_MAT_ID as src0, so the same bytes serve
the drop-in entry point and the fused layer entry points.

Identity discipline (sabah/runtime/identity.py:14-50): a matrix is addressed
by (layer, role) and an expert by (layer, role, expert) - never by a bare
expert number - so ids never alias across layers.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import rt

ROLES = ("gate", "up", "down")
_ALIGN = 256


class ExpertBank:
    """qtypes: role -> ggml type code for every layer, or (layer, role) -> code
    (a GGUF may quantise each layer's tensors differently).  `qtypes`,
    `row_bytes` and `expert_stride` stay keyed by role when every layer agrees;
    the per-layer forms are `layer_qtype`, `layer_row_bytes`, `layer_stride`."""

    def __init__(self, n_layers: int, n_experts: int, d_model: int, d_ff: int,
                 qtypes: dict, device: str = "cuda:0"):
        self.n_layers, self.n_experts = n_layers, n_experts
        self.d_model, self.d_ff = d_model, d_ff
        self.lq = {}
        for l in range(n_layers):
            for r in ROLES:
                self.lq[(l, r)] = int(qtypes[(l, r)] if (l, r) in qtypes else qtypes[r])
        self.device = torch.device(device)
        self.rows = {"gate": d_ff, "up": d_ff, "down": d_model}
        self.cols = {"gate": d_model, "up": d_model, "down": d_ff}
        uniform = all(len({self.lq[(l, r)] for l in range(n_layers)}) == 1 for r in ROLES)
        self.qtypes = {r: self.lq[(0, r)] for r in ROLES} if uniform else None
        self.row_bytes = {r: rt.row_bytes(self.qtypes[r], self.cols[r]) for r in ROLES} if uniform else None
        self.expert_stride = {r: self.rows[r] * self.row_bytes[r] for r in ROLES} if uniform else None
        self.offsets = {}
        off = 0
        for l in range(n_layers):
            for r in ROLES:
                self.offsets[(l, r)] = off
                off += (self.layer_stride(l, r) * n_experts + _ALIGN - 1) // _ALIGN * _ALIGN
        self.total_bytes = off
        self.storage = torch.empty(self.total_bytes, dtype=torch.uint8, device=self.device)
        self._registered = []

    def layer_qtype(self, layer: int, role: str) -> int:
        return self.lq[(layer, role)]

    def layer_row_bytes(self, layer: int, role: str) -> int:
        return rt.row_bytes(self.lq[(layer, role)], self.cols[role])

    def layer_stride(self, layer: int, role: str) -> int:
        return self.rows[role] * self.layer_row_bytes(layer, role)

    # ---- addressing ----------------------------------------------------------
    def tensor(self, layer: int, role: str) -> torch.Tensor:
        """[n_experts, rows, row_bytes] uint8 view of one (layer, role) tensor."""
        o = self.offsets[(layer, role)]
        n = self.layer_stride(layer, role) * self.n_experts
        return self.storage[o:o + n].view(self.n_experts, self.rows[role], self.layer_row_bytes(layer, role))

    def base_ptr(self, layer: int, role: str) -> int:
        return self.storage.data_ptr() + self.offsets[(layer, role)]

    def expert_ptr(self, layer: int, role: str, expert: int) -> int:
        if not 0 <= expert < self.n_experts:
            raise IndexError("expert %d outside [0, %d)" % (expert, self.n_experts))
        return self.base_ptr(layer, role) + expert * self.layer_stride(layer, role)

    def expert_bytes(self, layer: int, expert: int) -> int:
        return sum(self.layer_stride(layer, r) for r in ROLES)

    # ---- filling -------------------------------------------------------------
    def fill_synthetic(self, seed: int, sigma: float = 0.02, layers=None) -> None:
        """N(0, sigma) weights quantised on the device; (layer, role) gets its own seed."""
        L = rt.lib()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        for l in (range(self.n_layers) if layers is None else layers):
            for i, r in enumerate(ROLES):
                s = (int(seed) * 1000003 + l * 8 + i) & 0xFFFFFFFFFFFFFFFF
                rt.check(L.sabah_synth_weights(ctypes.c_void_p(self.base_ptr(l, r)), self.lq[(l, r)],
                                               self.n_experts * self.rows[r], self.cols[r],
                                               ctypes.c_ulonglong(s), ctypes.c_float(sigma),
                                               ctypes.c_void_p(stream)), "synth weights")

    def load(self, layer: int, role: str, raw: np.ndarray) -> None:
        """Copy host bytes [n_experts, rows, row_bytes] into (layer, role)."""
        t = self.tensor(layer, role)
        raw = np.ascontiguousarray(raw, np.uint8).reshape(t.shape)
        t.copy_(torch.from_numpy(raw))

    def read_expert(self, layer: int, role: str, expert: int) -> np.ndarray:
        """Host copy of one expert matrix [rows, row_bytes] (what the CPU baseline reads)."""
        return self.tensor(layer, role)[expert].cpu().numpy()

    # ---- runtime registration ----------------------------------------------
    def register(self, key_base: int | None = None) -> None:
        """Register every (layer, role) tensor with the runtime.  By default the
        key is the device address itself; pass key_base to key the tensors by a
        caller-side address range (as llama.cpp's host mmap addresses are)."""
        L = rt.lib()
        for (l, r), o in self.offsets.items():
            key = (key_base + o) if key_base is not None else self.base_ptr(l, r)
            self.register_tensor(l, r, key)

    def register_tensor(self, layer: int, role: str, key: int) -> None:
        """Register one (layer, role) tensor under a caller-side key address."""
        L = rt.lib()
        stride = self.layer_stride(layer, role)
        rt.check(L.sabah_rt_register_bank(ctypes.c_void_p(key), ctypes.c_void_p(self.base_ptr(layer, role)),
                                          stride * self.n_experts, stride, self.n_experts), "register bank")
        self._registered.append(key)

    def unregister(self) -> None:
        L = rt.lib()
        for key in self._registered:
            L.sabah_rt_unregister_bank(ctypes.c_void_p(key))
        self._registered = []

    def layer_desc(self, layer: int, shared=None) -> rt.MoeLayerDesc:
        """sabah_moe_layer_desc of one layer; shared = DenseExpert or None."""
        d = rt.MoeLayerDesc()
        d.gate, d.up, d.down = (self.base_ptr(layer, r) for r in ROLES)
        d.qt_gate, d.qt_up, d.qt_down = (self.lq[(layer, r)] for r in ROLES)
        d.d_model, d.d_ff, d.n_experts = self.d_model, self.d_ff, self.n_experts
        if shared is not None:
            d.shared_gate, d.shared_up, d.shared_down = shared.ptrs()
            d.qt_shared_gate = d.qt_shared_up = d.qt_shared_down = shared.qt
            d.d_ff_shared = shared.d_ff
            if shared.gate_inp is not None:
                d.shared_gate_inp = shared.gate_inp.data_ptr()
        return d


class DenseExpert:
    """An always-on shared expert: three dense matrices of one quant type, and
    optionally its f32 gate row (ffn_gate_inp_shexp, qwen4exp.cpp:877-885): the
    expert's output is then scaled by sigmoid(gate_inp . x) before it is added."""

    def __init__(self, d_model: int, d_ff: int, qt: int, device: str = "cuda:0"):
        self.d_model, self.d_ff, self.qt = d_model, d_ff, qt
        self.rows = {"gate": d_ff, "up": d_ff, "down": d_model}
        self.cols = {"gate": d_model, "up": d_model, "down": d_ff}
        self.mats = {r: torch.empty(self.rows[r], rt.row_bytes(qt, self.cols[r]), dtype=torch.uint8,
                                    device=device) for r in ROLES}
        self.gate_inp = None

    def set_gate(self, row: np.ndarray | None) -> None:
        """The shared expert's gate row ([d_model] f32), or None for an ungated add."""
        if row is None:
            self.gate_inp = None
            return
        row = np.ascontiguousarray(row, np.float32).reshape(-1)
        if row.size != self.d_model:
            raise ValueError("gate row has %d values, d_model is %d" % (row.size, self.d_model))
        self.gate_inp = torch.from_numpy(row).to(self.mats["gate"].device)

    def ptrs(self):
        return tuple(self.mats[r].data_ptr() for r in ROLES)

    def read(self, role: str) -> np.ndarray:
        """Host copy of one matrix [rows, row_bytes]."""
        return self.mats[role].cpu().numpy()

    def load(self, role: str, raw: np.ndarray) -> None:
        self.mats[role].copy_(torch.from_numpy(np.ascontiguousarray(raw, np.uint8).reshape(self.mats[role].shape)))

    def fill_synthetic(self, seed: int, sigma: float = 0.02) -> None:
        L = rt.lib()
        stream = torch.cuda.current_stream(self.mats["gate"].device).cuda_stream
        for i, r in enumerate(ROLES):
            rt.check(L.sabah_synth_weights(ctypes.c_void_p(self.mats[r].data_ptr()), self.qt, self.rows[r],
                                           self.cols[r], ctypes.c_ulonglong(seed * 7919 + i), ctypes.c_float(sigma),
                                           ctypes.c_void_p(stream)), "synth shared expert")
