"""
Sabah / runtime / workloads

The five expert-path workloads the runtime is checked and measured on, by
name and shape.  Each names its quant types per role, its routing
construction, and its algorithmic expert bytes (the quantity throughput is
quoted against: every distinct expert matrix a step touches, counted once).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import routing
from .rt import QTYPE, row_bytes


@dataclass(frozen=True)
class Workload:
    name: str
    n_layers: int
    n_experts: int
    top_k: int
    d_model: int
    d_ff: int
    n_tokens: int
    qt_gate: int
    qt_up: int
    qt_down: int
    routing: str                      # "distinct_uniform" | "topk_normal" | "zipf"
    shared_d_ff: int = 0              # dense shared expert (0: none)
    qt_shared: int = QTYPE["Q8_0"]
    op: str = "layer"                 # "layer": the fused MoE layer; "mul_mat_id": the drop-in calls
    note: str = ""

    def matrix_bytes(self, role: str) -> int:
        if role in ("gate", "up"):
            return self.d_ff * row_bytes(self.qt_gate if role == "gate" else self.qt_up, self.d_model)
        return self.d_model * row_bytes(self.qt_down, self.d_ff)

    def expert_bytes(self) -> int:
        """gate + up + down bytes of one expert."""
        return sum(self.matrix_bytes(r) for r in ("gate", "up", "down"))

    def shared_bytes(self) -> int:
        if not self.shared_d_ff:
            return 0
        return (2 * self.shared_d_ff * row_bytes(self.qt_shared, self.d_model)
                + self.d_model * row_bytes(self.qt_shared, self.shared_d_ff))

    def bank_bytes(self) -> int:
        return self.n_layers * self.n_experts * self.expert_bytes()

    def route(self, rng: np.random.Generator, n_tokens: int | None = None, n_layers: int | None = None):
        """ids, weights of shape [n_layers, n_tokens, top_k]."""
        T = self.n_tokens if n_tokens is None else n_tokens
        L = self.n_layers if n_layers is None else n_layers
        ids = np.empty((L, T, self.top_k), np.int32)
        w = np.empty((L, T, self.top_k), np.float32)
        for l in range(L):
            if self.routing == "zipf":
                ids[l], w[l] = routing.zipf_routing(rng, T, self.n_experts, self.top_k)
            elif self.routing == "topk_normal":
                ids[l], w[l] = routing.uniform_routing(rng, T, self.n_experts, self.top_k)
            else:
                ids[l], w[l] = routing.distinct_uniform_routing(rng, T, self.n_experts, self.top_k)
        return ids, w

    def step_expert_bytes(self, ids: np.ndarray) -> int:
        """Algorithmic weight bytes of one step over ids [n_layers, n_tokens, k]:
        every distinct (layer, expert) counted once, plus the shared expert per layer."""
        total = 0
        for l in range(ids.shape[0]):
            total += len(np.unique(ids[l])) * self.expert_bytes() + self.shared_bytes()
        return total


Q8_0, Q4_K, Q6_K, IQ3_S = QTYPE["Q8_0"], QTYPE["Q4_K"], QTYPE["Q6_K"], QTYPE["IQ3_S"]

WORKLOADS = {
    "q8_0_e8_top2": Workload("q8_0_e8_top2", 1, 8, 2, 1024, 2048, 1, Q8_0, Q8_0, Q8_0, "distinct_uniform",
                             note="single MUL_MAT_ID decode on the CPU reference path"),
    "q4k_e128_top8": Workload("q4k_e128_top8", 1, 128, 8, 2048, 768, 1, Q4_K, Q4_K, Q4_K, "topk_normal",
                              note="Q4_K decode, one MoE layer"),
    "iq3s_48x512_top10": Workload("iq3s_48x512_top10", 48, 512, 10, 2048, 768, 1, IQ3_S, IQ3_S, IQ3_S, "zipf",
                                  note="IQ3_S decode, 48 MoE layers, bank fully HBM-resident"),
    "iq3s_mmid_48x512_top10": Workload("iq3s_mmid_48x512_top10", 48, 512, 10, 2048, 768, 1, IQ3_S, IQ3_S, IQ3_S,
                                       "zipf", op="mul_mat_id",
                                       note="the drop-in operator at decode: each of the 48 layers' gate, up and "
                                            "down MUL_MAT_ID calls for one token, as llama.cpp's hook makes them"),
    "iq3s_prefill_t512": Workload("iq3s_prefill_t512", 1, 512, 10, 2048, 768, 512, IQ3_S, IQ3_S, IQ3_S, "zipf",
                                  note="group-major prefill, one layer"),
    "iq3s_mmid_t512": Workload("iq3s_mmid_t512", 1, 512, 10, 2048, 768, 512, IQ3_S, IQ3_S, IQ3_S, "zipf",
                               op="mul_mat_id",
                               note="the drop-in operator over a 512-token prompt batch: one layer's gate, up "
                                    "and down MUL_MAT_ID calls"),
    "mixed_t32_q4k_q6k_shared": Workload("mixed_t32_q4k_q6k_shared", 1, 512, 10, 2048, 768, 32, Q4_K, Q4_K, Q6_K,
                                         "topk_normal", shared_d_ff=512, qt_shared=Q8_0,
                                         note="mixed-quant small-batch decode with a dense shared expert"),
}
