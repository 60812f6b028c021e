"""
Sabah / runtime / routing

Seeded router outputs (expert ids and combine weights) for the workloads the
runtime is measured on.  The router itself is outside the hooked operator
(qwen4exp.cpp:848-862 computes softmax -> top-k -> renormalised weights before
MUL_MAT_ID); these functions produce the same kind of ids/weights from
synthetic logits so that the expert path can be driven and checked.

All weights are `softmax(logits[selected])`, i.e. ggml's SOFTMAX gating with
norm_w=true restricted to the chosen experts.
"""
from __future__ import annotations

import numpy as np

# Zipf popularity bias: logit_e += -ZIPF_S * ZIPF_TAU * ln(rank_e).  With
# TAU = 0.22 a 512-token batch over 512 experts at top-10 has per-expert row
# counts from 0 to ~100 (mean max 98 over seeds 0..9), the spread the
# prefill workload is specified with.
ZIPF_S = 1.1
ZIPF_TAU = 0.22


def softmax_rows(logits: np.ndarray) -> np.ndarray:
    z = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def topk_from_logits(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """ids = k largest logits per row (descending), weights = softmax over them."""
    ids = np.argsort(-logits, axis=-1, kind="stable")[..., :k]
    sel = np.take_along_axis(logits, ids, axis=-1)
    return ids.astype(np.int32), softmax_rows(sel)


def zipf_bias(rng: np.random.Generator, n_experts: int, s: float = ZIPF_S, tau: float = ZIPF_TAU) -> np.ndarray:
    """Additive logit bias: a random permutation ranks the experts, rank r gets -s*tau*ln(r)."""
    perm = rng.permutation(n_experts)
    rank = np.empty(n_experts)
    rank[perm] = np.arange(1, n_experts + 1)
    return -s * tau * np.log(rank)


def zipf_routing(rng: np.random.Generator, n_tokens: int, n_experts: int, k: int,
                 n_layers: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Top-k of N(0,1) + Zipf-bias logits.  With n_layers, each layer has its
    own popularity ranking, shared by all n_tokens tokens; shapes
    [n_layers, n_tokens, k] (else [n_tokens, k])."""
    layers = 1 if n_layers is None else n_layers
    ids = np.empty((layers, n_tokens, k), np.int32)
    w = np.empty((layers, n_tokens, k), np.float32)
    for l in range(layers):
        bias = zipf_bias(rng, n_experts)
        logits = rng.standard_normal((n_tokens, n_experts)) + bias
        ids[l], w[l] = topk_from_logits(logits, k)
    return (ids[0], w[0]) if n_layers is None else (ids, w)


def uniform_routing(rng: np.random.Generator, n_tokens: int, n_experts: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Top-k of N(0,1) logits per token (every expert equally likely)."""
    logits = rng.standard_normal((n_tokens, n_experts))
    return topk_from_logits(logits, k)


def distinct_uniform_routing(rng: np.random.Generator, n_tokens: int, n_experts: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """k distinct experts drawn uniformly per token; weights = softmax of N(0,1) logits over them."""
    ids = np.stack([rng.choice(n_experts, k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    w = softmax_rows(rng.standard_normal((n_tokens, k)))
    return ids, w


def expected_unique(n_experts: int, k: int, n_tokens: int) -> float:
    """Expected number of distinct experts touched by n_tokens independent uniform top-k draws."""
    return n_experts * (1.0 - (1.0 - k / n_experts) ** n_tokens)
