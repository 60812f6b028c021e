"""Synthetic GGUF model files for the loader tests (written by the package's own
writer, sabah.runtime.gguf.write_gguf; no reference file is read)."""
from __future__ import annotations

import numpy as np

from sabah.runtime import gguf

ARCH = "qwen4exp"


def expert_tensors(orc, rng, layer, role, qt, E, rows, cols):
    if qt in (18, 22):    # IQ3_XXS, IQ2_S: no encoder here; random valid blocks
        from helpers import random_blocks
        raw = random_blocks(rng, qt, E * rows, cols).reshape(E, rows, -1)
    else:
        w = (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32)
        raw = orc.quantize_weights(qt, w)
    t = gguf.WriterTensor("blk.%d.ffn_%s_exps.weight" % (layer, role), (cols, rows, E), qt, raw)
    return t, raw


def write_model(path, orc, rng, n_layers=2, E=8, D=512, F=256, n_used=4, layer_types=None, Fs=0,
                shared_qt=8, gate_inp_shexp=False, extra_kv=(), layers=None):
    """A qwen4exp GGUF with routed experts (and optionally a shared expert, its
    gate row, and router rows).  layer_types[l] = (qt_gate, qt_up, qt_down).
    Returns the raw expert bytes {(layer, role): [E, rows, row_bytes]} and the
    shared-expert bytes {(layer, role): [rows, row_bytes]}."""
    layer_types = layer_types or [(21, 21, 21)] * n_layers
    kv = [("general.architecture", gguf.STR, ARCH), ("general.alignment", gguf.U32, 32),
          ("%s.block_count" % ARCH, gguf.U32, n_layers), ("%s.embedding_length" % ARCH, gguf.U32, D),
          ("%s.expert_count" % ARCH, gguf.U32, E), ("%s.expert_used_count" % ARCH, gguf.U32, n_used),
          ("%s.expert_feed_forward_length" % ARCH, gguf.U32, F)] + list(extra_kv)
    tensors, raws, shared = [], {}, {}
    for l in (range(n_layers) if layers is None else layers):
        qg, qu, qd = layer_types[l]
        for role, qt, rows, cols in (("gate", qg, F, D), ("up", qu, F, D), ("down", qd, D, F)):
            t, raw = expert_tensors(orc, rng, l, role, qt, E, rows, cols)
            tensors.append(t)
            raws[(l, role)] = raw
        r = (rng.standard_normal((E, D)) * 0.1).astype(np.float32)
        tensors.append(gguf.WriterTensor("blk.%d.ffn_gate_inp.weight" % l, (D, E), 0, r))
        if Fs:
            for role, rows, cols in (("gate", Fs, D), ("up", Fs, D), ("down", D, Fs)):
                raw = orc.quantize_weights(shared_qt, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
                tensors.append(gguf.WriterTensor("blk.%d.ffn_%s_shexp.weight" % (l, role), (cols, rows), shared_qt,
                                                 raw))
                shared[(l, role)] = raw
            if gate_inp_shexp:
                g = (rng.standard_normal(D) * 0.05).astype(np.float32)
                tensors.append(gguf.WriterTensor("blk.%d.ffn_gate_inp_shexp.weight" % l, (D, 1), 0, g))
                shared[(l, "gate_inp")] = g
    gguf.write_gguf(path, kv, tensors)
    return raws, shared
