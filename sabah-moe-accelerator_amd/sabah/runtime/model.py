"""
Sabah / runtime / model

A GGUF model's routed-expert bank, from file to HBM.

inspect_model reads a GGUF (all shards of a split one) and returns a
ModelProfile: the geometry from the architecture's metadata keys, every
expert tensor with its absolute byte range, and the proof the runtime relies
on - each expert's slice of a tensor is one contiguous, block-aligned byte
range (expert axis slowest, per-expert bytes x n_experts = tensor bytes).  An
architecture is handled only if it is registered, and a model is "supported"
only if every expert tensor passes that proof and is a type the HIP kernels
decode.  This follows the reference's inspector
(sabah/core/model_inspector.py:122-327: registry, key prefix, tensor
patterns, contiguity proof, refusal with notes).

load_expert_bank copies the expert tensors of the chosen layers from the
read-only mapping into one ExpertBank allocation and verifies every copy
against the file with a position-weighted checksum computed on both sides,
in the spirit of the reference's byte-verify pass (sabah_rt.cu:553-618).
register_file_keys then registers each tensor under the host address
llama.cpp's mmap would hand MUL_MAT_ID as src0->data, so the drop-in entry
point runs on the HBM copy.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

import numpy as np
import torch

from . import gguf
from .bank import ROLES, ExpertBank

# the expert types the HIP kernels decode (ggml type codes)
RUNTIME_TYPES = {7: "Q5_1", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 18: "IQ3_XXS", 20: "IQ4_NL",
                 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 42: "Q2_0"}


class UnsupportedModel(Exception):
    """The file cannot be served by this runtime; the message says why."""


@dataclass
class ArchSpec:
    kv_prefix: str
    expert_pats: dict                   # role -> regex with the layer number as group 1
    shared_pats: dict = field(default_factory=dict)
    router_pat: str = ""
    shared_gate_inp_pat: str = ""


ARCHS = {
    "qwen4exp": ArchSpec(
        kv_prefix="qwen4exp",
        expert_pats={"gate": r"blk\.(\d+)\.ffn_gate_exps\.weight", "up": r"blk\.(\d+)\.ffn_up_exps\.weight",
                     "down": r"blk\.(\d+)\.ffn_down_exps\.weight"},
        shared_pats={"gate": r"blk\.(\d+)\.ffn_gate_shexp\.weight", "up": r"blk\.(\d+)\.ffn_up_shexp\.weight",
                     "down": r"blk\.(\d+)\.ffn_down_shexp\.weight"},
        router_pat=r"blk\.(\d+)\.ffn_gate_inp\.weight",
        shared_gate_inp_pat=r"blk\.(\d+)\.ffn_gate_inp_shexp\.weight",
    ),
}


@dataclass
class TensorRef:
    name: str
    layer: int
    role: str
    ggml_type: int
    shape: tuple                        # ne[0] first
    n_bytes: int
    shard: int
    data_offset: int                    # absolute offset in its shard
    per_expert_bytes: int = 0
    contiguous: bool = True


@dataclass
class ModelProfile:
    path: str
    shards: list
    architecture: str = ""
    n_layers: int = 0
    d_model: int = 0
    n_experts: int = 0
    n_used: int = 0
    expert_ff: int = 0
    experts: dict = field(default_factory=dict)      # (layer, role) -> TensorRef
    shared: dict = field(default_factory=dict)       # (layer, role) -> TensorRef (dense shared expert)
    shared_gate_inp: dict = field(default_factory=dict)   # layer -> TensorRef
    router: dict = field(default_factory=dict)       # layer -> TensorRef
    supported: bool = False
    notes: list = field(default_factory=list)

    @property
    def layers(self) -> list:
        return sorted({l for (l, _) in self.experts})

    @property
    def expert_bank_bytes(self) -> int:
        return sum(t.n_bytes for t in self.experts.values())

    def per_token_expert_bytes(self) -> int:
        return sum(t.per_expert_bytes for t in self.experts.values()) * self.n_used


def _kv_int(f: gguf.GgufFile, key: str) -> int:
    v = f.kv.get(key, 0)
    return int(v) if np.isscalar(v) or isinstance(v, (int, np.integer)) else 0


def inspect_model(path: str) -> ModelProfile:
    paths = gguf.shard_paths(path)
    files = [gguf.GgufFile(p) for p in paths]
    try:
        return _inspect(path, paths, files)
    finally:
        for f in files:
            f.close()


def _inspect(path, paths, files) -> ModelProfile:
    prof = ModelProfile(path=path, shards=list(paths))
    head = files[0]
    prof.architecture = str(head.kv.get("general.architecture", ""))
    spec = ARCHS.get(prof.architecture)
    if spec is None:
        prof.notes.append("architecture %r is not registered (registered: %s)"
                          % (prof.architecture, ", ".join(sorted(ARCHS))))
        return prof
    kp = spec.kv_prefix
    prof.n_layers = _kv_int(head, kp + ".block_count")
    prof.d_model = _kv_int(head, kp + ".embedding_length")
    prof.n_experts = _kv_int(head, kp + ".expert_count")
    prof.n_used = _kv_int(head, kp + ".expert_used_count")
    prof.expert_ff = _kv_int(head, kp + ".expert_feed_forward_length")
    if not (prof.n_layers and prof.d_model and prof.n_experts and prof.n_used and prof.expert_ff):
        prof.notes.append("the model does not declare its MoE geometry (block_count, embedding_length, "
                          "expert_count, expert_used_count, expert_feed_forward_length)")
        return prof
    ok = True
    want_shape = {"gate": (prof.d_model, prof.expert_ff), "up": (prof.d_model, prof.expert_ff),
                  "down": (prof.expert_ff, prof.d_model)}
    for si, f in enumerate(files):
        for t in f.tensors.values():
            for role, pat in spec.expert_pats.items():
                m = re.fullmatch(pat, t.name)
                if not m:
                    continue
                ref = TensorRef(t.name, int(m.group(1)), role, t.ggml_type, t.shape, t.n_bytes, si, t.data_offset)
                prof.experts[(ref.layer, role)] = ref
                if len(t.shape) != 3 or t.shape[2] != prof.n_experts:
                    ok = ref.contiguous = False
                    prof.notes.append("%s: the expert axis is not the slowest dimension (shape %s)"
                                      % (t.name, t.shape))
                    continue
                if tuple(t.shape[:2]) != want_shape[role]:
                    ok = ref.contiguous = False
                    prof.notes.append("%s: shape %s, expected %s x n_experts" % (t.name, t.shape, want_shape[role]))
                    continue
                if t.ggml_type not in gguf.GGML_TYPES:
                    ok = ref.contiguous = False
                    prof.notes.append("%s: unknown ggml type %d" % (t.name, t.ggml_type))
                    continue
                _, be, bb = gguf.GGML_TYPES[t.ggml_type]
                per = t.shape[0] // be * bb * t.shape[1]
                ref.per_expert_bytes = per
                if t.shape[0] % be or per * prof.n_experts != t.n_bytes:
                    ok = ref.contiguous = False
                    prof.notes.append("%s: per-expert slice is not block aligned" % t.name)
                if t.ggml_type not in RUNTIME_TYPES:
                    ok = False
                    prof.notes.append("%s: type %s is not decoded by the HIP kernels (they decode %s)"
                                      % (t.name, t.type_name, ", ".join(sorted(RUNTIME_TYPES.values()))))
            for role, pat in spec.shared_pats.items():
                m = re.fullmatch(pat, t.name)
                if m:
                    prof.shared[(int(m.group(1)), role)] = TensorRef(t.name, int(m.group(1)), role, t.ggml_type,
                                                                     t.shape, t.n_bytes, si, t.data_offset)
            for attr, pat in (("router", spec.router_pat), ("shared_gate_inp", spec.shared_gate_inp_pat)):
                m = re.fullmatch(pat, t.name) if pat else None
                if m:
                    getattr(prof, attr)[int(m.group(1))] = TensorRef(t.name, int(m.group(1)), attr, t.ggml_type,
                                                                     t.shape, t.n_bytes, si, t.data_offset)
    for l in range(prof.n_layers):
        missing = [r for r in ROLES if (l, r) not in prof.experts]
        if missing:
            ok = False
            prof.notes.append("layer %d has no %s expert tensor" % (l, "/".join(missing)))
        elif prof.experts[(l, "gate")].ggml_type != prof.experts[(l, "up")].ggml_type:
            ok = False
            prof.notes.append("layer %d: gate and up expert tensors differ in type (the fused kernel "
                              "takes one)" % l)
    prof.supported = ok and bool(prof.experts)
    if prof.supported:
        prof.notes.append("expert slices verified contiguous and block aligned across %d tensors"
                          % len(prof.experts))
    return prof


_CK_WORDS = 1 << 22


def _checksum(words: np.ndarray) -> int:
    """sum_i w_i * (i + 1) over the int32 words as int64, modulo 2^64 (in chunks)."""
    total = np.int64(0)
    with np.errstate(over="ignore"):
        for o in range(0, words.size, _CK_WORDS):
            w = words[o:o + _CK_WORDS].astype(np.int64)
            total = total + np.sum(w * np.arange(o + 1, o + 1 + w.size, dtype=np.int64), dtype=np.int64)
    return int(total)


def _checksum_dev(t: torch.Tensor) -> int:
    """The same on the device, over a uint8 tensor whose size is a multiple of 4."""
    words = t.view(torch.int32)
    total = torch.zeros((), dtype=torch.int64, device=t.device)
    for o in range(0, words.numel(), _CK_WORDS):
        w = words[o:o + _CK_WORDS].to(torch.int64)
        total += (w * torch.arange(o + 1, o + 1 + w.numel(), dtype=torch.int64, device=t.device)).sum()
    return int(total.item())


def load_expert_bank(prof: ModelProfile, device: str = "cuda:0", layers=None, verify: bool = True,
                     chunk_bytes: int = 64 << 20) -> ExpertBank:
    """The expert tensors of `layers` (default: all) copied into one HBM bank,
    bank layer i = model layer layers[i].  With verify, every tensor's device
    copy is checked against the file (position-weighted checksum of its 32-bit
    words, the odd tail bytes compared directly)."""
    if not prof.supported:
        raise UnsupportedModel("; ".join(prof.notes) or "model not supported")
    layers = list(prof.layers if layers is None else layers)
    qtypes = {(i, r): prof.experts[(l, r)].ggml_type for i, l in enumerate(layers) for r in ROLES}
    bank = ExpertBank(len(layers), prof.n_experts, prof.d_model, prof.expert_ff, qtypes, device=device)
    bank.model_layers = layers
    files = [gguf.GgufFile(p) for p in prof.shards]
    try:
        for i, l in enumerate(layers):
            for r in ROLES:
                ref = prof.experts[(l, r)]
                src = files[ref.shard].data(ref.name)
                dst = bank.tensor(i, r).view(-1)
                if src.size != dst.numel():
                    raise UnsupportedModel("%s: %d bytes in the file, %d in the bank" % (ref.name, src.size,
                                                                                         dst.numel()))
                for o in range(0, src.size, chunk_bytes):
                    n = min(chunk_bytes, src.size - o)
                    dst[o:o + n].copy_(torch.from_numpy(np.array(src[o:o + n])), non_blocking=False)
                if verify:
                    n4 = src.size // 4 * 4
                    host = _checksum(src[:n4].view(np.int32))
                    dev = _checksum_dev(dst[:n4]) if n4 else 0
                    tail_ok = np.array_equal(src[n4:], dst[n4:].cpu().numpy())
                    if host != dev or not tail_ok:
                        raise UnsupportedModel("%s: the HBM copy does not match the file" % ref.name)
    finally:
        for f in files:
            f.close()
    return bank


def register_file_keys(bank: ExpertBank, prof: ModelProfile, files=None) -> list:
    """Register every bank tensor under the host address its bytes have in a
    read-only mapping of the model file (what llama.cpp passes as
    src0->data).  `files` are open GgufFile objects for prof.shards (opened
    here if not given; the caller keeps them open while the keys are used).
    Returns the files."""
    files = files or [gguf.GgufFile(p) for p in prof.shards]
    for i, l in enumerate(getattr(bank, "model_layers", prof.layers)):
        for r in ROLES:
            ref = prof.experts[(l, r)]
            bank.register_tensor(i, r, files[ref.shard].base_address() + ref.data_offset)
    return files


def load_shared_expert(prof: ModelProfile, layer: int, device: str = "cuda:0"):
    """The layer's dense shared expert (and its sigmoid gate row, when the file
    has one) as a DenseExpert, or None when the layer has none."""
    from .bank import DenseExpert
    if not all((layer, r) in prof.shared for r in ROLES):
        return None
    g, u, d = (prof.shared[(layer, r)] for r in ROLES)
    if not (g.ggml_type == u.ggml_type == d.ggml_type) or g.ggml_type not in RUNTIME_TYPES:
        raise UnsupportedModel("layer %d: the shared expert needs one decodable type for its three tensors" % layer)
    fs = g.shape[1]
    ex = DenseExpert(prof.d_model, fs, g.ggml_type, device=device)
    files = [gguf.GgufFile(p) for p in prof.shards]
    try:
        for r, ref in zip(ROLES, (g, u, d)):
            ex.load(r, np.array(files[ref.shard].data(ref.name)))
        gi = prof.shared_gate_inp.get(layer)
        if gi is not None:
            if gi.ggml_type != 0 or gi.shape[0] != prof.d_model:
                raise UnsupportedModel("%s: the shared gate row must be f32 [d_model]" % gi.name)
            ex.set_gate(np.array(files[gi.shard].data(gi.name)).view(np.float32))
    finally:
        for f in files:
            f.close()
    return ex
