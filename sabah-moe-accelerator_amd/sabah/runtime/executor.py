"""
Sabah / runtime / executor

Executes routed-MoE work on the HBM-resident bank.

The contract this file keeps (the reference's, executor.py:1-16):

    given router output (expert ids, routing weights), the arithmetic performed
    is exactly

        y = sum_k  w_k * W_down[e_k]^T ( silu(W_gate[e_k]^T x) * W_up[e_k]^T x )

    over the ids the router produced, using those experts' real quantized
    weights - with the activations quantised to q8 as ggml's CPU path does.

Every method calls the HIP runtime through the C ABI; there is no host-side
arithmetic and no fallback.  Work is enqueued on torch's current stream
(except `run_block`, which keeps the reference's library-stream signature).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import rt
from .bank import ROLES, DenseExpert, ExpertBank


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _vp(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


class MoEExecutor:
    def __init__(self, bank: ExpertBank, max_used: int = 16, max_tokens: int = 512,
                 shared: DenseExpert | None = None):
        rt.init(bank.device.index or 0)
        self.bank = bank
        self.shared = shared
        self.device = bank.device
        self.d_model = bank.d_model
        self.ff = bank.d_ff
        self.max_used = max_used
        dev = self.device
        self.d_x = torch.zeros(self.d_model, dtype=torch.float32, device=dev)
        self.d_out = torch.zeros(self.d_model, dtype=torch.float32, device=dev)
        self.d_h = torch.zeros(max_used * self.ff, dtype=torch.float32, device=dev)
        self.d_w = torch.zeros(max_used, dtype=torch.float32, device=dev)
        self.d_ptr = torch.zeros(3 * max_used, dtype=torch.int64, device=dev)

    # ---- reference-shaped block API (executor.py:42-98) --------------------
    def upload_x(self, x: np.ndarray) -> None:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.size != self.d_model:
            raise ValueError("x has %d elements, expected %d" % (x.size, self.d_model))
        self.d_x.copy_(torch.from_numpy(x))
        torch.cuda.current_stream(self.device).synchronize()

    def download_out(self) -> np.ndarray:
        self.sync()
        return self.d_out.cpu().numpy()

    def zero_out(self) -> None:
        self.d_out.zero_()
        torch.cuda.current_stream(self.device).synchronize()

    def run_block(self, block: int, ids, weights, accumulate: bool = False) -> None:
        """One MoE block for one token through sabah_moe_block (pointer table + weights on the device)."""
        ids = [int(i) for i in ids]
        w = np.ascontiguousarray(weights, dtype=np.float32)
        n = len(ids)
        if n != w.size:
            raise ValueError("%d ids but %d weights" % (n, w.size))
        if n > self.max_used:
            raise ValueError("n_used %d exceeds executor capacity %d" % (n, self.max_used))
        flat = np.array([self.bank.expert_ptr(block, r, e) for r in ROLES for e in ids], dtype=np.int64)
        self.d_ptr[:3 * n].copy_(torch.from_numpy(flat))
        self.d_w[:n].copy_(torch.from_numpy(w))
        torch.cuda.current_stream(self.device).synchronize()     # the block runs on the library stream
        q = {r: self.bank.layer_qtype(block, r) for r in ROLES}
        rt.check(rt.lib().sabah_moe_block(_vp(self.d_x), _vp(self.d_out), _vp(self.d_h), _vp(self.d_ptr),
                                          _vp(self.d_w), self.d_model, self.ff, n,
                                          q["gate"], q["up"], q["down"], 1 if accumulate else 0), "moe_block")

    def sync(self) -> None:
        rt.check(rt.lib().sabah_sync_compute(), "sync library stream")
        torch.cuda.current_stream(self.device).synchronize()

    # ---- the drop-in operator ----------------------------------------------
    def mul_mat_id(self, layer: int, role: str, x: torch.Tensor, ids: torch.Tensor,
                   out: torch.Tensor | None = None, source: int | None = None) -> torch.Tensor:
        """ggml MUL_MAT_ID through sabah_rt_mul_mat_id_v2 on (layer, role).

        x [n_tokens, x_rows, k] f32 (x_rows = 1 or n_ids), ids [n_tokens, n_ids] i32
        -> [n_tokens, n_ids, rows] f32.  `source` overrides the src0 address
        (e.g. a registered caller-side key)."""
        b = self.bank
        T, n_ids = ids.shape
        rows, k, qt = b.rows[role], b.cols[role], b.layer_qtype(layer, role)
        if out is None:
            out = torch.empty(T, n_ids, rows, dtype=torch.float32, device=self.device)
        src = b.base_ptr(layer, role) if source is None else source
        rc = rt.lib().sabah_rt_mul_mat_id_v2(
            ctypes.c_void_p(src), b.layer_stride(layer, role), b.layer_row_bytes(layer, role),
            _vp(x), x.stride(1) * 4, x.shape[1], x.stride(0) * 4,
            _vp(ids), ids.stride(1) * 4, ids.stride(0) * 4, n_ids, T,
            _vp(out), out.stride(1) * 4, out.stride(0) * 4,
            rows, k, b.n_experts, qt, _stream(self.device), _vp(ids))
        rt.check(rc, "MUL_MAT_ID")
        return out

    # ---- fused layer / chain --------------------------------------------------
    def run_layer(self, layer: int, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor,
                  out: torch.Tensor | None = None, resid: torch.Tensor | None = None) -> torch.Tensor:
        """One MoE layer for x [T, d_model] with ids/w [T, k]; adds the shared expert if the
        executor has one and `resid` if given."""
        if out is None:
            out = torch.empty_like(x)
        desc = self.bank.layer_desc(layer, self.shared)
        T, k = ids.shape
        rt.check(rt.lib().sabah_moe_layer(ctypes.byref(desc), _vp(x), _vp(ids), _vp(w), k, T, _vp(out),
                                          _vp(resid) if resid is not None else None, _stream(self.device)),
                 "moe_layer")
        return out

    def route(self, logits: torch.Tensor, n_used: int | None = None, norm_w: bool = True,
              w_scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
        """Router gating on the device (sabah_moe_route): ids [T, n_used] int32 and
        weights [T, n_used] f32 from router logits [T, n_experts] f32."""
        k = self.max_used if n_used is None else n_used
        T, E = logits.shape
        ids = torch.empty((T, k), dtype=torch.int32, device=logits.device)
        w = torch.empty((T, k), dtype=torch.float32, device=logits.device)
        rt.check(rt.lib().sabah_moe_route(_vp(logits), T, E, k, int(norm_w), ctypes.c_float(w_scale), _vp(ids),
                                          _vp(w), _stream(self.device)), "moe_route")
        return ids, w

    def run_prefill_layer(self, layer: int, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor,
                          out: torch.Tensor | None = None, resid: torch.Tensor | None = None) -> torch.Tensor:
        """run_layer computed group-major (sabah_moe_prefill_layer): the (token, slot)
        pairs grouped by expert on the device, each expert's rows read once."""
        if out is None:
            out = torch.empty_like(x)
        desc = self.bank.layer_desc(layer, self.shared)
        T, k = ids.shape
        rt.check(rt.lib().sabah_moe_prefill_layer(ctypes.byref(desc), _vp(x), _vp(ids), _vp(w), k, T, _vp(out),
                                                  _vp(resid) if resid is not None else None,
                                                  _stream(self.device)), "moe_prefill_layer")
        return out

    def layer_descs(self) -> ctypes.Array:
        arr = (rt.MoeLayerDesc * self.bank.n_layers)()
        for l in range(self.bank.n_layers):
            arr[l] = self.bank.layer_desc(l, self.shared)
        return arr

    def run_chain(self, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, descs=None) -> torch.Tensor:
        """x <- x + layer_l(x) for every layer, in place; ids/w [n_layers, T, k]."""
        L, T, k = ids.shape
        descs = self.layer_descs() if descs is None else descs
        rt.check(rt.lib().sabah_moe_chain(descs, L, _vp(x), _vp(ids), _vp(w), k, T, _stream(self.device)),
                 "moe_chain")
        return x


class ChainGraph:
    """The decode chain (every layer's gate/up and down kernels) captured once
    as a HIP graph over static x / ids / weights buffers.  replay() copies one
    step's inputs in and replays the graph: the host submits one graph per
    step instead of two kernels per layer.  An eager call before the capture
    sizes the library scratch, so nothing is allocated inside it.  The graph
    keeps the scratch it was captured with: a later, larger call grows the
    library scratch by allocating new buffers and retires the old ones without
    freeing them (they live until sabah_rt_shutdown), so replays stay valid.
    Replays and eager calls must not overlap on different streams: both use
    the same scratch while no call has outgrown it."""

    def __init__(self, ex: MoEExecutor, n_tokens: int, k: int, descs=None):
        dev = ex.device
        self.ex = ex
        self.descs = ex.layer_descs() if descs is None else descs
        L = len(self.descs)                   # a chain may apply a layer more than once
        self.x = torch.zeros(n_tokens, ex.d_model, dtype=torch.float32, device=dev)
        self.ids = torch.zeros(L, n_tokens, k, dtype=torch.int32, device=dev)
        self.w = torch.zeros(L, n_tokens, k, dtype=torch.float32, device=dev)
        ex.run_chain(self.x, self.ids, self.w, self.descs)       # eager: sizes the library scratch
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            ex.run_chain(self.x, self.ids, self.w, self.descs)
        torch.cuda.synchronize(dev)

    def replay(self, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """x [n_tokens, d_model], ids / w [n_layers, n_tokens, k]; returns the
        static output buffer (valid in stream order)."""
        self.x.copy_(x)
        self.ids.copy_(ids)
        self.w.copy_(w)
        self.graph.replay()
        return self.x

    def replay_static(self) -> torch.Tensor:
        """Replay on the inputs already in place: the graph's launches only."""
        self.graph.replay()
        return self.x
