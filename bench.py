#!/usr/bin/env python3
"""Decode benchmark of the MoE MUL_MAT_ID expert path on one MI355X.

Workload (default): IQ3_S decode at the shipped model shape - 48 MoE layers x
512 experts, top-10, d_model 2048, d_ff 768, one token per step.  The whole
49.8 GB bank is generated in HBM (N(0, 0.02) weights quantised on the
device); per-layer ids are the top-10 of N(0,1) + Zipf(1.1) popularity-biased
router logits; x ~ N(0, 1).  A step is one token through the 48 layers on a
residual stream (x <- x + layer(x)); each layer's expert weights are read
only after the previous layer has finished, as a real decode must.  128
distinct tokens rotate, so a step's 973 MB of expert bytes are never served
from the 256 MB last-level cache of the previous step.

Prints one JSON line (rank 0).  `value` is expert GB/s: algorithmic expert
bytes (each routed expert matrix counted once per layer) / wall time.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "sabah-moe-accelerator_amd")
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0
METRIC = "MUL_MAT_ID expert GB/s (% HBM peak) + decode tok/s over 48 MoE layers, 1 GPU"
ONE_LAYER_CHAIN = 48                   # layer calls per step for a one-layer workload


def quant_note(W):
    from sabah.runtime.rt import QTYPE_NAME
    names = [QTYPE_NAME[q] for q in (W.qt_gate, W.qt_up, W.qt_down)]
    return names[0] if len(set(names)) == 1 else "%s gate/up, %s down" % (names[0], names[2])


def compute_note(W):
    from sabah.runtime.rt import QTYPE_NAME
    acts = sorted({"q8_0" if q in (8, 20, 42) else "q8_K" for q in (W.qt_gate, W.qt_up, W.qt_down)})
    return ("int8 x int8 -> int32 dot products (%s weights decoded to int8, %s activations), fp32 scales and "
            "accumulation" % (quant_note(W), " / ".join(acts)))


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="iq3s_48x512_top10")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--pool", type=int, default=128, help="distinct tokens rotated through the steps")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0: every CPU this process may run on (OMP_NUM_THREADS when set: the host's CPU share)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--layer-fusion", type=int, default=1, choices=(0, 1),
                    help="1 (the library's default): one fused launch per layer; 0: gate/up then down + combine")
    ap.add_argument("--grouping", default="auto", choices=("auto", "off"),
                    help="batch workloads: auto runs the group-major layer when it takes the workload's types "
                         "(gate/up of one type, each of IQ3_S, Q4_K, Q6_K) and there are at least 2 "
                         "(token, slot) pairs per expert; off runs token-major")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="finish with one device-to-device copy of this many MiB (a plain copy kernel of known "
                         "size, to calibrate the FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: the expert path here runs on a single MI355X "
              "(--gpus %d requested; multi-GPU sharding is a design note, not a measured mode)" % args.gpus,
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from sabah.runtime import rt
    from sabah.runtime.bank import ExpertBank
    from sabah.runtime.executor import ChainGraph, MoEExecutor
    from sabah.runtime.workloads import WORKLOADS

    W = WORKLOADS[args.workload]
    if W.n_tokens > 1:
        return bench_batch(args, W)
    if W.op == "mul_mat_id":
        return bench_mmid_decode(args, W)
    dev = torch.device("cuda:0")
    rt.init(0)
    rt.check(rt.lib().sabah_rt_set_layer_fusion(args.layer_fusion), "layer fusion mode")
    t0 = time.time()
    bank = ExpertBank(W.n_layers, W.n_experts, W.d_model, W.d_ff,
                      {"gate": W.qt_gate, "up": W.qt_up, "down": W.qt_down}, device="cuda:0")
    bank.fill_synthetic(seed=args.seed)
    torch.cuda.synchronize()
    print("bank: %.1f GB generated in HBM in %.1f s" % (bank.total_bytes / 1e9, time.time() - t0),
          file=sys.stderr, flush=True)

    rng = np.random.default_rng(args.seed)
    P = args.pool
    # a step runs the chain of G layer calls: the model's layers, or for a
    # one-layer workload G calls of that layer (each with its own ids), so a
    # ~10 us layer is not measured behind one graph launch per call
    G = W.n_layers if W.n_layers > 1 else ONE_LAYER_CHAIN
    ids_np, w_np = W.route(rng, n_tokens=P, n_layers=G)             # [G, P, k]
    ids_np = np.ascontiguousarray(ids_np.transpose(1, 0, 2))[:, :, None, :]   # [P, G, 1, k]
    w_np = np.ascontiguousarray(w_np.transpose(1, 0, 2))[:, :, None, :]
    # a model's chain carries x from layer to layer; a one-layer workload's G
    # calls each get their own input row (the same layer applied G times on
    # one residual stream grows x without bound: the gated FFN is quadratic)
    x_np = rng.standard_normal((P, 1 if W.n_layers > 1 else G, W.d_model)).astype(np.float32)
    ids = torch.from_numpy(ids_np).to(dev)
    wts = torch.from_numpy(w_np).to(dev)
    xs = torch.from_numpy(x_np).to(dev)
    ex = MoEExecutor(bank, max_used=W.top_k)
    step_bytes = [W.step_expert_bytes(ids_np[p, :, 0][:, None, :]) for p in range(P)]
    if W.n_layers > 1:
        x_buf = torch.empty(1, W.d_model, dtype=torch.float32, device=dev)
        descs = ex.layer_descs()

        def eager_step(i):
            p = i % P
            x_buf.copy_(xs[p])
            ex.run_chain(x_buf, ids[p], wts[p], descs)
            return x_buf

        # the timed steps replay the chain captured as one HIP graph
        cg = ChainGraph(ex, 1, W.top_k, descs)
    else:
        y_buf = torch.empty(G, W.d_model, dtype=torch.float32, device=dev)

        def eager_step(i):
            p = i % P
            for g in range(G):
                ex.run_layer(0, xs[p, g:g + 1], ids[p, g], wts[p, g], out=y_buf[g:g + 1])
            return y_buf

        cg = LayerCallsGraph(ex, G, W.d_model, W.top_k)

    def graph_step(i):
        p = i % P
        cg.replay(xs[p], ids[p], wts[p])

    # the graph computes what the eager calls compute, bit for bit
    y_eager = eager_step(0).clone()
    graph_step(0)
    torch.cuda.synchronize()
    if not torch.equal(y_eager, cg.x):
        print("graph replay differs from the eager calls", file=sys.stderr)
        return 1

    def timed(step_fn, steps):
        for i in range(args.warmup):
            step_fn(i)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for i in range(args.warmup, args.warmup + steps):
            step_fn(i)
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1)

    ms_total = timed(graph_step, args.steps)
    ms_step = ms_total / args.steps
    nbytes = sum(step_bytes[i % P] for i in range(args.warmup, args.warmup + args.steps))
    gbs = nbytes / (ms_total * 1e6)

    # a layer's launches as the replayed graph runs them: the bare graph (the
    # last step's inputs in place, no copies in) replayed R times, HIP events
    # on the stream it replays on; per layer = one fused launch, or the
    # gate/up and down launches
    R = max(4, args.steps // 2)
    cg.replay_static()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(R):
        cg.replay_static()
    ev1.record()
    torch.cuda.synchronize()
    us_layer_graph = 1000.0 * ev0.elapsed_time(ev1) / (R * G)
    last = (args.warmup + args.steps - 1) % P
    layer_bytes_last = step_bytes[last] / G                        # distinct expert bytes per layer call

    # per-kernel durations: the same steps run eagerly, each dispatch recording
    # its own start/stop HIP event pair on the stream it runs on
    L = rt.lib()
    L.sabah_rt_set_kernel_timing(1)
    for kind in rt.KERNEL_KINDS:
        rt.kernel_timing(kind, reset=True)
    ms_eager = timed(eager_step, args.steps)
    L.sabah_rt_set_kernel_timing(0)
    kernels = {}
    for kind in rt.KERNEL_KINDS:
        ms, n = rt.kernel_timing(kind)
        if n:
            kernels[kind] = {"launches": n, "avg_us": 1000.0 * ms / n, "total_ms": ms}
    # algorithmic bytes of one layer call: its k routed expert matrices (every
    # slot's, as the kernels read them: distinct ids at one token), x, h
    # written and read, the weights and the output
    k_used = W.top_k
    per_launch = {
        "gate_up": k_used * (W.matrix_bytes("gate") + W.matrix_bytes("up")) + 4 * W.d_model + 4 * k_used * W.d_ff,
        "down": k_used * W.matrix_bytes("down") + 4 * k_used * W.d_ff + 4 * (2 * W.d_model + k_used),
    }
    per_launch["layer"] = per_launch["gate_up"] + per_launch["down"]
    fused = "layer" in kernels
    achieved = per_launch["layer"] / (us_layer_graph * 1e3)                  # GB/s
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(W.name, ["layer"] if fused else ["gate_up", "down"]),
                "kernel": "layer" if fused else "layer (gate_up + down launches)",
                "bytes_per_launch": per_launch["layer"], "avg_launch_us": round(us_layer_graph, 3),
                "timing": "replayed graph, %d replays of %d layer calls" % (R, G)}

    cpu = None
    parity = None
    if not args.no_cpu:
        cpu, parity = cpu_baseline(args, W, bank, ex, ids_np, w_np, x_np[:, :1], dev)

    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "compute": compute_note(W),
        "data": "synthetic (N(0,0.02) weights quantised on device; %s routing; seeded)" % W.routing,
        "config": {"workload": W.name, "n_layers": W.n_layers, "n_experts": W.n_experts, "top_k": W.top_k,
                   "d_model": W.d_model, "d_ff": W.d_ff, "n_tokens": W.n_tokens, "quant": quant_note(W),
                   "bank_bytes": bank.total_bytes, "expert_bytes_per_step": nbytes // args.steps,
                   "layer_calls_per_step": G,
                   "mode": ("%s; %s" % (
                       "one fused launch per layer (gate/up+SwiGLU and down+combine workgroups in one grid, h "
                       "handed over in the kernel)" if fused else
                       "two launches per layer (gate/up+SwiGLU, down+combine)",
                       "the %d layers' launches replayed as one HIP graph per step (a residual chain)" % G
                       if W.n_layers > 1 else
                       "%d calls of the layer, each on its own input row, replayed as one HIP graph per step" % G))},
        "tok_s": round(1000.0 * (1 if W.n_layers > 1 else G) / ms_step, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "us_per_layer": round(1000.0 * ms_step / G, 3),
        "kernels": {k: {"launches": v["launches"], "avg_us": round(v["avg_us"], 3)} for k, v in kernels.items()},
        "eager_ms_per_step": round(ms_eager / args.steps, 4),
        "roofline": roofline, "cpu_baseline": cpu, "parity": parity,
    }
    print(json.dumps(line), flush=True)
    copy_probe(args, dev)
    return 0


def bench_mmid_decode(args, W):
    """Decode through the drop-in operator: per layer, the gate, up and down
    sabah_rt_mul_mat_id_v2 calls of one token, as llama.cpp's hook makes them
    (its graph's SwiGLU and weighted combine between and after the calls are
    ggml ops, outside the path: down reads a fixed synthetic h).  The 48
    layers' 144 calls replay as one HIP graph per step over static id
    buffers; `value` is the step's distinct expert bytes / wall time, as for
    the fused chain.  Layer 0's three calls are checked against the oracle,
    bit for bit."""
    import numpy as np
    import torch

    from sabah.runtime import rt
    from sabah.runtime.bank import ExpertBank
    from sabah.runtime.executor import MoEExecutor

    dev = torch.device("cuda:0")
    rt.init(0)
    t0 = time.time()
    bank = ExpertBank(W.n_layers, W.n_experts, W.d_model, W.d_ff,
                      {"gate": W.qt_gate, "up": W.qt_up, "down": W.qt_down}, device="cuda:0")
    bank.fill_synthetic(seed=args.seed)
    torch.cuda.synchronize()
    print("bank: %.1f GB generated in HBM in %.1f s" % (bank.total_bytes / 1e9, time.time() - t0),
          file=sys.stderr, flush=True)
    rng = np.random.default_rng(args.seed)
    P, G, k = args.pool, W.n_layers, W.top_k
    ids_np, _ = W.route(rng, n_tokens=P, n_layers=G)                # [G, P, k]
    ids_np = np.ascontiguousarray(ids_np.transpose(1, 0, 2))[:, :, None, :]   # [P, G, 1, k]
    x_np = rng.standard_normal((P, 1, 1, W.d_model)).astype(np.float32)
    h_np = rng.standard_normal((1, k, W.d_ff)).astype(np.float32)
    ids_all = torch.from_numpy(ids_np).to(dev)
    xs = torch.from_numpy(x_np).to(dev)
    ex = MoEExecutor(bank, max_used=k)
    ids_s = torch.zeros(G, 1, k, dtype=torch.int32, device=dev)
    x_s = torch.zeros(1, 1, W.d_model, dtype=torch.float32, device=dev)
    h_s = torch.from_numpy(h_np).to(dev)
    g_out = torch.empty(G, 1, k, W.d_ff, device=dev)
    u_out = torch.empty_like(g_out)
    d_out = torch.empty(G, 1, k, W.d_model, device=dev)

    def calls():
        for l in range(G):
            ex.mul_mat_id(l, "gate", x_s, ids_s[l], out=g_out[l])
            ex.mul_mat_id(l, "up", x_s, ids_s[l], out=u_out[l])
            ex.mul_mat_id(l, "down", h_s, ids_s[l], out=d_out[l])

    calls()                                                          # eager: checks every source once
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    torch.cuda.synchronize()

    def step(i):
        p = i % P
        ids_s.copy_(ids_all[p])
        x_s.copy_(xs[p])
        graph.replay()

    step_bytes = [W.step_expert_bytes(ids_np[p, :, 0][:, None, :]) for p in range(P)]
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(args.warmup, args.warmup + args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / args.steps
    nbytes = sum(step_bytes[i % P] for i in range(args.warmup, args.warmup + args.steps))
    gbs = nbytes / (ms_total * 1e6)
    # the bare graph (inputs in place) replayed R times: per-call duration
    R = max(4, args.steps // 2)
    graph.replay()
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(R):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    us_call = 1000.0 * ev0.elapsed_time(ev1) / (R * 3 * G)
    # a call's algorithmic bytes: its k expert matrices (distinct at one
    # token), the activation row(s) it reads and the rows it writes; per call,
    # averaged over a layer's two gate/up-form calls and its down call
    gate_call = k * W.matrix_bytes("gate") + 4 * W.d_model + 4 * k * W.d_ff
    down_call = k * W.matrix_bytes("down") + 4 * k * W.d_ff + 4 * k * W.d_model
    per_call = (2 * gate_call + down_call) / 3
    # per-dispatch durations: the same calls run eagerly, each recording its own
    # start/stop HIP event pair on the stream it runs on
    L = rt.lib()
    L.sabah_rt_set_kernel_timing(1)
    rt.kernel_timing("mmid", reset=True)
    for i in range(args.steps):
        ids_s.copy_(ids_all[i % P])
        calls()
    torch.cuda.synchronize()
    L.sabah_rt_set_kernel_timing(0)
    kms, kn = rt.kernel_timing("mmid")

    # parity: layer 0 of step 0's token against the oracle, all three calls
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    step(0)
    torch.cuda.synchronize()
    e_ids = ids_np[0, 0, 0]
    used = np.unique(e_ids)
    lid = np.searchsorted(used, e_ids).astype(np.int32)[None]
    worst = 0.0
    exact = True
    for role, inp, out in (("gate", x_np[0], g_out[0]), ("up", x_np[0], u_out[0]), ("down", h_np, d_out[0])):
        sub = np.stack([bank.read_expert(0, role, int(e)) for e in used])
        rows = W.d_ff if role != "down" else W.d_model
        kk = W.d_model if role != "down" else W.d_ff
        want = O.mul_mat_id(sub, inp, lid, rows, kk, W.qt_down if role == "down" else W.qt_gate)
        got = out.cpu().numpy()
        worst = max(worst, float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max()))
        exact &= bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
    parity = {"layer": 0, "calls": ["gate", "up", "down"], "max_rel": worst, "bit_identical": exact,
              "tolerance": {"max_rel": 1e-3, "cos": 0.99999}}
    cpu = None
    if not args.no_cpu:
        # the oracle's MUL_MAT_ID on this host's cores: whole tokens (the 144
        # calls of the 48 layers) over the routed experts read back from HBM
        threads = cpu_threads(args)
        layers = []
        for l in range(G):
            e_ids = ids_np[0, l, 0]
            used = np.unique(e_ids)
            lid = np.searchsorted(used, e_ids).astype(np.int32)[None]
            layers.append(({r: np.stack([bank.read_expert(l, r, int(e)) for e in used])
                            for r in ("gate", "up", "down")}, lid))
        xq, hq = x_np[0], h_np
        t1 = time.perf_counter()
        tokens = cbytes = 0
        while True:
            for sub, lid in layers:
                for role in ("gate", "up", "down"):
                    down = role == "down"
                    O.mul_mat_id(sub[role], hq if down else xq, lid, W.d_model if down else W.d_ff,
                                 W.d_ff if down else W.d_model, W.qt_down if down else W.qt_gate, n_threads=threads)
                cbytes += len(lid[0]) * W.expert_bytes()
            tokens += 1
            if time.perf_counter() - t1 >= args.cpu_seconds:
                break
        dt = time.perf_counter() - t1
        cpu = {"value": round(cbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "tok_s": round(tokens / dt, 3),
               "sample": "%d decode token(s) x %d layers x 3 MUL_MAT_ID calls (%.0f MB of routed expert bytes "
                         "read back from HBM), %.1f s" % (tokens, G, cbytes / tokens / 1e6, dt),
               "host": host_info(threads)}
    achieved = per_call / (us_call * 1e3)
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "compute": compute_note(W),
        "data": "synthetic (N(0,0.02) weights quantised on device; %s routing; seeded)" % W.routing,
        "config": {"workload": W.name, "n_layers": G, "n_experts": W.n_experts, "top_k": k, "d_model": W.d_model,
                   "d_ff": W.d_ff, "n_tokens": 1, "quant": quant_note(W), "bank_bytes": bank.total_bytes,
                   "expert_bytes_per_step": nbytes // args.steps, "calls_per_step": 3 * G,
                   "mode": "drop-in sabah_rt_mul_mat_id_v2: gate, up and down calls per layer (h synthetic), "
                           "the %d calls replayed as one HIP graph per step" % (3 * G)},
        "tok_s": round(1000.0 / ms_step, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "us_per_layer": round(1000.0 * ms_step / G, 3),
        "kernels": {"mmid": {"launches": kn, "avg_us": round(1000.0 * kms / max(kn, 1), 3)}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(W.name, ["mmid"]),
                     "kernel": "mmid", "bytes_per_launch": int(per_call), "avg_launch_us": round(us_call, 3),
                     "timing": "replayed graph, %d replays of %d calls" % (R, 3 * G)},
        "cpu_baseline": cpu, "parity": parity,
    }
    print(json.dumps(line), flush=True)
    copy_probe(args, dev)
    return 0


def copy_probe(args, dev):
    """One device-to-device copy of --copy-probe-mib MiB at the end of the run:
    a plain copy kernel of known size, to calibrate the FETCH_SIZE / WRITE_SIZE
    counters of the same run."""
    if not args.copy_probe_mib:
        return
    import torch
    n = args.copy_probe_mib << 18                                       # floats
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print("copy probe: %d MiB read, %d MiB written" % (args.copy_probe_mib, args.copy_probe_mib),
          file=sys.stderr, flush=True)


class LayerCallsGraph:
    """G calls of a one-layer workload's layer (sabah_moe_layer), each on its
    own input row with its own ids and weights, captured as one HIP graph over
    static buffers; `x` holds the G output rows after a replay."""

    def __init__(self, ex, G, d_model, k):
        import torch
        dev = ex.device
        self.ex, self.G = ex, G
        self.xin = torch.zeros(G, d_model, dtype=torch.float32, device=dev)
        self.ids = torch.zeros(G, 1, k, dtype=torch.int32, device=dev)
        self.w = torch.zeros(G, 1, k, dtype=torch.float32, device=dev)
        self.x = torch.zeros(G, d_model, dtype=torch.float32, device=dev)
        self._calls()                                  # eager: sizes the library scratch
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._calls()
        torch.cuda.synchronize(dev)

    def _calls(self):
        for g in range(self.G):
            self.ex.run_layer(0, self.xin[g:g + 1], self.ids[g], self.w[g], out=self.x[g:g + 1])

    def replay(self, x, ids, w):
        self.xin.copy_(x)
        self.ids.copy_(ids)
        self.w.copy_(w)
        self.graph.replay()
        return self.x

    def replay_static(self):
        self.graph.replay()
        return self.x


# kernel symbols of each timing kind, as the traffic summaries name them
KERNEL_SYMBOL = {"gate_up": ("k_gate_up_rounds", "k_gate_up"), "down": ("k_down_combine",), "mmid": ("k_mmid_rounds", "k_mmid"),
                 "layer": ("k_layer_decode",),
                 "grouped_gate_up": ("k_grouped_gate_up",), "grouped_down": ("k_grouped_down",)}
INT8_PEAK_TOPS = 5000.0                # MI355X dense int8 MFMA, TOP/s


def bench_batch(args, W):
    """One MoE layer over a batch of tokens (prefill / small-batch decode).

    Layers of IQ3_S, Q4_K and Q6_K with at least 2 (token, slot) pairs per
    expert run group-major (sabah_moe_prefill_layer: pairs grouped by expert,
    each expert read once, int8 MFMA); other layers, and every layer under
    --grouping off, run token-major (sabah_moe_layer).  The bank holds 8 layers of the workload's shape and
    the steps rotate through them, so a step never finds the previous step's
    experts in the 256 MB last-level cache.  `value` is the step's algorithmic
    bytes / wall time: every distinct routed expert matrix once, the shared
    expert, x in, out, and h written and read back."""
    import numpy as np
    import torch

    from sabah.runtime import rt
    from sabah.runtime.bank import DenseExpert, ExpertBank
    from sabah.runtime.executor import MoEExecutor
    from sabah.runtime.rt import row_bytes

    dev = torch.device("cuda:0")
    rt.init(0)
    n_rot = 8
    qts = {"gate": W.qt_gate, "up": W.qt_up, "down": W.qt_down}
    bank = ExpertBank(n_rot, W.n_experts, W.d_model, W.d_ff, qts, device="cuda:0")
    bank.fill_synthetic(seed=args.seed)
    shared = None
    if W.shared_d_ff:
        shared = DenseExpert(W.d_model, W.shared_d_ff, W.qt_shared, device="cuda:0")
        shared.fill_synthetic(seed=args.seed + 1)
    torch.cuda.synchronize()
    rng = np.random.default_rng(args.seed)
    P = min(args.pool, 16)
    ids_np, w_np = W.route(rng, n_layers=P)                           # [P, T, k]
    x_np = rng.standard_normal((W.n_tokens, W.d_model)).astype(np.float32)
    ids = torch.from_numpy(ids_np).to(dev)
    wts = torch.from_numpy(w_np).to(dev)
    x = torch.from_numpy(x_np).to(dev)
    out = torch.empty_like(x)
    ex = MoEExecutor(bank, max_used=W.top_k, max_tokens=W.n_tokens, shared=shared)
    grouped_types = {rt.QTYPE["IQ3_S"], rt.QTYPE["Q4_K"], rt.QTYPE["Q6_K"]}
    # group-major from 2 (token, slot) pairs per expert on average: measured at top-10 of
    # 512 (2048 / 768), the token-major layer is faster below that for every format
    grouped = (args.grouping == "auto" and W.qt_gate == W.qt_up and W.qt_gate in grouped_types
               and W.qt_down in grouped_types and W.n_tokens * W.top_k >= 2 * W.n_experts)
    T, k = W.n_tokens, W.top_k
    mmid = W.op == "mul_mat_id"
    if mmid:
        # the drop-in path: three sabah_rt_mul_mat_id_v2 calls per layer, as ggml's graph makes
        # them; h is synthetic (SwiGLU between the calls is ggml's op, outside the path)
        L0 = rt.lib()
        x3 = x.view(T, 1, W.d_model)
        h_in = torch.randn(T, k, W.d_ff, device=dev)
        g_out = torch.empty(T, k, W.d_ff, device=dev)
        u_out = torch.empty_like(g_out)
        d_out = torch.empty(T, k, W.d_model, device=dev)

        def run(l, x_, ids_, w_, out=None):
            ex.mul_mat_id(l, "gate", x3, ids_, out=g_out)
            ex.mul_mat_id(l, "up", x3, ids_, out=u_out)
            ex.mul_mat_id(l, "down", h_in, ids_, out=d_out)
            return d_out

        def run_token_major(l, x_, ids_, w_, out=None):
            rt.check(L0.sabah_rt_set_mmid_grouping(1), "grouping mode")
            try:
                return run(l, x_, ids_, w_)
            finally:
                rt.check(L0.sabah_rt_set_mmid_grouping(0), "grouping mode")
    else:
        run = ex.run_prefill_layer if grouped else ex.run_layer
        run_token_major = ex.run_layer
    U = [len(np.unique(ids_np[p])) for p in range(P)]
    if mmid:
        act = 4 * T * W.d_model * 2 + 3 * 4 * T * k * W.d_ff + 4 * T * k * W.d_model
    else:
        act = 4 * T * W.d_model * 2 + 2 * 4 * T * k * W.d_ff
    step_bytes = [U[p] * W.expert_bytes() + W.shared_bytes() + act for p in range(P)]

    def step(i, fn):
        fn(i % n_rot, x, ids[i % P], wts[i % P], out=out)

    def timed(fn, steps):
        for i in range(args.warmup):
            step(i, fn)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for i in range(args.warmup, args.warmup + steps):
            step(i, fn)
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1)

    steps = max(1, args.steps)
    ms = timed(run, steps)
    nbytes = sum(step_bytes[i % P] for i in range(args.warmup, args.warmup + steps))
    gbs = nbytes / (ms * 1e6)
    # bit-identity of the grouped layer with the token-major one, and its per-kernel times
    parity = None
    ms_token_major = None
    if grouped:
        outs = []
        for fn in (run, run_token_major):
            r = fn(0, x, ids[0], wts[0])
            outs.append(torch.cat([g_out.flatten(), u_out.flatten(), r.flatten()]) if mmid else r.clone())
        torch.cuda.synchronize()
        parity = {"grouped_equals_token_major": bool(torch.equal(outs[0], outs[1]))}
        ms_token_major = timed(run_token_major, max(1, steps // 4)) / max(1, steps // 4)
    elif not mmid and not args.no_cpu:
        parity = batch_parity(W, bank, shared, ex, ids_np, w_np, x_np, dev)
    L = rt.lib()
    L.sabah_rt_set_kernel_timing(1)
    for kind in rt.KERNEL_KINDS:
        rt.kernel_timing(kind, reset=True)
    timed(run, steps)
    L.sabah_rt_set_kernel_timing(0)
    kernels = {}
    for kind in rt.KERNEL_KINDS:
        kms, n = rt.kernel_timing(kind)
        if n:
            kernels[kind] = {"launches": n, "avg_us": round(1000.0 * kms / n, 3), "total_ms": kms}
    dom = max(kernels, key=lambda q: kernels[q]["total_ms"])
    u_mean = float(np.mean(U))
    pairs = T * k
    D, F, Fs = W.d_model, W.d_ff, W.shared_d_ff
    sh_gu = 2 * Fs * row_bytes(W.qt_shared, D) if Fs else 0
    sh_down = D * row_bytes(W.qt_shared, Fs) if Fs else 0
    # algorithmic bytes per step of each kernel kind: every distinct routed expert matrix once,
    # the activations each launch reads and writes.  Token-major: gate_up covers the routed and
    # (when present) the shared expert's gate/up launch, mmid the shared down launch.
    step_kind_bytes = {
        "grouped_gate_up": u_mean * (W.matrix_bytes("gate") + W.matrix_bytes("up")) + 4 * pairs * F,
        "grouped_down": u_mean * W.matrix_bytes("down") + 4 * pairs * F,
        "gate_up": (u_mean * (W.matrix_bytes("gate") + W.matrix_bytes("up")) + sh_gu
                    + 4 * T * D * (2 if Fs else 1) + 4 * pairs * F + 4 * T * Fs),
        "down": u_mean * W.matrix_bytes("down") + 4 * pairs * F + 4 * T * (2 * D + k),
        "mmid": (u_mean * W.expert_bytes() + act) if mmid else sh_down + 4 * T * Fs + 4 * T * D,
    }
    launches_per_step = kernels[dom]["launches"] / (args.warmup + steps)
    per_launch = step_kind_bytes[dom] / launches_per_step
    achieved = per_launch / (kernels[dom]["avg_us"] * 1e3)
    flops = 2.0 * pairs * 3 * W.d_model * W.d_ff
    us_step = 1000.0 * ms / steps
    line = {
        "metric": "MUL_MAT_ID expert GB/s (% HBM peak), one MoE layer over a token batch, 1 GPU",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8",
        "compute": ("int8 MFMA (v_mfma_i32_16x16x32_i8) on weights decoded to int8 x q8_K activations, "
                    "fp32 scales and accumulation" if grouped else
                    "int8 x int8 -> int32 dot products, fp32 scales and accumulation"),
        "data": "synthetic (N(0,0.02) weights quantised on device; seeded routing)",
        "config": {"workload": W.name, "n_experts": W.n_experts, "top_k": k, "d_model": W.d_model, "d_ff": W.d_ff,
                   "n_tokens": T, "quant": "%d/%d/%d" % (W.qt_gate, W.qt_up, W.qt_down),
                   "shared_d_ff": W.shared_d_ff,
                   "mode": ("drop-in sabah_rt_mul_mat_id_v2: gate, up, down (grouped by expert)" if mmid
                            else "group-major (sabah_moe_prefill_layer)" if grouped
                            else "token-major (sabah_moe_layer)")},
        "us_per_layer": round(us_step, 2), "tok_s": round(T / (us_step * 1e-6), 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "unique_experts": {"mean": u_mean, "min": min(U), "max": max(U)},
        "int8_tops": round(flops / (us_step * 1e-6) / 1e12, 2),
        "mfma_frac": round(flops / (us_step * 1e-6) / 1e12 / INT8_PEAK_TOPS, 5) if grouped else None,
        "token_major_us_per_layer": round(1000.0 * ms_token_major, 2) if ms_token_major else None,
        "kernels": {q: {"launches": v["launches"], "avg_us": v["avg_us"]} for q, v in kernels.items()},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(W.name, [dom]), "kernel": dom,
                     "bytes_per_launch": int(per_launch), "avg_launch_us": kernels[dom]["avg_us"]},
        "cpu_baseline": None if args.no_cpu else cpu_batch_baseline(args, W, bank, ids_np, w_np, x_np, mmid),
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    copy_probe(args, dev)
    return 0


def batch_parity(W, bank, shared, ex, ids_np, w_np, x_np, dev, n=8):
    """The token-major layer on the GPU against the oracle's layer (ggml's CPU
    MUL_MAT_ID path with the shared expert), on the first n tokens of the
    first routing, with the routed and shared experts read back from HBM."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    e_ids = ids_np[0, :n]
    used = np.unique(e_ids)
    remap = {int(e): i for i, e in enumerate(used)}
    sub = {r: np.stack([bank.read_expert(0, r, int(e)) for e in used]) for r in ("gate", "up", "down")}
    lid = np.vectorize(remap.get)(e_ids).astype(np.int32)
    sh = None
    if shared is not None:
        sh = (shared.read("gate"), shared.read("up"), shared.read("down"), (shared.qt,) * 3,
              None if shared.gate_inp is None else shared.gate_inp.cpu().numpy())
    x = np.ascontiguousarray(x_np[:n])
    got = ex.run_layer(0, torch.from_numpy(x).to(dev), torch.from_numpy(np.ascontiguousarray(e_ids)).to(dev),
                       torch.from_numpy(np.ascontiguousarray(w_np[0, :n])).to(dev)).cpu().numpy()
    ref = O.moe_layer(sub["gate"], sub["up"], sub["down"], (W.qt_gate, W.qt_up, W.qt_down), x, lid,
                      w_np[0, :n], shared=sh)
    d = (got.astype(np.float64) - ref).ravel()
    r = ref.astype(np.float64).ravel()
    return {"tokens": n, "max_rel": float(np.abs(d).max() / np.abs(r).max()),
            "cos": float((got.ravel() @ r) / np.sqrt((got.ravel() @ got.ravel()) * (r @ r))),
            "tolerance": {"max_rel": 1e-3, "cos": 0.99999}}


def cpu_batch_baseline(args, W, bank, ids_np, w_np, x_np, mmid=False):
    """The oracle's layer (token-major, as ggml's CPU MUL_MAT_ID) on the host's
    cores, over a sample of the batch's tokens whose routed experts are read
    back from HBM; for the drop-in workload, the oracle's three MUL_MAT_ID calls."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = cpu_threads(args)
    n = 8
    e_ids = ids_np[0, :n]
    used = np.unique(e_ids)
    remap = {int(e): i for i, e in enumerate(used)}
    sub = {r: np.stack([bank.read_expert(0, r, int(e)) for e in used]) for r in ("gate", "up", "down")}
    lid = np.vectorize(remap.get)(e_ids).astype(np.int32)
    qts = (W.qt_gate, W.qt_up, W.qt_down)
    t0 = time.perf_counter()
    tokens = 0
    h_np = np.random.default_rng(1).standard_normal((n, W.top_k, W.d_ff)).astype(np.float32)
    while True:
        if mmid:
            for role, xx, rows, kk, qt in (("gate", x_np[:n, None], W.d_ff, W.d_model, W.qt_gate),
                                           ("up", x_np[:n, None], W.d_ff, W.d_model, W.qt_up),
                                           ("down", h_np, W.d_model, W.d_ff, W.qt_down)):
                O.mul_mat_id(sub[role], xx, lid, rows, kk, qt, n_threads=threads)
        else:
            O.moe_layer(sub["gate"], sub["up"], sub["down"], qts, x_np[:n], lid, w_np[0, :n], n_threads=threads)
        tokens += n
        if time.perf_counter() - t0 >= args.cpu_seconds / 3:
            break
    dt = time.perf_counter() - t0
    return {"value": round(tokens * W.top_k * W.expert_bytes() / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "tok_s": round(tokens / dt, 2),
            "sample": "%d tokens of the batch, their %d routed experts read back from HBM, %.1f s "
                      "(token-major: each (token, slot) reads its expert)" % (tokens, len(used), dt),
            "host": host_info(threads)}


# the committed profiles' name of each workload's summaries
PROFILE_PREFIX = {"iq3s_48x512_top10": "decode_kernels_iq3s_48x512_top10",
                  "q8_0_e8_top2": "decode_kernels_q8_0_e8_top2",
                  "q4k_e128_top8": "decode_kernels_q4k_e128_top8",
                  "iq3s_prefill_t512": "prefill_layer_iq3s_t512_e512_top10",
                  "iq3s_mmid_t512": "mul_mat_id_iq3s_t512_e512_top10",
                  "iq3s_mmid_48x512_top10": "mul_mat_id_iq3s_48x512_top10_decode",
                  "mixed_t32_q4k_q6k_shared": "mixed_layer_q4k_q6k_shared_t32"}


def measured_traffic(workload, kinds):
    """HBM bytes per launch from the committed FETCH_SIZE / WRITE_SIZE counter
    runs (calibrated against a plain copy), summed over the kernel kinds
    `kinds` (a layer's launches) and averaged over the kernels of one kind (a
    kind's routed and shared-expert launches); None if one was not measured."""
    if not kinds or workload not in PROFILE_PREFIX:
        return None
    path = os.path.join(ROOT, "profiles", "%s_traffic.json" % PROFILE_PREFIX[workload])
    try:
        with open(path) as f:
            kernels = json.load(f)["kernels"]
    except (OSError, KeyError, ValueError):
        return None
    total = 0
    for kind in kinds:
        hit = [v["traffic_bytes"] for name, v in kernels.items()
               if any(name == sym or name.startswith(sym + "<") for sym in KERNEL_SYMBOL[kind])]
        if not hit:
            return None
        total += sum(hit) / len(hit)                # a kind's launches of one step, on average
    return int(total)


def cpu_threads(args):
    """Threads of the CPU baseline: --cpu-threads, else OMP_NUM_THREADS (the
    CPU share a shared host grants this process), else every CPU in this
    process's affinity mask."""
    if args.cpu_threads:
        return args.cpu_threads
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def host_info(threads):
    """What the CPU baseline ran on: model, logical CPUs, this process's
    affinity, NUMA nodes, and the thread count used."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nodes = len([d for d in os.listdir("/sys/devices/system/node") if d.startswith("node") and d[4:].isdigit()])
    except OSError:
        nodes = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "numa_nodes": nodes, "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"), "threads_used": threads}


def cpu_baseline(args, W, bank, ex, ids_np, w_np, x_np, dev):
    """The oracle (C restatement of ggml's CPU MUL_MAT_ID path) on this host's
    cores, over the routed experts of one decode token read back from HBM, and
    a parity check of the same layer on the GPU."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    threads = cpu_threads(args)
    p = 0
    layers = []
    for l in range(W.n_layers):
        e_ids = ids_np[p, l, 0]
        used = np.unique(e_ids)
        remap = {int(e): i for i, e in enumerate(used)}
        sub = {r: np.stack([bank.read_expert(l, r, int(e)) for e in used]) for r in ("gate", "up", "down")}
        layers.append((sub, np.vectorize(remap.get)(e_ids).astype(np.int32)[None], w_np[p, l]))
    qts = (W.qt_gate, W.qt_up, W.qt_down)
    # parity: layer 0 on the GPU vs the oracle, same x / ids / weights
    x0 = x_np[p]
    got = ex.run_layer(0, torch.from_numpy(x0).to(dev), torch.from_numpy(ids_np[p, 0]).to(dev),
                       torch.from_numpy(w_np[p, 0]).to(dev)).cpu().numpy()
    sub, lid, lw = layers[0]
    ref = O.moe_layer(sub["gate"], sub["up"], sub["down"], qts, x0, lid, lw, n_threads=threads)
    d = (got.astype(np.float64) - ref).ravel()
    r = ref.astype(np.float64).ravel()
    parity = {"layer": 0, "max_rel": float(np.abs(d).max() / np.abs(r).max()),
              "cos": float((got.ravel() @ r) / np.sqrt((got.ravel() @ got.ravel()) * (r @ r))),
              "tolerance": {"max_rel": 1e-3, "cos": 0.99999}}
    # timing: whole tokens (48 chained layers) until the target CPU time is
    # reached, with every thread of the host's share and with one thread
    def time_tokens(nt, seconds):
        t0 = time.perf_counter()
        tokens = nbytes = 0
        while True:
            x = x0.copy()
            for sub, lid, lw in layers:
                x = x + O.moe_layer(sub["gate"], sub["up"], sub["down"], qts, x, lid, lw, n_threads=nt)
                nbytes += len(np.unique(lid)) * W.expert_bytes()
            tokens += 1
            if time.perf_counter() - t0 >= seconds:
                break
        return tokens, nbytes, time.perf_counter() - t0

    tokens, nbytes, dt = time_tokens(threads, args.cpu_seconds)
    tok1, nb1, dt1 = time_tokens(1, args.cpu_seconds / 3)
    cpu = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
           "tok_s": round(tokens / dt, 3),
           "sample": "%d decode token(s) x %d layers (%.0f MB of routed expert bytes read back from HBM), %.1f s"
                     % (tokens, W.n_layers, nbytes / tokens / 1e6, dt),
           "one_thread": {"value": round(nb1 / dt1 / 1e9, 3), "unit": "GB/s", "tok_s": round(tok1 / dt1, 3),
                          "sample": "%d decode token(s), %.1f s" % (tok1, dt1)},
           "host": host_info(threads)}
    return cpu, parity


if __name__ == "__main__":
    sys.exit(main())
