"""The in-library sampled self-check of sabah_rt_mul_mat_id_v2 (the
reference's sb_selfcheck, sabah_rt.cu:3435-3492, enabled there by
SABAH_LLAMA_SELFCHECK): after each call, k sampled (token, slot) output rows
are recomputed on the host in float64 by the library's own decoders and
activation quantisers (host_decode.h, never the oracle) and compared by
relative L2 error.

Correct calls pass every sample, across formats, both x forms and the grouped
path.  The three mapping errors the reference's sentinel builds plant
(sabah_rt.cu:76-86: the neighbouring expert, the next slot's input row, the
next token's input row) are planted in the host recomputation (the kernels
stay untouched) and every one is caught.  The status file and the exit trace
are checked through the bridge's C caller in a fresh process."""
from __future__ import annotations

import ctypes
import json
import os
import subprocess

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_1, Q6_K, IQ3_S = 8, 12, 7, 14, 21
DEV = torch.device("cuda:0")


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.fixture
def selfcheck(hip_rt):
    lib = hip_rt.lib()

    def set_check(k, tol=1e-5, sentinel=0):
        hip_rt.check(lib.sabah_rt_set_selfcheck(k, tol, sentinel), "set selfcheck")

    yield set_check
    set_check(0)


def diag(hip_rt):
    return hip_rt.diag()


def call_v2(hip_rt, orc, rng, qt, k, rows, E, n_ids, n_tokens, x_rows):
    raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    ids = np.stack([rng.choice(E, n_ids, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    x = rng.standard_normal((n_tokens, x_rows, k)).astype(np.float32)
    bank, xt, it = T(raw), T(x), T(ids)
    out = torch.zeros(n_tokens, n_ids, rows, dtype=torch.float32, device=DEV)
    rb = raw.shape[-1]
    rc = hip_rt.lib().sabah_rt_mul_mat_id_v2(
        ctypes.c_void_p(bank.data_ptr()), rows * rb, rb, vp(xt), xt.stride(1) * 4, x_rows, xt.stride(0) * 4,
        vp(it), 4, it.stride(0) * 4, n_ids, n_tokens, vp(out), out.stride(1) * 4, out.stride(0) * 4, rows, k, E, qt,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), None)
    hip_rt.check(rc, "v2")
    torch.cuda.synchronize()
    return out


# (qt, k, rows, E, n_ids, n_tokens, x_rows): token-major calls of several
# formats, the down form (one input row per slot), and 64 tokens of a 16-expert
# IQ3_S bank (grouped by expert)
CALLS = [(Q8_0, 1024, 96, 8, 2, 3, 1), (Q4_K, 2048, 64, 16, 4, 2, 1), (Q5_1, 1024, 64, 8, 3, 2, 3),
         (Q6_K, 768, 128, 8, 4, 2, 4), (IQ3_S, 2048, 64, 16, 8, 64, 1)]


@pytest.mark.parametrize("qt,k,rows,E,n_ids,n_tokens,x_rows", CALLS)
def test_selfcheck_passes_every_sample_of_correct_calls(hip_rt, orc, selfcheck, qt, k, rows, E, n_ids, n_tokens,
                                                         x_rows):
    rng = np.random.default_rng(qt + k + rows)
    selfcheck(4)
    before = diag(hip_rt)
    call_v2(hip_rt, orc, rng, qt, k, rows, E, n_ids, n_tokens, x_rows)
    call_v2(hip_rt, orc, rng, qt, k, rows, E, n_ids, n_tokens, x_rows)
    after = diag(hip_rt)
    assert after["verify_fail"] - before["verify_fail"] == 0, hip_rt.snapshot()
    assert after["verify_ok"] - before["verify_ok"] == 2 * min(4, n_ids * n_tokens)
    snap = hip_rt.snapshot()
    assert snap["selfcheck_k"] == 4 and snap["selfcheck_max_rel"] < 1e-5 and snap["sentinel"] == 0


@pytest.mark.parametrize("sentinel,x_rows,n_tokens", [(1, 1, 2), (2, 4, 2), (3, 1, 3)])
def test_selfcheck_catches_each_planted_mapping_error(hip_rt, orc, selfcheck, sentinel, x_rows, n_tokens):
    """1: every sample recomputed with the neighbouring expert; 2: with the
    next slot's input row (the down form, one row per slot); 3: with the next
    token's input row.  Every sample fails, by far more than the tolerance."""
    rng = np.random.default_rng(40 + sentinel)
    selfcheck(6, 1e-5, sentinel)
    call_v2(hip_rt, orc, rng, Q8_0, 1024, 64, 8, 4, n_tokens, x_rows)
    d = diag(hip_rt)
    assert d["verify_ok"] == 0 and d["verify_fail"] == 6
    assert hip_rt.snapshot()["selfcheck_max_rel"] > 0.1


def test_selfcheck_settings_are_validated(hip_rt):
    lib = hip_rt.lib()
    assert lib.sabah_rt_set_selfcheck(-1, 1e-5, 0) == -1
    assert lib.sabah_rt_set_selfcheck(2, 0.0, 0) == -1
    assert lib.sabah_rt_set_selfcheck(2, 1e-5, 4) == -1
    assert lib.sabah_rt_set_selfcheck(0, 1e-5, 0) == 0


def test_status_file_and_exit_trace_from_the_bridge(tmp_path, orc):
    """SABAH_LLAMA_SELFCHECK=3, SABAH_LLAMA_STATUS_FILE and SABAH_LLAMA_TRACE
    in the environment of the bridge's C caller (a fresh process): the status
    file holds the snapshot after its last call, with every self-check sample
    passed, and the exit report names the same counters."""
    from test_bridge_caller import CALLER, LIB, write_case
    rng = np.random.default_rng(77)
    write_case(str(tmp_path), orc, rng, Q4_K, 2048, 256, 16, 4, 2, 1, 16, False)
    status = tmp_path / "status.json"
    env = dict(os.environ, SABAH_RT_LIB=LIB, SABAH_LLAMA_SELFCHECK="3", SABAH_LLAMA_STATUS_FILE=str(status),
               SABAH_LLAMA_TRACE="1")
    p = subprocess.run([CALLER, str(tmp_path)], capture_output=True, text=True, timeout=120, env=env)
    assert p.returncode == 0, p.stdout + p.stderr
    snap = json.loads(status.read_text())
    assert snap["calls"] == 3 and snap["selfcheck_k"] == 3
    assert snap["selfcheck_ok"] == 9 and snap["selfcheck_fail"] == 0
    assert "SABAH_SNAPSHOT" in p.stderr and "verify_ok=9 verify_fail=0" in p.stderr
