"""The llama.cpp bridge's side of the boundary, from C: tests/bridge/bridge_caller
drives sabah-hip-bridge.h (the header the patched ggml HIP build includes) the
way ggml-cuda.cu does in the reference's bridge
(patches/llama.cpp/0001-sabah-native-mul-mat-id.patch:138-206):
dlopen + dlsym, an mmap'd expert tensor registered by its host address, v2
called with ggml's nb[] strides and ids as a view into a wider argsort result,
and a 20-argument caller.  Its outputs are compared with the oracle."""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest

from helpers import assert_bits_equal, assert_parity, random_blocks

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(ROOT, "tests", "bridge", "bridge_caller")
LIB = os.path.join(ROOT, "sabah-moe-accelerator_amd", "csrc", "libsabah_rt.so")

Q8_0, Q4_K, Q6_K, IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, Q2_0 = 8, 12, 14, 18, 20, 21, 22, 23, 42
Q5_1, Q5_K = 7, 13
BIT_EXACT = (Q8_0, IQ3_S, IQ3_XXS, IQ4_NL, IQ4_XS, IQ2_S, Q2_0, Q5_1)


def run_caller(arg, lib=LIB, timeout=120):
    if not os.path.exists(CALLER):
        raise FileNotFoundError("%s is not built: run __graft_entry__.build()" % CALLER)
    env = dict(os.environ, SABAH_RT_LIB=lib)
    p = subprocess.run([CALLER, arg], capture_output=True, text=True, timeout=timeout, env=env)
    lines = [l for l in p.stdout.splitlines() if l.startswith("{")]
    assert lines, "no JSON from the caller (rc %d): %s %s" % (p.returncode, p.stdout, p.stderr)
    return p.returncode, json.loads(lines[-1])


# ---- the loader, on the CPU: every failure is a message, never a crash ----
def test_loader_reports_a_missing_library():
    rc, r = run_caller("--load-only", lib="/nonexistent/libsabah_rt.so")
    assert rc == 0 and r["ready"] is False
    assert "could not be loaded" in r["error"] and "/nonexistent/libsabah_rt.so" in r["error"]


def test_loader_reports_a_library_without_the_abi():
    import ctypes.util
    libm = ctypes.util.find_library("m")
    rc, r = run_caller("--load-only", lib=libm)
    assert rc == 0 and r["ready"] is False and "missing the native MUL_MAT_ID ABI" in r["error"]


def test_loader_resolves_the_abi_and_reports_init_failure_without_a_gpu():
    from conftest import gpu_available
    if gpu_available():
        pytest.skip("a GPU is visible: init succeeds")
    rc, r = run_caller("--load-only")
    assert rc == 0 and r["ready"] is False and r["error"].startswith("Sabah runtime init failed: ")


# ---- the calls, on the GPU ----
def write_case(d, orc, rng, qt, k, rows, E, n_ids, n_tokens, x_rows, ids_ld, on_device):
    if qt in (IQ3_XXS, IQ2_S):
        raw = random_blocks(rng, qt, E * rows, k).reshape(E, rows, -1)
    else:
        raw = orc.quantize_weights(qt, (rng.standard_normal((E, rows, k)) * 0.02).astype(np.float32))
    # ids as llama.cpp's argsort of every expert's score, of which the first n_ids are used
    full = np.stack([rng.permutation(E)[:ids_ld] for _ in range(n_tokens)]).astype(np.int32)
    x = rng.standard_normal((n_tokens, x_rows, k)).astype(np.float32)
    raw.tofile(os.path.join(d, "weights.bin"))
    x.tofile(os.path.join(d, "x.f32"))
    full.tofile(os.path.join(d, "ids.i32"))
    with open(os.path.join(d, "meta.txt"), "w") as f:
        f.write("%d %d %d %d %d %d %d %d %d\n" % (qt, k, rows, E, n_ids, n_tokens, x_rows, ids_ld, int(on_device)))
    return raw, x, np.ascontiguousarray(full[:, :n_ids])


# (qt, k, rows, E, n_ids, n_tokens, x_rows, ids_ld, src0 on device)
CASES = [
    (IQ3_S, 2048, 768, 64, 10, 1, 1, 64, False),     # one decode token, gate/up form
    (IQ3_S, 768, 2048, 64, 10, 3, 10, 64, False),    # down form: one activation row per slot
    (IQ3_S, 2048, 512, 32, 8, 64, 1, 8, False),      # a prompt batch, dense ids: grouped by expert
    (Q4_K, 2048, 512, 32, 8, 5, 1, 32, True),        # experts offloaded by ggml: a device pointer
    (Q6_K, 512, 2048, 32, 8, 2, 8, 8, False),
    (Q8_0, 1024, 256, 8, 2, 4, 1, 8, False),
    (IQ4_XS, 1024, 256, 16, 4, 2, 4, 16, False),
    (IQ2_S, 1024, 256, 16, 4, 2, 1, 16, True),
    (Q2_0, 960, 512, 16, 4, 3, 1, 16, False),        # 64-element blocks, a partial last unit
    (Q5_1, 2048, 256, 16, 4, 2, 1, 16, False),
    (Q5_K, 768, 512, 16, 4, 2, 4, 16, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("qt,k,rows,E,n_ids,n_tokens,x_rows,ids_ld,on_device", CASES)
def test_bridge_caller_matches_the_oracle(tmp_path, orc, qt, k, rows, E, n_ids, n_tokens, x_rows, ids_ld, on_device):
    from conftest import gpu_available
    if not gpu_available():
        pytest.skip("no GPU visible")
    rng = np.random.default_rng(qt * 100 + k + rows + n_tokens)
    raw, x, ids = write_case(str(tmp_path), orc, rng, qt, k, rows, E, n_ids, n_tokens, x_rows, ids_ld, on_device)
    print("bridge case qt=%d k=%d rows=%d E=%d n_ids=%d T=%d x_rows=%d ids_ld=%d device=%d"
          % (qt, k, rows, E, n_ids, n_tokens, x_rows, ids_ld, on_device), flush=True)
    rc, r = run_caller(str(tmp_path))
    assert rc == 0 and r["ok"], r
    want = orc.mul_mat_id(raw, x, ids, rows, k, qt)
    got21, got20, again = (np.fromfile(str(tmp_path / n), np.float32).reshape(want.shape)
                           for n in ("dst21.f32", "dst20.f32", "dst21_again.f32"))
    assert_parity(got21, want, "bridge qt=%d" % qt)
    if qt in BIT_EXACT:
        assert_bits_equal(got21, want, "bridge qt=%d against the oracle" % qt)
    assert_bits_equal(got20, got21, "20-argument caller")
    assert_bits_equal(again, got21, "repeated op")
    # one upload, on the first call, of a host expert tensor; none of a device one
    assert r["banks_after_first"] == r["banks"] == (0 if on_device else 1)
    assert r["uploaded_bytes"] == (0 if on_device else raw.nbytes)
    assert r["resident_bytes"] == (0 if on_device else raw.nbytes)
    assert r["hits"] == 3 * n_tokens * n_ids and r["misses"] == 0
    assert r["bad_layout_rc"] == -1 and "unsupported MUL_MAT_ID layout" in r["bad_layout_error"]


# ---- the patch for ggml's HIP build ----
PATCH_DIR = os.path.join(ROOT, "sabah-moe-accelerator_amd", "integration", "llama.cpp")


def test_committed_patch_is_generated_from_the_bridge_header():
    import sys
    r = subprocess.run([sys.executable, os.path.join(PATCH_DIR, "make_patch.py"), "--check"])
    assert r.returncode == 0, "0001-sabah-hip-mul-mat-id.patch is stale: rerun make_patch.py"


def test_patch_routes_exactly_the_types_the_library_decodes():
    import re
    from sabah.runtime import rt
    text = open(os.path.join(PATCH_DIR, "0001-sabah-hip-mul-mat-id.patch")).read()
    body = text[text.index("static bool ggml_cuda_sabah_type"):]
    body = body[:body.index("default:")]
    routed = set(re.findall(r"GGML_TYPE_(\w+)", body))
    assert routed == {"Q8_0", "Q5_1", "Q4_K", "Q5_K", "Q6_K", "IQ3_XXS", "IQ4_NL", "IQ3_S", "IQ2_S", "IQ4_XS",
                      "Q2_0"}
    assert routed <= set(rt.QTYPE)
    assert all(rt.row_bytes(rt.QTYPE[n], 256) > 0 for n in routed)
