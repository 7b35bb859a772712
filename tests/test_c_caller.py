"""The C ABI from plain C: tests/abi_caller.c is compiled with gcc -std=gnu11
(warnings as errors) against include/qmm_hip.h and linked to libqmm_hip.so,
as the engine's own C code would bind it. On the CPU it checks the host-only
entry points (row sizes against their closed forms, status strings,
activation buffer sizes and offsets against the ctypes binding); on the GPU
it runs one dispatch from C and compares the output with the oracle bit for
bit."""
import os
import subprocess

import numpy as np
import pytest

import qmm_hip
import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "npu880-mtk-npu-llm-runtime_amd")


@pytest.fixture(scope="module")
def caller(tmp_path_factory):
    lib = os.path.join(PKG, "libqmm_hip.so")
    if not os.path.exists(lib):
        pytest.fail("libqmm_hip.so is not built (python __graft_entry__.py build)")
    exe = str(tmp_path_factory.mktemp("c_caller") / "abi_caller")
    cmd = ["gcc", "-std=gnu11", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic",
           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "abi_caller.c"),
           "-L", PKG, "-lqmm_hip", f"-Wl,-rpath,{PKG}", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"C caller does not compile against include/qmm_hip.h:\n{r.stderr}"
    return exe


def _kv(out):
    return dict(ln.split(" ", 1) for ln in out.strip().splitlines())


def test_c_caller_host_entry_points(caller):
    r = subprocess.run([caller, "sizes"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    kv = _kv(r.stdout)
    # values per block and bytes per block (F32 / F16 rows: K a multiple of 32 on this path)
    block = {0: (32, 128), 1: (32, 64), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
    for t in (0, 1, 8, 12, 13, 14, 3):
        for k in (256, 2560, 4096, 9728, 100):
            want = 0
            if t in block and k % block[t][0] == 0:
                want = k // block[t][0] * block[t][1]
            assert int(kv[f"row_bytes.{t}.{k}"]) == want, (t, k)
    assert kv["status.0"] != kv["status.1"]
    lib = qmm_hip.load_library()
    for s in range(8):
        assert kv[f"status.{s}"] == lib.qmm_status_string(s).decode()
    for M, K in ((1, 2560), (8, 2560), (64, 9728), (512, 4096)):
        for f in ("q8k_bytes", "q8k_d_offset", "q8k_bsum_offset", "q8k_tile_offset", "q8k_h_offset",
                  "q8k_bh_offset", "q8_0_bytes", "q8_0_d_offset"):
            assert int(kv[f"{f}.{M}.{K}"]) == int(getattr(lib, f"qmm_{f}")(M, K)), (f, M, K)
        # the codes section is [M][K] int8 at 0; every later section 256-B aligned
        assert int(kv[f"q8k_d_offset.{M}.{K}"]) >= M * K
        for f in ("q8k_d_offset", "q8k_bsum_offset", "q8k_tile_offset", "q8k_h_offset", "q8k_bh_offset"):
            assert int(kv[f"{f}.{M}.{K}"]) % 256 == 0
    assert int(kv["noalloc_scratch_bytes"]) == 32 << 20


@pytest.mark.gpu
@pytest.mark.parametrize("type_id,N,K,M", [(qmm_hip.TYPE_Q4_K, 9728, 2560, 1), (qmm_hip.TYPE_Q6_K, 512, 2560, 8)])
def test_c_caller_dispatch_matches_oracle(caller, oracle, tmp_path, type_id, N, K, M):
    print(f"[gpu] C caller dispatch {qmm_hip.TYPE_NAMES[type_id]} {N}x{K} M={M}", flush=True)
    w = synth.weights(type_id, N, K, seed=600 + M)
    x = synth.activations(M, K, seed=610 + M)
    w.tofile(tmp_path / "w.bin")
    x.astype(np.float32).tofile(tmp_path / "x.bin")
    r = subprocess.run([caller, "dispatch", str(tmp_path), str(type_id), str(N), str(K), str(M)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"C caller failed: {r.stderr}"
    assert "dispatch ok start_row 0" in r.stdout
    y = np.fromfile(tmp_path / "y.bin", np.float32).reshape(M, N)
    ref = oracle.gemm(type_id, w, N, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), \
        f"max |d| / max |ref| = {np.abs(y - ref).max() / np.abs(ref).max():.3e}"
