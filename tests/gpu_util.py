"""Helpers for the GPU parity tests."""
import numpy as np

# stated tolerance for fp32 dot / GEMM outputs: max|y - ref| / max|ref|
TOL = 1e-3


def norm_err(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    return float(np.abs(y - ref).max() / (scale if scale > 0 else 1.0))


def check_outputs(y, ref, what=""):
    """Within the stated tolerance, and — by construction of the kernels —
    equal to the reference's fp32 sums bit for bit."""
    y = np.ascontiguousarray(y, np.float32)
    ref = np.ascontiguousarray(ref, np.float32)
    assert y.shape == ref.shape, (what, y.shape, ref.shape)
    err = norm_err(y, ref)
    assert err <= TOL, f"{what}: normalized max error {err:.3e} > {TOL}"
    nbad = int(np.count_nonzero(y.view(np.uint32) != ref.view(np.uint32)))
    assert nbad == 0, f"{what}: {nbad} of {y.size} outputs differ in bits (norm err {err:.3e})"


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
