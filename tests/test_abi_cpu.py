"""The C ABI library (libqmm_hip.so) loads and exports every entry point
declared in include/qmm_hip.h; host-only helpers and argument checks that
need no device. No kernels run here."""
import ctypes as C
import re

import numpy as np
import pytest

import qmm_hip


def _declared_functions():
    src = open(qmm_hip.HEADER_PATH).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[a-z_][a-z0-9_ ]*?\**\s*\b(qmm_[a-z0-9_]+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = _declared_functions()
    for must in ("qmm_init", "qmm_gemm_multi_dispatch", "qmm_gemm_multi_dispatch_prequantized",
                 "qmm_quantize_q8k", "qmm_quantize_q8_0", "qmm_dequantize_f16", "qmm_swiglu_q8k",
                 "qmm_weight_upload", "qmm_row_bytes", "qmm_lm_head_scan", "qmm_eval_rows_argmax",
                 "qmm_q8k_h_offset"):
        assert must in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    lib = qmm_hip.load_library()
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    bound = {s[0] for s in qmm_hip._SIGNATURES}
    assert set(_declared_functions()) == bound


def test_row_bytes_and_layout_sizes():
    lib = qmm_hip.load_library()
    assert lib.qmm_row_bytes(12, 2560) == 1440
    assert lib.qmm_row_bytes(13, 2560) == 1760
    assert lib.qmm_row_bytes(14, 2560) == 2100
    assert lib.qmm_row_bytes(8, 2560) == 2720
    assert lib.qmm_row_bytes(14, 9728) == 7980
    assert lib.qmm_row_bytes(12, 300) == 0  # not a multiple of 256
    assert lib.qmm_row_bytes(0, 2560) == 10240  # F32 rows (E:366)
    assert lib.qmm_row_bytes(1, 2560) == 5120   # F16 rows (E:367)
    assert lib.qmm_row_bytes(1, 40) == 0        # F32 / F16 K must be a multiple of 32
    assert lib.qmm_row_bytes(2, 2560) == 0      # Q4_0: not on this path
    M, K = 3, 2560
    d_off, bs_off, total = lib.qmm_q8k_d_offset(M, K), lib.qmm_q8k_bsum_offset(M, K), lib.qmm_q8k_bytes(M, K)
    assert d_off >= M * K and d_off % 256 == 0
    assert bs_off >= d_off + 4 * M * K // 256 and bs_off % 256 == 0
    tile_off = lib.qmm_q8k_tile_offset(M, K)
    assert tile_off >= bs_off + 4 * M * K // 32 and tile_off % 256 == 0
    h_off = lib.qmm_q8k_h_offset(M, K)
    assert h_off >= tile_off + 16 * K and h_off % 256 == 0  # one 16-token tile for M = 3
    bh_off = lib.qmm_q8k_bh_offset(M, K)
    assert bh_off >= h_off + 2 * M * K and bh_off % 256 == 0
    assert total >= bh_off + 16 * K // 8  # fp16 sums of 16 codes for one 16-token tile
    assert lib.qmm_q8_0_d_offset(M, K) >= M * K and lib.qmm_q8_0_bytes(M, K) >= M * K + 4 * M * K // 32
    assert lib.qmm_q8k_bytes(0, K) == 0


@pytest.mark.parametrize("M,K", [(1, 256), (16, 512), (37, 768)])
def test_q8k_tiles_order(M, K):
    """The tiles section's order, from its definition: slot 16c + n of chunk
    h of block j of token tile t holds token 16t + n's codes at block
    offsets 64h + 8c .. +7, then 64h + 32 + 8c .. +7."""
    rng = np.random.default_rng(M + K)
    qs = rng.integers(-127, 128, (M, K)).astype(np.int8)
    t = qmm_hip.q8k_tile(qs)
    assert t.size == (M + 15) // 16 * 16 * K
    assert np.array_equal(qmm_hip.q8k_untile(t, M, K), qs)
    nb = K // 256
    for m in range(M):
        for j in range(nb):
            for h in range(4):
                for c in range(4):
                    slot = t[(((m // 16) * nb + j) * 4 + h) * 1024 + 16 * (16 * c + m % 16):][:16]
                    base = 256 * j + 64 * h + 8 * c
                    assert np.array_equal(slot[:8], qs[m, base:base + 8])
                    assert np.array_equal(slot[8:], qs[m, base + 32:base + 40])


def test_status_strings_and_null_context():
    lib = qmm_hip.load_library()
    assert lib.qmm_status_string(0) == b"ok"
    assert lib.qmm_status_string(2) == b"unsupported ggml type"
    assert lib.qmm_destroy(None) == qmm_hip.QMM_EINVAL
    assert lib.qmm_synchronize(None) == qmm_hip.QMM_EINVAL
    assert lib.qmm_gemm_multi_dispatch(None, None, 1, 256, None, 0) == qmm_hip.QMM_EINVAL
    assert lib.qmm_quantize_q8k(None, None, 1, 256, None) == qmm_hip.QMM_EINVAL
    assert lib.qmm_init(0, None) == qmm_hip.QMM_EINVAL


def test_init_without_device_reports_hip_error():
    lib = qmm_hip.load_library()
    h = C.c_void_p()
    rc = lib.qmm_init(0, C.byref(h))
    if rc == qmm_hip.QMM_OK:  # a GPU is present: nothing to check here
        lib.qmm_destroy(h)
        pytest.skip("GPU present")
    assert rc == qmm_hip.QMM_EHIP and not h.value
