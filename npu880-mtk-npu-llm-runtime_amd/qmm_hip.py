"""ctypes binding of libqmm_hip.so (the C ABI in include/qmm_hip.h).

Host-side mirror of the reference engine's matmul interface
(src/v182_r22_breakthrough_engine.c): :class:`MatrixTask` is SdotMatrixTask
(E:888-899) with fp32 dst/residual and device pointers, and
:meth:`Context.gemm_multi_dispatch` is sdot_gemm_multi_dispatch
(E:4188-4262). Device memory is managed through the library's own
allocator, so nothing here depends on another GPU runtime.

The library must be built (``make -C npu880-mtk-npu-llm-runtime_amd``);
loading raises :class:`QmmUnavailable` otherwise — there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqmm_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "qmm_hip.h")

QMM_OK, QMM_EINVAL, QMM_ETYPE, QMM_ESHAPE, QMM_EHIP, QMM_ENOMEM, QMM_EALIGN = range(7)
TYPE_F32, TYPE_F16 = 0, 1
TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 8, 12, 13, 14
TYPE_NAMES = {TYPE_F32: "F32", TYPE_F16: "F16", TYPE_Q8_0: "Q8_0", TYPE_Q4_K: "Q4_K", TYPE_Q5_K: "Q5_K",
              TYPE_Q6_K: "Q6_K"}
BLOCK_BYTES = {TYPE_F32: 4, TYPE_F16: 2, TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}
BLOCK_VALUES = {TYPE_F32: 1, TYPE_F16: 1, TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256, TYPE_Q6_K: 256}

_p = C.c_void_p


class QmmUnavailable(RuntimeError):
    """libqmm_hip.so is missing: build it; there is no fallback path."""


class QmmError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"qmm status {status}: {message}")
        self.status = status


class LmScanParams(C.Structure):
    """qmm_lm_scan_params (the chunked vocabulary scan, E:11107-11262)."""
    _fields_ = [("chunk_rows", C.c_int), ("thresholds", C.POINTER(C.c_float)), ("n_thresholds", C.c_int),
                ("first_checkpoint", C.c_int), ("prune_margin", C.c_float), ("chunk_begin", C.c_int),
                ("chunk_end", C.c_int), ("resume", C.c_int)]


class _Task(C.Structure):
    _fields_ = [
        ("w_base", _p), ("type", C.c_uint32), ("row_bytes", C.c_size_t),
        ("dst", _p), ("dst_stride", C.c_size_t), ("residual", _p),
        ("res_stride", C.c_size_t), ("rows", C.c_int), ("cols", C.c_int),
        ("start_row", C.c_int),
    ]


# (name, restype, argtypes) of every entry point in include/qmm_hip.h
_SIGNATURES = [
    ("qmm_init", C.c_int, [C.c_int, C.POINTER(_p)]),
    ("qmm_destroy", C.c_int, [_p]),
    ("qmm_set_stream", C.c_int, [_p, _p]),
    ("qmm_get_stream", _p, [_p]),
    ("qmm_synchronize", C.c_int, [_p]),
    ("qmm_reserve", C.c_int, [_p, C.c_int, C.c_int]),
    ("qmm_status_string", C.c_char_p, [C.c_int]),
    ("qmm_last_error", C.c_char_p, [_p]),
    ("qmm_device_info", C.c_int, [_p, C.POINTER(C.c_int), C.POINTER(C.c_size_t), C.c_char_p, C.c_size_t]),
    ("qmm_row_bytes", C.c_size_t, [C.c_uint32, C.c_int64]),
    ("qmm_q8k_bytes", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8k_d_offset", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8k_bsum_offset", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8k_tile_offset", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8k_h_offset", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8k_bh_offset", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8_0_bytes", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_q8_0_d_offset", C.c_size_t, [C.c_int, C.c_int]),
    ("qmm_malloc", C.c_int, [_p, C.c_size_t, C.POINTER(_p)]),
    ("qmm_free", C.c_int, [_p, _p]),
    ("qmm_memcpy_h2d", C.c_int, [_p, _p, _p, C.c_size_t]),
    ("qmm_memcpy_d2h", C.c_int, [_p, _p, _p, C.c_size_t]),
    ("qmm_memcpy_d2d", C.c_int, [_p, _p, _p, C.c_size_t]),
    ("qmm_weight_upload", C.c_int, [_p, _p, C.c_uint32, C.c_int64, C.c_int64, C.POINTER(_p)]),
    ("qmm_quantize_q8k", C.c_int, [_p, _p, C.c_int, C.c_int, _p]),
    ("qmm_quantize_q8_0", C.c_int, [_p, _p, C.c_int, C.c_int, _p]),
    ("qmm_swiglu_q8k", C.c_int, [_p, _p, _p, C.c_int, C.c_int, _p, _p]),
    ("qmm_rmsnorm_q8k", C.c_int, [_p, _p, _p, C.c_int, C.c_int, _p, _p]),
    ("qmm_ffn_block", C.c_int, [_p, _p, _p, C.c_int, _p, _p, _p, _p]),
    ("qmm_ffn_block_rmsnorm", C.c_int, [_p, _p, _p, C.c_int, _p, _p, _p, _p]),
    ("qmm_gguf_open", C.c_int, [C.c_char_p, _p]),
    ("qmm_gguf_close", C.c_int, [_p]),
    ("qmm_gguf_header", C.c_int, [_p, _p, _p, _p, _p]),
    ("qmm_gguf_tensor_at", C.c_int, [_p, C.c_int, _p]),
    ("qmm_gguf_find_tensor", C.c_int, [_p, C.c_char_p, _p]),
    ("qmm_gguf_data", _p, [_p, _p]),
    ("qmm_gguf_upload", C.c_int, [_p, _p, C.c_char_p, _p, _p]),
    ("qmm_lm_head_argmax", C.c_int, [_p, _p, _p, C.c_int, C.c_int, _p, C.c_uint32, C.c_int, C.c_uint32,
                                     _p, _p, _p]),
    ("qmm_eval_rows_argmax", C.c_int, [_p, _p, _p, C.c_int, C.c_int, _p, C.c_int64, C.c_uint32, _p, C.c_int,
                                       _p, _p, _p]),
    ("qmm_lm_head_scan", C.c_int, [_p, _p, _p, C.c_int, C.c_int, _p, C.c_uint32, C.c_int,
                                   C.POINTER(LmScanParams), _p, C.c_int, _p, _p, _p, _p]),
    ("qmm_lm_head_scan_rmsnorm", C.c_int, [_p, _p, _p, C.c_int, C.c_int, _p, C.c_uint32, C.c_int,
                                           C.POINTER(LmScanParams), _p, C.c_int, _p, _p, _p, _p]),
    ("qmm_dequantize_f16", C.c_int, [_p, _p, C.c_uint32, C.c_int64, C.c_int64, _p]),
    ("qmm_gemm_multi_dispatch", C.c_int, [_p, _p, C.c_int, C.c_int, C.POINTER(_Task), C.c_int]),
    ("qmm_gemm_multi_dispatch_prequantized", C.c_int,
     [_p, _p, _p, C.c_int, C.c_int, C.POINTER(_Task), C.c_int]),
    ("qmm_gemm_multi_dispatch_noalloc", C.c_int, [_p, _p, C.c_int, C.c_int, C.POINTER(_Task), C.c_int]),
    ("qmm_gemm_multi_dispatch_rmsnorm", C.c_int, [_p, _p, _p, C.c_int, C.c_int, C.POINTER(_Task), C.c_int]),
    ("qmm_noalloc_scratch_bytes", C.c_size_t, []),
    ("qmm_graph_begin", C.c_int, [_p]),
    ("qmm_graph_end", C.c_int, [_p, C.POINTER(_p)]),
    ("qmm_graph_launch", C.c_int, [_p, _p]),
    ("qmm_graph_destroy", C.c_int, [_p, _p]),
    ("qmm_stream_read", C.c_int, [_p, _p, C.c_size_t, C.c_int, C.c_int, _p]),
    ("qmm_timer_begin", C.c_int, [_p]),
    ("qmm_timer_end", C.c_int, [_p, C.POINTER(C.c_float)]),
]

_LIB = None


def load_library(path: str = LIB_PATH):
    """Load libqmm_hip.so and declare every entry point's signature."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise QmmUnavailable(f"{path} not built: run make -C {HERE}")
    lib = C.CDLL(path)
    for name, res, args in _SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def row_bytes(type_id: int, cols: int) -> int:
    """ggml_row_bytes (E:3940-3942), computed by the library."""
    return int(load_library().qmm_row_bytes(type_id, cols))


def q8k_tile(qs: np.ndarray) -> np.ndarray:
    """Codes [M][K] -> the tiles section of a Q8_K buffer (flat int8): for
    token tile t, block j and 64-value chunk h, 1 KB whose 16-B slot 16c + n
    holds token 16t + n's codes at block offsets 64h + 8c..+7, then
    64h + 32 + 8c..+7 (slots of tokens past M are zero here)."""
    M, K = qs.shape
    T, nb = (M + 15) // 16, K // 256
    p = np.zeros((T * 16, K), np.int8)
    p[:M] = qs
    # axes (t, n, j, h, half, c, byte) -> (t, j, h, c, n, half, byte)
    return np.ascontiguousarray(p.reshape(T, 16, nb, 4, 2, 4, 8).transpose(0, 2, 3, 5, 1, 4, 6)).reshape(-1)


def q8k_untile(t: np.ndarray, M: int, K: int) -> np.ndarray:
    """Inverse of q8k_tile: the first M tokens' codes in [M][K] order."""
    T, nb = (M + 15) // 16, K // 256
    return np.ascontiguousarray(t.reshape(T, nb, 4, 4, 16, 2, 8).transpose(0, 4, 1, 2, 5, 3, 6)).reshape(T * 16, K)[:M]


def q8k_bh(qs: np.ndarray) -> np.ndarray:
    """Codes [M][K] -> the bh section of a Q8_K buffer (fp16 bits, flat
    uint16): for token tile t and block j, 256 values whose 4-value slot
    16c + n holds token 16t + n's sums of 16-value groups 4c..4c+3."""
    M, K = qs.shape
    T, nb = (M + 15) // 16, K // 256
    p = np.zeros((T * 16, K), np.int32)
    p[:M] = qs
    s16 = p.reshape(T, 16, nb, 4, 4, 16).sum(axis=5)  # (t, n, j, c, g%4)
    return np.ascontiguousarray(s16.transpose(0, 2, 3, 1, 4)).astype(np.float16).view(np.uint16).reshape(-1)


def q8k_bytes(M: int, K: int) -> int:
    return int(load_library().qmm_q8k_bytes(M, K))


def q8_0_bytes(M: int, K: int) -> int:
    return int(load_library().qmm_q8_0_bytes(M, K))


class DevBuf:
    """A device allocation owned by a Context."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes

    def __int__(self):
        return self.ptr

    def offset(self, nbytes: int) -> int:
        return self.ptr + nbytes

    def free(self):
        if self.ptr and self.ctx._h:
            self.ctx._call("qmm_free", self.ctx._h, _p(self.ptr))
        self.ptr = 0


@dataclass
class MatrixTask:
    """SdotMatrixTask (E:888-899): fp32 dst/residual, device pointers."""
    w: object            # DevBuf or int device address of packed rows
    type: int
    rows: int
    cols: int
    dst: object          # DevBuf or int: fp32 [M][dst_stride]
    dst_stride: int = 0  # defaults to rows
    residual: object = None
    res_stride: int = 0
    start_row: int = 0   # written back by the dispatcher


def _addr(x) -> int:
    if x is None:
        return 0
    return int(x)


class GgufTensor(C.Structure):
    """qmm_gguf_tensor (GgufTensorInfo, E:168-177)."""
    _fields_ = [("name", C.c_char * 128), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("type", C.c_uint32), ("rel_offset", C.c_uint64), ("abs_offset", C.c_uint64),
                ("n_elems", C.c_uint64), ("byte_size", C.c_uint64)]

    def as_dict(self):
        return dict(name=self.name.decode("utf-8", "replace"), n_dims=self.n_dims, dims=list(self.dims),
                    type=self.type, rel_offset=self.rel_offset, abs_offset=self.abs_offset,
                    n_elems=self.n_elems, byte_size=self.byte_size)


class Gguf:
    """A GGUF file, memory-mapped by the library (host only; no GPU needed)."""

    def __init__(self, path: str):
        self.lib = load_library()
        h = _p()
        rc = self.lib.qmm_gguf_open(os.fsencode(path), C.byref(h))
        if rc != 0:
            raise QmmError(rc, f"qmm_gguf_open({path}): {self.lib.qmm_status_string(rc).decode()}")
        self._h = h

    def close(self):
        if self._h:
            self.lib.qmm_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def header(self):
        v, al, do, n = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_int()
        self.lib.qmm_gguf_header(self._h, C.byref(v), C.byref(al), C.byref(do), C.byref(n))
        return dict(version=v.value, alignment=al.value, data_offset=do.value, n_tensors=n.value)

    def tensors(self):
        out = []
        for i in range(self.header()["n_tensors"]):
            t = GgufTensor()
            self.lib.qmm_gguf_tensor_at(self._h, i, C.byref(t))
            out.append(t.as_dict())
        return out

    def find(self, name: str):
        t = GgufTensor()
        rc = self.lib.qmm_gguf_find_tensor(self._h, name.encode(), C.byref(t))
        return t.as_dict() if rc == 0 else None

    def data(self, name: str) -> np.ndarray:
        t = GgufTensor()
        rc = self.lib.qmm_gguf_find_tensor(self._h, name.encode(), C.byref(t))
        if rc != 0:
            raise QmmError(rc, f"no tensor {name}")
        p = self.lib.qmm_gguf_data(self._h, C.byref(t))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(t.byte_size,)).copy()

    def upload(self, ctx: "Context", name: str):
        p = _p()
        t = GgufTensor()
        ctx._call("qmm_gguf_upload", ctx._h, self._h, name.encode(), C.byref(p), C.byref(t))
        return p.value, t.as_dict()


class Context:
    """qmm_context: one device, one stream, the dispatcher's activation buffers."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _p()
        rc = self.lib.qmm_init(device, C.byref(h))
        if rc != QMM_OK:
            raise QmmError(rc, f"qmm_init(device={device}) failed: "
                               f"{self.lib.qmm_status_string(rc).decode()}")
        self._h = h
        self._bufs: list[DevBuf] = []

    # -- plumbing --------------------------------------------------------
    def _call(self, name, *args):
        rc = getattr(self.lib, name)(*args)
        if rc != QMM_OK:
            msg = self.lib.qmm_last_error(self._h).decode()
            raise QmmError(rc, f"{name}: {msg or self.lib.qmm_status_string(rc).decode()}")
        return rc

    def status_of(self, name, *args) -> int:
        """Call an entry point and return its raw status (for error tests)."""
        return int(getattr(self.lib, name)(self._h, *args))

    def last_error(self) -> str:
        return self.lib.qmm_last_error(self._h).decode()

    def close(self):
        if getattr(self, "_h", None):
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            self.lib.qmm_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def device_info(self):
        cu = C.c_int()
        hbm = C.c_size_t()
        arch = C.create_string_buffer(64)
        self._call("qmm_device_info", self._h, C.byref(cu), C.byref(hbm), arch, 64)
        return {"cu_count": cu.value, "hbm_bytes": hbm.value, "arch": arch.value.decode()}

    def sync(self):
        self._call("qmm_synchronize", self._h)

    def reserve(self, M: int, K: int):
        self._call("qmm_reserve", self._h, M, K)

    # -- memory ------------------------------------------------------------
    def malloc(self, nbytes: int) -> DevBuf:
        p = _p()
        self._call("qmm_malloc", self._h, max(int(nbytes), 1), C.byref(p))
        b = DevBuf(self, p.value, int(nbytes))
        self._bufs.append(b)
        return b

    def free(self, b: DevBuf):
        if b in self._bufs:
            self._bufs.remove(b)
        b.free()

    def upload(self, a: np.ndarray) -> DevBuf:
        a = np.ascontiguousarray(a)
        b = self.malloc(a.nbytes)
        self.h2d(b, a)
        return b

    def h2d(self, dst, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        self._call("qmm_memcpy_h2d", self._h, _p(_addr(dst) + offset), _p(a.ctypes.data), a.nbytes)

    def d2h(self, src, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        self._call("qmm_memcpy_d2h", self._h, _p(out.ctypes.data), _p(_addr(src) + offset), out.nbytes)
        return out

    def d2d(self, dst, src, nbytes: int):
        self._call("qmm_memcpy_d2d", self._h, _p(_addr(dst)), _p(_addr(src)), nbytes)

    def weight_upload(self, blocks: np.ndarray, type_id: int, rows: int, cols: int) -> DevBuf:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        p = _p()
        self._call("qmm_weight_upload", self._h, _p(blocks.ctypes.data), type_id, rows, cols, C.byref(p))
        b = DevBuf(self, p.value, rows * row_bytes(type_id, cols))
        self._bufs.append(b)
        return b

    # -- compute -------------------------------------------------------------
    def quantize_q8k(self, x, M: int, K: int, out):
        self._call("qmm_quantize_q8k", self._h, _p(_addr(x)), M, K, _p(_addr(out)))

    def quantize_q8_0(self, x, M: int, K: int, out):
        self._call("qmm_quantize_q8_0", self._h, _p(_addr(x)), M, K, _p(_addr(out)))

    def rmsnorm_q8k(self, x, gamma, M: int, K: int, y_out, out):
        self._call("qmm_rmsnorm_q8k", self._h, _p(_addr(x)), _p(_addr(gamma)), M, K,
                   _p(_addr(y_out)), _p(_addr(out)))

    def lm_head_argmax(self, q8k, q80, M: int, K: int, w_rows, type_id: int, rows: int, row_base: int,
                       logits_out, best_val, best_id):
        self._call("qmm_lm_head_argmax", self._h, _p(_addr(q8k)), _p(_addr(q80)), M, K, _p(_addr(w_rows)),
                   type_id, rows, row_base, _p(_addr(logits_out)), _p(_addr(best_val)), _p(_addr(best_id)))

    def eval_rows_argmax(self, q8k, q80, M: int, K: int, w_tensor, tensor_rows: int, type_id: int, row_ids,
                         n_ids: int, vals_out, best_val, best_id):
        self._call("qmm_eval_rows_argmax", self._h, _p(_addr(q8k)), _p(_addr(q80)), M, K, _p(_addr(w_tensor)),
                   tensor_rows, type_id, _p(_addr(row_ids)), n_ids, _p(_addr(vals_out)), _p(_addr(best_val)),
                   _p(_addr(best_id)))

    def lm_head_scan(self, q8k, q80, M: int, K: int, w_lm, type_id: int, vocab_rows: int, chunk_rows: int,
                     thresholds=None, first_checkpoint: int = 0, prune_margin: float = 1e-3, pre_ids=None,
                     n_pre: int = 0, draft_ids=None, best_val=None, best_id=None, scan_state=None,
                     chunk_begin: int = 0, chunk_end: int = 0, resume: bool = False):
        """qmm_lm_head_scan: the chunked vocabulary scan with early exit and pruning; chunks
        [chunk_begin, chunk_end) of it (chunk_end 0: to the end), a new scan or (resume) the
        continuation of the one best_val / best_id / scan_state hold."""
        thr = None if thresholds is None else (C.c_float * len(thresholds))(*[float(t) for t in thresholds])
        prm = LmScanParams(chunk_rows, thr if thr is not None else None, 0 if thr is None else len(thresholds),
                           first_checkpoint, prune_margin, chunk_begin, chunk_end, 1 if resume else 0)
        self._call("qmm_lm_head_scan", self._h, _p(_addr(q8k)), _p(_addr(q80)), M, K, _p(_addr(w_lm)), type_id,
                   vocab_rows, C.byref(prm), _p(_addr(pre_ids)), n_pre, _p(_addr(draft_ids)), _p(_addr(best_val)),
                   _p(_addr(best_id)), _p(_addr(scan_state)))

    def lm_head_scan_rmsnorm(self, x, gamma, M: int, K: int, w_lm, type_id: int, vocab_rows: int, chunk_rows: int,
                             thresholds=None, first_checkpoint: int = 0, prune_margin: float = 1e-3, pre_ids=None,
                             n_pre: int = 0, draft_ids=None, best_val=None, best_id=None, scan_state=None,
                             chunk_begin: int = 0, chunk_end: int = 0, resume: bool = False):
        """qmm_lm_head_scan_rmsnorm: the final RMSNorm of x with gamma, then the chunked vocabulary scan."""
        thr = None if thresholds is None else (C.c_float * len(thresholds))(*[float(t) for t in thresholds])
        prm = LmScanParams(chunk_rows, thr if thr is not None else None, 0 if thr is None else len(thresholds),
                           first_checkpoint, prune_margin, chunk_begin, chunk_end, 1 if resume else 0)
        self._call("qmm_lm_head_scan_rmsnorm", self._h, _p(_addr(x)), _p(_addr(gamma)), M, K, _p(_addr(w_lm)),
                   type_id, vocab_rows, C.byref(prm), _p(_addr(pre_ids)), n_pre, _p(_addr(draft_ids)),
                   _p(_addr(best_val)), _p(_addr(best_id)), _p(_addr(scan_state)))

    def swiglu_q8k(self, gate, up, M: int, N: int, h_out, out):
        self._call("qmm_swiglu_q8k", self._h, _p(_addr(gate)), _p(_addr(up)), M, N,
                   _p(_addr(h_out)), _p(_addr(out)))

    def ffn_block(self, x, q8k, K: int, gate: MatrixTask, up: MatrixTask, down: MatrixTask, h_out=None):
        """qmm_ffn_block: give exactly one of x (fp32 [K]) and q8k."""
        gu = self._tasks(1, K, [gate, up])
        dn = self._tasks(1, down.cols, [down])
        self._call("qmm_ffn_block", self._h, _p(_addr(x)), _p(_addr(q8k)), K, C.byref(gu[0]), C.byref(gu[1]),
                   C.byref(dn[0]), _p(_addr(h_out)))

    def ffn_block_rmsnorm(self, x, gamma, K: int, gate: MatrixTask, up: MatrixTask, down: MatrixTask,
                          h_out=None):
        """qmm_ffn_block_rmsnorm: the block on x (fp32 [K]) after its RMSNorm with gamma."""
        gu = self._tasks(1, K, [gate, up])
        dn = self._tasks(1, down.cols, [down])
        self._call("qmm_ffn_block_rmsnorm", self._h, _p(_addr(x)), _p(_addr(gamma)), K, C.byref(gu[0]),
                   C.byref(gu[1]), C.byref(dn[0]), _p(_addr(h_out)))

    def dequantize_f16(self, w, type_id: int, rows: int, cols: int, dst):
        self._call("qmm_dequantize_f16", self._h, _p(_addr(w)), type_id, rows, cols, _p(_addr(dst)))

    @staticmethod
    def _tasks(M: int, K: int, tasks: Sequence[MatrixTask]):
        arr = (_Task * len(tasks))()
        for i, t in enumerate(tasks):
            arr[i] = _Task(_addr(t.w), t.type, int(load_library().qmm_row_bytes(t.type, t.cols)),
                           _addr(t.dst), t.dst_stride or t.rows, _addr(t.residual),
                           t.res_stride or t.rows, t.rows, t.cols, 0)
        return arr

    def gemm_multi_dispatch(self, x, M: int, K: int, tasks: Sequence[MatrixTask]):
        arr = self._tasks(M, K, tasks)
        self._call("qmm_gemm_multi_dispatch", self._h, _p(_addr(x)), M, K, arr, len(tasks))
        for t, a in zip(tasks, arr):
            t.start_row = a.start_row

    def gemm_multi_dispatch_rmsnorm(self, x, gamma, M: int, K: int, tasks: Sequence[MatrixTask]):
        """qmm_gemm_multi_dispatch_rmsnorm: RMSNorm of x with gamma, then the tasks."""
        arr = self._tasks(M, K, tasks)
        self._call("qmm_gemm_multi_dispatch_rmsnorm", self._h, _p(_addr(x)), _p(_addr(gamma)), M, K, arr,
                   len(tasks))
        for t, a in zip(tasks, arr):
            t.start_row = a.start_row

    def gemm_multi_dispatch_noalloc(self, x, M: int, K: int, tasks: Sequence[MatrixTask]):
        """qmm_gemm_multi_dispatch_noalloc: the dispatcher on the device scratch."""
        arr = self._tasks(M, K, tasks)
        self._call("qmm_gemm_multi_dispatch_noalloc", self._h, _p(_addr(x)), M, K, arr, len(tasks))
        for t, a in zip(tasks, arr):
            t.start_row = a.start_row

    def gemm_multi_dispatch_prequantized(self, q8k, q80, M: int, K: int,
                                         tasks: Sequence[MatrixTask]):
        arr = self._tasks(M, K, tasks)
        self._call("qmm_gemm_multi_dispatch_prequantized", self._h, _p(_addr(q8k)),
                   _p(_addr(q80)), M, K, arr, len(tasks))
        for t, a in zip(tasks, arr):
            t.start_row = a.start_row

    # -- graphs / timing -----------------------------------------------------
    def graph_begin(self):
        self._call("qmm_graph_begin", self._h)

    def graph_end(self) -> int:
        g = _p()
        self._call("qmm_graph_end", self._h, C.byref(g))
        return g.value

    def graph_launch(self, g: int):
        self._call("qmm_graph_launch", self._h, _p(g))

    def stream_read(self, src, nbytes: int, workgroups: int, loads_per_wave: int, sink):
        self._call("qmm_stream_read", self._h, _p(_addr(src)), nbytes, workgroups, loads_per_wave, _p(_addr(sink)))

    def graph_destroy(self, g: int):
        self._call("qmm_graph_destroy", self._h, _p(g))

    def timer_begin(self):
        self._call("qmm_timer_begin", self._h)

    def timer_end(self) -> float:
        ms = C.c_float()
        self._call("qmm_timer_end", self._h, C.byref(ms))
        return ms.value

    # -- numpy conveniences (tests, smoke) -----------------------------------
    def read_q8k(self, buf, M: int, K: int):
        """Device Q8_K buffer -> (d[M,K/256] f32, qs[M,K] i8, bsum32[M,K/32] i32)."""
        lib = self.lib
        qs = self.d2h(buf, np.int8, (M, K))
        d = self.d2h(buf, np.float32, (M, K // 256), offset=int(lib.qmm_q8k_d_offset(M, K)))
        bs = self.d2h(buf, np.int32, (M, K // 32), offset=int(lib.qmm_q8k_bsum_offset(M, K)))
        return d, qs, bs

    def read_q8k_tiles(self, buf, M: int, K: int) -> np.ndarray:
        """The tiles section of a device Q8_K buffer, put back in [M][K] order."""
        T = (M + 15) // 16
        t = self.d2h(buf, np.int8, (T * 16 * K,), offset=int(self.lib.qmm_q8k_tile_offset(M, K)))
        return q8k_untile(t, M, K)

    def read_q8k_bh(self, buf, M: int, K: int) -> np.ndarray:
        """The bh section of a device Q8_K buffer as fp32 sums [M][K/16]."""
        T, nb = (M + 15) // 16, K // 256
        v = self.d2h(buf, np.float16, (T, nb, 4, 16, 4), offset=int(self.lib.qmm_q8k_bh_offset(M, K)))
        return np.ascontiguousarray(v.transpose(0, 3, 1, 2, 4)).reshape(T * 16, K // 16)[:M].astype(np.float32)

    def write_q8k(self, buf, d, qs, bs, x16=None):
        """All sections of a device Q8_K buffer; x16 = the fp16 values (bits
        [M][K]) for the h section, zeros if None."""
        M, K = qs.shape
        lib = self.lib
        self.h2d(buf, np.ascontiguousarray(qs, np.int8))
        self.h2d(buf, np.ascontiguousarray(d, np.float32), offset=int(lib.qmm_q8k_d_offset(M, K)))
        self.h2d(buf, np.ascontiguousarray(bs, np.int32), offset=int(lib.qmm_q8k_bsum_offset(M, K)))
        self.h2d(buf, q8k_tile(qs), offset=int(lib.qmm_q8k_tile_offset(M, K)))
        h = np.zeros((M, K), np.uint16) if x16 is None else np.ascontiguousarray(x16, np.uint16).reshape(M, K)
        self.h2d(buf, h, offset=int(lib.qmm_q8k_h_offset(M, K)))
        self.h2d(buf, q8k_bh(qs), offset=int(lib.qmm_q8k_bh_offset(M, K)))

    def write_q80(self, buf, d, qs):
        """Both sections of a device Q8_0 buffer from its codes and scales."""
        M, K = qs.shape
        self.h2d(buf, np.ascontiguousarray(qs, np.int8))
        self.h2d(buf, np.ascontiguousarray(d, np.float32), offset=int(self.lib.qmm_q8_0_d_offset(M, K)))

    def read_q8k_h(self, buf, M: int, K: int) -> np.ndarray:
        """The h section (fp16 bits [M][K]) of a device Q8_K buffer."""
        return self.d2h(buf, np.uint16, (M, K), offset=int(self.lib.qmm_q8k_h_offset(M, K)))

    def read_q8_0(self, buf, M: int, K: int):
        qs = self.d2h(buf, np.int8, (M, K))
        d = self.d2h(buf, np.float32, (M, K // 32), offset=int(self.lib.qmm_q8_0_d_offset(M, K)))
        return d, qs

    def gemm(self, type_id: int, w, N: int, K: int, x: np.ndarray,
             residual: Optional[np.ndarray] = None) -> np.ndarray:
        """One task through the dispatcher: y[M, N] = x[M, K] . W^T (+ residual)."""
        x = np.ascontiguousarray(x, np.float32)
        if x.ndim == 1:
            x = x[None, :]
        M = x.shape[0]
        xb = self.upload(x)
        yb = self.malloc(M * N * 4)
        rb = self.upload(np.ascontiguousarray(residual, np.float32)) if residual is not None else None
        try:
            self.gemm_multi_dispatch(xb, M, K, [MatrixTask(w, type_id, N, K, yb, N, rb, N)])
            self.sync()
            return self.d2h(yb, np.float32, (M, N))
        finally:
            for b in (xb, yb, rb):
                if b is not None:
                    self.free(b)
