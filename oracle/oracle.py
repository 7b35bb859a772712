"""numpy/ctypes front end of the CPU checker — TEST INFRASTRUCTURE ONLY.

Two libraries are wrapped:

* ``liboracle.so`` — the C restatement of the reference's scalar path
  (``qmm_oracle.c``), built by ``oracle/Makefile`` with gcc.
* ``_ref/libref.so`` — the reference engine's own translation unit
  (src/v182_r22_breakthrough_engine.c) compiled in place through
  ``ref_harness.c``; present only where it was built from the reference
  checkout.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this module. Q8_K activations are returned as the
triple ``(d[M, K/256] f32, qs[M, K] i8, bsum32[M, K/32] i32)``; Q8_0 as
``(d[M, K/32] f32, qs[M, K] i8)``.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

TYPE_F32, TYPE_F16 = 0, 1
TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 8, 12, 13, 14
BLOCK_BYTES = {TYPE_F32: 4, TYPE_F16: 2, TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}
BLOCK_VALUES = {TYPE_F32: 1, TYPE_F16: 1, TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256, TYPE_Q6_K: 256}

_p = C.c_void_p


def _ptr(a: np.ndarray) -> C.c_void_p:
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return C.c_void_p(a.ctypes.data)


def row_bytes(type_id: int, cols: int) -> int:
    """compute_ggml_bytes (E:364-374); 0 for an unsupported type."""
    if type_id not in BLOCK_BYTES:
        return 0
    return (cols // BLOCK_VALUES[type_id]) * BLOCK_BYTES[type_id]


class _MatrixTask(C.Structure):
    _fields_ = [
        ("w_base", _p), ("type", C.c_uint32), ("row_bytes", C.c_size_t),
        ("dst", _p), ("dst_stride", C.c_size_t), ("residual", _p),
        ("res_stride", C.c_size_t), ("rows", C.c_int), ("cols", C.c_int),
        ("start_row", C.c_int),
    ]


class _Script(C.Structure):
    """qo_script: the LM head's extended-script state (E:9690-9733, E:11185-11241)."""
    _fields_ = [("is_cyr", _p), ("is_cjk", _p), ("cyr_rows", _p), ("n_cyr", C.c_int), ("cjk_rows", _p),
                ("n_cjk", C.c_int), ("has_cyr", C.c_int), ("has_cjk", C.c_int), ("require_full", C.c_int),
                ("batch1", C.c_int)]


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.qo_fp16_to_f32.restype = C.c_float
        L.qo_fp16_to_f32.argtypes = [C.c_uint16]
        L.qo_f32_to_fp16.restype = C.c_uint16
        L.qo_f32_to_fp16.argtypes = [C.c_float]
        L.qo_f32_to_fp16_array.argtypes = [_p, _p, C.c_size_t]
        L.qo_fp16_to_f32_array.argtypes = [_p, _p, C.c_size_t]
        L.qo_row_bytes.restype = C.c_uint64
        L.qo_row_bytes.argtypes = [C.c_uint32, C.c_uint64]
        L.qo_get_scale_min_k4.argtypes = [C.c_int, _p, _p, _p]
        L.qo_dequant_rows.restype = C.c_int
        L.qo_dequant_rows.argtypes = [C.c_uint32, _p, C.c_int64, C.c_int64, _p]
        L.qo_quantize_row_q8k_f16.argtypes = [_p, C.c_int, _p, _p, _p]
        L.qo_quantize_row_q8_0_f16.argtypes = [_p, C.c_int, _p, _p]
        L.qo_quantize_q8k_f32.argtypes = [_p, C.c_int, C.c_int, _p, _p, _p]
        L.qo_quantize_q8_0_f32.argtypes = [_p, C.c_int, C.c_int, _p, _p]
        L.qo_dot_row.restype = C.c_float
        L.qo_dot_row.argtypes = [C.c_uint32, _p, C.c_int, _p, _p, _p]
        L.qo_dot_row_float.restype = C.c_float
        L.qo_dot_row_float.argtypes = [C.c_uint32, _p, C.c_int, _p]
        L.qo_block_partials.restype = C.c_int
        L.qo_block_partials.argtypes = [C.c_uint32, _p, C.c_int, _p, _p, _p, _p]
        L.qo_gemm_multi.restype = C.c_int
        L.qo_gemm_multi.argtypes = [_p, C.c_int, C.c_int, C.POINTER(_MatrixTask), C.c_int]
        L.qo_gemm_multi_prequantized.restype = C.c_int
        L.qo_gemm_multi_prequantized.argtypes = [_p, _p, _p, _p, _p, _p, C.c_int, C.c_int,
                                                 C.POINTER(_MatrixTask), C.c_int]
        L.qo_swiglu_q8k.argtypes = [_p, _p, C.c_int, C.c_int, _p, _p, _p, _p]
        L.qo_rmsnorm_q8k_f16.argtypes = [_p, _p, C.c_int, C.c_int, _p, _p, _p, _p]
        L.qo_chunk_argmax.argtypes = [_p, C.c_int, C.c_int, C.c_size_t, C.c_int, _p, C.c_uint32, _p, _p]
        L.qo_lm_head_scan.restype = C.c_int
        L.qo_lm_head_scan.argtypes = [C.c_uint32, _p, C.c_int, C.c_int, C.c_int, _p, _p, _p, C.c_int, _p, C.c_int,
                                      C.c_int, C.c_float, _p, C.c_int, _p, _p, _p, _p, _p]
        L.qo_lm_head_scan_script.restype = C.c_int
        L.qo_lm_head_scan_script.argtypes = [C.c_uint32, _p, C.c_int, C.c_int, C.c_int, _p, _p, _p, C.c_int, _p,
                                             C.c_int, C.c_float, _p, C.c_int, _p, C.POINTER(_Script), _p, _p, _p, _p]

    # fp16 ----------------------------------------------------------------
    def f32_to_fp16(self, x) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.qo_f32_to_fp16_array(_ptr(x), _ptr(out), x.size)
        return out

    def fp16_to_f32(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.qo_fp16_to_f32_array(_ptr(h), _ptr(out), h.size)
        return out

    def get_scale_min_k4(self, j: int, scales12: bytes):
        q = np.frombuffer(bytes(scales12), np.uint8).copy()
        d = np.zeros(1, np.uint8)
        m = np.zeros(1, np.uint8)
        self.lib.qo_get_scale_min_k4(j, _ptr(q), _ptr(d), _ptr(m))
        return int(d[0]), int(m[0])

    # dequant / quantize --------------------------------------------------
    def dequant_rows(self, type_id: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        assert w.size >= rows * row_bytes(type_id, cols)
        out = np.empty((rows, cols), np.uint16)
        rc = self.lib.qo_dequant_rows(type_id, _ptr(w), rows, cols, _ptr(out))
        assert rc == 0
        return out

    def quantize_row_q8k_f16(self, x16: np.ndarray):
        x16 = np.ascontiguousarray(x16, dtype=np.uint16).ravel()
        k = x16.size
        d = np.empty(k // 256, np.float32)
        qs = np.empty(k, np.int8)
        bs = np.empty(k // 32, np.int32)
        self.lib.qo_quantize_row_q8k_f16(_ptr(x16), k, _ptr(d), _ptr(qs), _ptr(bs))
        return d, qs, bs

    def quantize_row_q8_0_f16(self, x16: np.ndarray):
        x16 = np.ascontiguousarray(x16, dtype=np.uint16).ravel()
        k = x16.size
        d = np.empty(k // 32, np.float32)
        qs = np.empty(k, np.int8)
        self.lib.qo_quantize_row_q8_0_f16(_ptr(x16), k, _ptr(d), _ptr(qs))
        return d, qs

    def quantize_q8k(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        M, K = x.shape
        d = np.empty((M, K // 256), np.float32)
        qs = np.empty((M, K), np.int8)
        bs = np.empty((M, K // 32), np.int32)
        self.lib.qo_quantize_q8k_f32(_ptr(x), M, K, _ptr(d), _ptr(qs), _ptr(bs))
        return d, qs, bs

    def quantize_q8_0(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        M, K = x.shape
        d = np.empty((M, K // 32), np.float32)
        qs = np.empty((M, K), np.int8)
        self.lib.qo_quantize_q8_0_f32(_ptr(x), M, K, _ptr(d), _ptr(qs))
        return d, qs

    # dots ------------------------------------------------------------------
    def dot_row(self, type_id: int, w_row: np.ndarray, K: int, d, qs, bsum=None) -> float:
        w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
        d = np.ascontiguousarray(d, dtype=np.float32)
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        bs = None if bsum is None else np.ascontiguousarray(bsum, dtype=np.int32)
        return float(self.lib.qo_dot_row(type_id, _ptr(w_row), K, _ptr(d), _ptr(qs),
                                          None if bs is None else _ptr(bs)))

    def dot_row_float(self, type_id: int, w_row: np.ndarray, K: int, x16) -> float:
        """An F32 / F16 row against one fp16 activation row (bits)."""
        w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
        x16 = np.ascontiguousarray(x16, dtype=np.uint16)
        return float(self.lib.qo_dot_row_float(type_id, _ptr(w_row), K, _ptr(x16)))

    def block_partials(self, type_id: int, w_row: np.ndarray, K: int, qs, bsum=None):
        nb = K // BLOCK_VALUES[type_id]
        S = np.zeros(nb, np.int32)
        Mb = np.zeros(nb, np.int32)
        w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        bs = np.zeros(K // 32, np.int32) if bsum is None else np.ascontiguousarray(bsum, np.int32)
        n = self.lib.qo_block_partials(type_id, _ptr(w_row), K, _ptr(qs), _ptr(bs), _ptr(S), _ptr(Mb))
        assert n == nb
        return S, Mb

    def gemm_multi(self, x: np.ndarray, tasks, prequantized=None):
        """Reference dispatcher semantics (E:4188-4262, E:3491-3619).

        ``tasks``: list of dicts with keys ``w`` (uint8 packed rows), ``type``,
        ``rows`` and optional ``residual`` (float32 [M, rows]). Returns one
        float32 [M, rows] array per task. ``prequantized`` = (q8k triple or
        None, q80 pair or None) skips the quantizer; F32 / F16 tasks then read
        x rounded to fp16 (the input the engine still passes, E:4206).
        """
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        M, K = x.shape
        arr = (_MatrixTask * len(tasks))()
        outs, keep = [], []
        for i, t in enumerate(tasks):
            w = np.ascontiguousarray(t["w"], dtype=np.uint8)
            rows = int(t["rows"])
            out = np.zeros((M, rows), np.float32)
            res = t.get("residual")
            if res is not None:
                res = np.ascontiguousarray(res, dtype=np.float32).reshape(M, rows)
            keep += [w, out, res]
            arr[i] = _MatrixTask(_ptr(w), t["type"], row_bytes(t["type"], K), _ptr(out), rows,
                                 None if res is None else _ptr(res), rows, rows, K, 0)
            outs.append(out)
        if prequantized is None:
            rc = self.lib.qo_gemm_multi(_ptr(x), M, K, arr, len(tasks))
        else:
            q8k, q80 = prequantized
            ptrs = []
            x16 = self.f32_to_fp16(x)
            for a in (q8k or (None, None, None)) + (q80 or (None, None)) + (x16,):
                if a is None:
                    ptrs.append(None)
                else:
                    a = np.ascontiguousarray(a)
                    keep.append(a)
                    ptrs.append(_ptr(a))
            rc = self.lib.qo_gemm_multi_prequantized(*ptrs, M, K, arr, len(tasks))
        if rc != 0:
            raise ValueError("oracle rejected the task list")
        return outs

    def gemm(self, type_id: int, w: np.ndarray, N: int, x: np.ndarray) -> np.ndarray:
        return self.gemm_multi(x, [dict(w=w, type=type_id, rows=N)])[0]

    def swiglu_q8k(self, gate: np.ndarray, up: np.ndarray):
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        up = np.ascontiguousarray(up, dtype=np.float32)
        if gate.ndim == 1:
            gate, up = gate[None, :], up[None, :]
        M, N = gate.shape
        h = np.empty((M, N), np.float32)
        d = np.empty((M, N // 256), np.float32)
        qs = np.empty((M, N), np.int8)
        bs = np.empty((M, N // 32), np.int32)
        self.lib.qo_swiglu_q8k(_ptr(gate), _ptr(up), M, N, _ptr(h), _ptr(d), _ptr(qs), _ptr(bs))
        return h, (d, qs, bs)

    def chunk_argmax(self, logits: np.ndarray, best_val, best_id, round16=True, ids=None, row_base=0):
        """The running argmax update over logits [M][rows]; returns new (best_val, best_id)."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        if lg.ndim == 1:
            lg = lg[None, :]
        M, rows = lg.shape
        bv = np.array(best_val, dtype=np.float32).reshape(M).copy()
        bi = np.array(best_id, dtype=np.uint32).reshape(M).copy()
        idp = None
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.uint32)
            idp = _ptr(ids)
        self.lib.qo_chunk_argmax(_ptr(lg), M, rows, rows, 1 if round16 else 0, idp, row_base, _ptr(bv), _ptr(bi))
        return bv, bi

    def lm_head_argmax(self, prequantized, w_rows, type_id: int, rows: int, row_base: int, best_val, best_id):
        """One LM-head chunk on prequantized Q8_K rows: (logits, best_val, best_id)."""
        M = prequantized[0].shape[0]
        K = prequantized[1].shape[1]
        lg = self.gemm_multi(np.zeros((M, K), np.float32), [dict(w=w_rows, type=type_id, rows=rows)],
                             prequantized=(prequantized, None))[0]
        bv, bi = self.chunk_argmax(lg, best_val, best_id, True, None, row_base)
        return lg, bv, bi

    def eval_rows_argmax(self, prequantized, w_tensor, type_id: int, K: int, row_ids, best_val, best_id):
        """Indexed rows: (vals [M][n], best_val, best_id) in list order, fp32 values."""
        rb = row_bytes(type_id, K)
        ids = np.asarray(row_ids, dtype=np.uint32)
        w = np.asarray(w_tensor, np.uint8).reshape(-1)
        rows = np.concatenate([w[int(i) * rb:(int(i) + 1) * rb] for i in ids])
        M = prequantized[0].shape[0]
        vals = self.gemm_multi(np.zeros((M, K), np.float32), [dict(w=rows, type=type_id, rows=len(ids))],
                               prequantized=(prequantized, None))[0]
        bv, bi = self.chunk_argmax(vals, best_val, best_id, False, ids, 0)
        return vals, bv, bi

    def lm_head_scan(self, q8k, w, type_id: int, vocab_rows: int, K: int, chunk_rows: int, thresholds=None,
                     first_checkpoint: int = 0, margin: float = 1e-3, pre_ids=None, draft_ids=None):
        """The chunked vocabulary scan on Q8_K rows q8k = (d, qs, bsum):
        (best_val, best_id, chunks_read, active, stopped)."""
        d, qs, bs = (np.ascontiguousarray(a) for a in q8k)
        M = qs.shape[0]
        w = np.ascontiguousarray(w, np.uint8)
        thr = None if thresholds is None else np.ascontiguousarray(thresholds, np.float32)
        pre = None if pre_ids is None else np.ascontiguousarray(pre_ids, np.uint32)
        dr = None if draft_ids is None else np.ascontiguousarray(draft_ids, np.uint32)
        bv = np.empty(M, np.float32)
        bi = np.empty(M, np.uint32)
        act, stp = C.c_int(), C.c_int()
        n = self.lib.qo_lm_head_scan(type_id, _ptr(w), vocab_rows, K, M, _ptr(d), _ptr(qs), _ptr(bs), chunk_rows,
                                     None if thr is None else _ptr(thr), 0 if thr is None else thr.size,
                                     first_checkpoint, margin, None if pre is None else _ptr(pre),
                                     0 if pre is None else pre.size, None if dr is None else _ptr(dr), _ptr(bv),
                                     _ptr(bi), C.byref(act), C.byref(stp))
        if n < 0:
            raise ValueError("oracle rejected the scan")
        return bv, bi, n, act.value, stp.value

    def lm_head_scan_script(self, q8k, w, type_id: int, vocab_rows: int, K: int, chunk_rows: int, thresholds=None,
                            margin: float = 1e-3, pre_ids=None, draft_ids=None, is_cyr=None, is_cjk=None,
                            cyr_rows=None, cjk_rows=None, has_cyr=False, has_cjk=False, require_full=False,
                            batch1=False):
        """The whole LM-head scan with its script-gated exit (qo_lm_head_scan_script):
        (best_val, best_id, chunks_read, active, stopped, has_cyr, has_cjk)."""
        d, qs, bs = (np.ascontiguousarray(a) for a in q8k)
        M = qs.shape[0]
        w = np.ascontiguousarray(w, np.uint8)
        keep = []

        def arr(a, dt):
            if a is None:
                return None, 0
            a = np.ascontiguousarray(a, dt)
            keep.append(a)
            return _ptr(a), a.size

        thr, nthr = arr(thresholds, np.float32)
        pre, npre = arr(pre_ids, np.uint32)
        dr, _ = arr(draft_ids, np.uint32)
        fc, _ = arr(is_cyr, np.uint8)
        fj, _ = arr(is_cjk, np.uint8)
        rc_, nc = arr(cyr_rows, np.uint32)
        rj, nj = arr(cjk_rows, np.uint32)
        sc = _Script(fc, fj, rc_, nc, rj, nj, int(has_cyr), int(has_cjk), int(require_full), int(batch1))
        bv = np.empty(M, np.float32)
        bi = np.empty(M, np.uint32)
        act, stp = C.c_int(), C.c_int()
        n = self.lib.qo_lm_head_scan_script(type_id, _ptr(w), vocab_rows, K, M, _ptr(d), _ptr(qs), _ptr(bs),
                                            chunk_rows, thr, nthr, margin, pre, npre, dr, C.byref(sc), _ptr(bv),
                                            _ptr(bi), C.byref(act), C.byref(stp))
        if n < 0:
            raise ValueError("oracle rejected the scan")
        return bv, bi, n, act.value, stp.value, bool(sc.has_cyr), bool(sc.has_cjk)

    def rmsnorm_q8k_f16(self, x16: np.ndarray, gamma16: np.ndarray):
        """rmsnorm_fp16_rows_fast on fp16 bits: (y16 [M][K], (d, qs, bsum32))."""
        x16 = np.ascontiguousarray(x16, dtype=np.uint16)
        gamma16 = np.ascontiguousarray(gamma16, dtype=np.uint16)
        if x16.ndim == 1:
            x16 = x16[None, :]
        M, K = x16.shape
        y = np.empty((M, K), np.uint16)
        d = np.empty((M, K // 256), np.float32)
        qs = np.empty((M, K), np.int8)
        bs = np.empty((M, K // 32), np.int32)
        self.lib.qo_rmsnorm_q8k_f16(_ptr(x16), _ptr(gamma16), M, K, _ptr(y), _ptr(d), _ptr(qs), _ptr(bs))
        return y, (d, qs, bs)

    def rmsnorm_q8k(self, x: np.ndarray, gamma: np.ndarray):
        """The fp32 contract: x and gamma rounded to fp16 first; y as fp32."""
        y16, q = self.rmsnorm_q8k_f16(self.f32_to_fp16(np.asarray(x, np.float32)),
                                      self.f32_to_fp16(np.asarray(gamma, np.float32)))
        return self.fp16_to_f32(y16), q


class Reference:
    """The reference's own scalar code compiled in place (oracle/_ref/libref.so)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.ref_fp16_to_f32.restype = C.c_float
        L.ref_fp16_to_f32.argtypes = [C.c_uint16]
        L.ref_f32_to_fp16.restype = C.c_uint16
        L.ref_f32_to_fp16.argtypes = [C.c_float]
        L.ref_get_scale_min_k4.argtypes = [C.c_int, _p, _p, _p]
        L.ref_dequant_block.restype = C.c_int
        L.ref_dequant_block.argtypes = [C.c_uint32, _p, _p]
        L.ref_quantize_row_q8k.argtypes = [_p, C.c_int, _p, _p, _p]
        L.ref_quantize_row_q8_0.argtypes = [_p, C.c_int, _p, _p]
        L.ref_capacity_k.restype = C.c_int
        L.ref_capacity_m.restype = C.c_int
        L.ref_dot_rows.restype = C.c_int
        L.ref_dot_rows.argtypes = [C.c_uint32, _p, C.c_int, C.c_int, _p, _p, _p, C.c_int, _p]
        L.ref_dot_rows_float.restype = C.c_int
        L.ref_dot_rows_float.argtypes = [C.c_uint32, _p, C.c_int, C.c_int, _p, _p]
        L.ref_dequant_contiguous.restype = C.c_int
        L.ref_dequant_contiguous.argtypes = [C.c_uint32, _p, C.c_size_t, _p]
        L.ref_swiglu_q8k.restype = C.c_int
        L.ref_swiglu_q8k.argtypes = [_p, _p, C.c_int, C.c_int, _p, _p, _p]
        L.ref_gguf_parse.restype = C.c_int
        L.ref_gguf_parse.argtypes = [_p, C.c_size_t, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, C.c_int]
        L.ref_rmsnorm_q8k.restype = C.c_int
        L.ref_rmsnorm_q8k.argtypes = [_p, _p, _p, C.c_int, C.c_int, _p, _p, _p]
        L.ref_bench_gemv.restype = C.c_double
        L.ref_bench_gemv.argtypes = [C.c_uint32, _p, C.c_int, C.c_int, _p, _p, C.c_int, C.c_int, C.c_int,
                                     C.c_size_t]
        self.max_k = L.ref_capacity_k()
        self.max_m = L.ref_capacity_m()

    def fp16_to_f32(self, h: int) -> float:
        return float(self.lib.ref_fp16_to_f32(int(h)))

    def f32_to_fp16(self, f: float) -> int:
        return int(self.lib.ref_f32_to_fp16(float(f)))

    def get_scale_min_k4(self, j: int, scales12: bytes):
        q = np.frombuffer(bytes(scales12), np.uint8).copy()
        d = np.zeros(1, np.uint8)
        m = np.zeros(1, np.uint8)
        self.lib.ref_get_scale_min_k4(j, _ptr(q), _ptr(d), _ptr(m))
        return int(d[0]), int(m[0])

    def dequant_rows(self, type_id: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        qk, bb = BLOCK_VALUES[type_id], BLOCK_BYTES[type_id]
        nblk = rows * cols // qk
        out = np.empty(nblk * qk, np.uint16)
        for b in range(nblk):
            blk = np.ascontiguousarray(w[b * bb:(b + 1) * bb])
            o = np.empty(qk, np.uint16)
            assert self.lib.ref_dequant_block(type_id, _ptr(blk), _ptr(o)) == 0
            out[b * qk:(b + 1) * qk] = o
        return out.reshape(rows, cols)

    def quantize_row_q8k_f16(self, x16: np.ndarray):
        x16 = np.ascontiguousarray(x16, dtype=np.uint16).ravel()
        k = x16.size
        d = np.empty(k // 256, np.float32)
        qs = np.empty(k, np.int8)
        bs = np.empty(k // 32, np.int32)
        self.lib.ref_quantize_row_q8k(_ptr(x16), k, _ptr(d), _ptr(qs), _ptr(bs))
        return d, qs, bs

    def quantize_row_q8_0_f16(self, x16: np.ndarray):
        x16 = np.ascontiguousarray(x16, dtype=np.uint16).ravel()
        k = x16.size
        d = np.empty(k // 32, np.float32)
        qs = np.empty(k, np.int8)
        self.lib.ref_quantize_row_q8_0(_ptr(x16), k, _ptr(d), _ptr(qs))
        return d, qs

    def dot_rows(self, type_id: int, w_row: np.ndarray, K: int, d, qs, bsum=None,
                 batch_kernel: bool = False) -> np.ndarray:
        """Dots of one weight row with M activation rows (arrays shaped [M, ...])."""
        d = np.ascontiguousarray(d, dtype=np.float32)
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        M = qs.shape[0] if qs.ndim == 2 else 1
        bs = np.zeros((M, K // 32), np.int32) if bsum is None else np.ascontiguousarray(bsum, np.int32)
        w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
        out = np.empty(M, np.float32)
        rc = self.lib.ref_dot_rows(type_id, _ptr(w_row), M, K, _ptr(d), _ptr(qs), _ptr(bs),
                                   1 if batch_kernel else 0, _ptr(out))
        if rc != 0:
            raise ValueError("outside the reference's static capacity")
        return out

    def dot_rows_float(self, type_id: int, w_row: np.ndarray, K: int, x16) -> np.ndarray:
        """sdot_row_f32_batch / _f16_batch: one row against M fp16 rows [M, K]."""
        x16 = np.ascontiguousarray(x16, dtype=np.uint16)
        if x16.ndim == 1:
            x16 = x16[None, :]
        M = x16.shape[0]
        w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
        out = np.empty(M, np.float32)
        if self.lib.ref_dot_rows_float(type_id, _ptr(w_row), M, K, _ptr(x16), _ptr(out)) != 0:
            raise ValueError("outside the reference's static capacity")
        return out

    def dequant_contiguous(self, type_id: int, w: np.ndarray, n_elems: int) -> np.ndarray:
        """dequant_contiguous_fast -> fp16 bits (any supported type, incl. F32 / F16)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        out = np.zeros(n_elems, np.uint16)
        self.lib.ref_dequant_contiguous(type_id, _ptr(w), n_elems, _ptr(out))
        return out

    def swiglu_q8k(self, gate16: np.ndarray, up16: np.ndarray):
        g = np.ascontiguousarray(gate16, dtype=np.uint16).copy()
        u = np.ascontiguousarray(up16, dtype=np.uint16)
        if g.ndim == 1:
            g, u = g[None, :], u[None, :]
        M, N = g.shape
        d = np.empty((M, N // 256), np.float32)
        qs = np.empty((M, N), np.int8)
        bs = np.empty((M, N // 32), np.int32)
        rc = self.lib.ref_swiglu_q8k(_ptr(g), _ptr(u), M, N, _ptr(d), _ptr(qs), _ptr(bs))
        if rc != 0:
            raise ValueError("outside the reference's static capacity")
        return g, (d, qs, bs)

    def gguf_parse(self, data: bytes, cap: int = 512):
        """parse_gguf_file on the bytes: None if rejected, else (alignment,
        data_offset, [tensor dicts])."""
        buf = np.frombuffer(data, dtype=np.uint8).copy()
        al, do = np.zeros(1, np.uint64), np.zeros(1, np.uint64)
        names = np.zeros((cap, 128), np.uint8)
        nd, ty = np.zeros(cap, np.uint32), np.zeros(cap, np.uint32)
        dims = np.zeros((cap, 4), np.uint64)
        rel, ab, ne, bs = (np.zeros(cap, np.uint64) for _ in range(4))
        n = self.lib.ref_gguf_parse(_ptr(buf), buf.size, _ptr(al), _ptr(do), _ptr(names), _ptr(nd), _ptr(dims),
                                    _ptr(ty), _ptr(rel), _ptr(ab), _ptr(ne), _ptr(bs), cap)
        if n < 0:
            return None
        ts = []
        for i in range(min(n, cap)):
            ts.append(dict(name=bytes(names[i]).split(b"\0")[0].decode("utf-8", "replace"), n_dims=int(nd[i]),
                           dims=[int(v) for v in dims[i]], type=int(ty[i]), rel_offset=int(rel[i]),
                           abs_offset=int(ab[i]), n_elems=int(ne[i]), byte_size=int(bs[i])))
        return int(al[0]), int(do[0]), ts

    def rmsnorm_q8k(self, x16: np.ndarray, gamma16: np.ndarray):
        x = np.ascontiguousarray(x16, dtype=np.uint16)
        gm = np.ascontiguousarray(gamma16, dtype=np.uint16)
        if x.ndim == 1:
            x = x[None, :]
        M, K = x.shape
        y = np.empty((M, K), np.uint16)
        d = np.empty((M, K // 256), np.float32)
        qs = np.empty((M, K), np.int8)
        bs = np.empty((M, K // 32), np.int32)
        rc = self.lib.ref_rmsnorm_q8k(_ptr(x), _ptr(gm), _ptr(y), M, K, _ptr(d), _ptr(qs), _ptr(bs))
        if rc != 0:
            raise ValueError("outside the reference's static capacity")
        return y, (d, qs, bs)

    def bench_gemv(self, type_id: int, w: np.ndarray, N: int, K: int, x16: np.ndarray,
                   threads: int, iters: int, replicas: int = 1):
        """Wall seconds of `iters` GEMVs; w holds `replicas` copies of the
        tensor back to back, pass i reads copy i mod replicas."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x16 = np.ascontiguousarray(x16, dtype=np.uint16)
        y = np.empty(N, np.float32)
        stride = w.size // replicas
        t = self.lib.ref_bench_gemv(type_id, _ptr(w), N, K, _ptr(x16), _ptr(y), threads, iters, replicas, stride)
        if t < 0:
            raise ValueError("bench_gemv rejected its arguments")
        return t, y


def load_oracle() -> Oracle:
    return Oracle()


def load_reference():
    """The compiled reference, or None where it was not built."""
    return Reference() if os.path.exists(REF_SO) else None
