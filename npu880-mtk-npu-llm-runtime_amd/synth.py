"""Seeded synthetic GGUF-layout tensors and activations for the benchmark
workloads (Philox counter-based generator, seed per tensor).

Distributions: fp16 super-block scales d / dmin ~ U[1e-3, 4e-3]; packed
scale bytes and code bytes uniform random, which makes the 6-bit Q4_K /
Q5_K sub-block scales and mins ~U{0..63} and the 4/5/6-bit codes uniform;
Q6_K sub-block scales int8 ~U{-32..31}; Q8_0 codes int8 ~U{-127..127};
activations fp32 ~N(0, 1).
"""
from __future__ import annotations

import numpy as np

TYPE_F32, TYPE_F16 = 0, 1
TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 8, 12, 13, 14
BLOCK_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}
BLOCK_VALUES = {TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256, TYPE_Q6_K: 256}


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(key=int(seed)))


def _fp16_scales(g: np.random.Generator, n: int) -> np.ndarray:
    v = g.uniform(1e-3, 4e-3, n).astype(np.float32).astype(np.float16)
    return v.view(np.uint16)


def _bytes(g: np.random.Generator, n: int, width: int) -> np.ndarray:
    return np.frombuffer(g.bytes(n * width), np.uint8).reshape(n, width)


def blocks(type_id: int, n_blocks: int, seed: int) -> np.ndarray:
    """n_blocks packed blocks of `type_id`, shape [n_blocks, block_bytes]."""
    g = rng(seed)
    bb = BLOCK_BYTES[type_id]
    out = np.empty((n_blocks, bb), np.uint8)
    if type_id in (TYPE_Q4_K, TYPE_Q5_K):
        out[:, 0:2] = _fp16_scales(g, n_blocks).view(np.uint8).reshape(n_blocks, 2)
        out[:, 2:4] = _fp16_scales(g, n_blocks).view(np.uint8).reshape(n_blocks, 2)
        out[:, 4:] = _bytes(g, n_blocks, bb - 4)
    elif type_id == TYPE_Q6_K:
        out[:, 0:192] = _bytes(g, n_blocks, 192)
        out[:, 192:208] = g.integers(-32, 32, (n_blocks, 16), dtype=np.int8).view(np.uint8)
        out[:, 208:210] = _fp16_scales(g, n_blocks).view(np.uint8).reshape(n_blocks, 2)
    elif type_id == TYPE_Q8_0:
        out[:, 0:2] = _fp16_scales(g, n_blocks).view(np.uint8).reshape(n_blocks, 2)
        out[:, 2:] = g.integers(-127, 128, (n_blocks, 32), dtype=np.int8).view(np.uint8)
    else:
        raise ValueError(f"unsupported type {type_id}")
    return out


def weights(type_id: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols tensor as packed rows: uint8 [rows * row_bytes]."""
    nb = cols // BLOCK_VALUES[type_id]
    assert nb * BLOCK_VALUES[type_id] == cols
    return blocks(type_id, rows * nb, seed).reshape(-1)


def activations(M: int, K: int, seed: int) -> np.ndarray:
    return rng(seed).standard_normal((M, K), dtype=np.float32)


def row_bytes(type_id: int, cols: int) -> int:
    if type_id in (TYPE_F32, TYPE_F16):
        return cols * (4 if type_id == TYPE_F32 else 2)
    return (cols // BLOCK_VALUES[type_id]) * BLOCK_BYTES[type_id]


def float_rows(type_id: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """F32 / F16 weight rows ~N(0, 0.05^2) as bytes [rows * row_bytes]."""
    v = rng(seed).standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    return (v if type_id == TYPE_F32 else v.astype(np.float16)).view(np.uint8).reshape(-1)


def q6k_row_following(x: np.ndarray, target: float) -> np.ndarray:
    """One Q6_K row (K = x.size) whose codes follow x — per block
    q - 32 = round(31 x / max|x|), every scale 16 — with the fp16 d that puts
    its fp32 dot with x near `target` (the dot with x's Q8_K codes differs by
    the quantization error, about 1 %)."""
    K = x.size
    xb = x.astype(np.float64).reshape(K // 256, 256)
    q = np.clip(np.rint(31.0 * xb / np.maximum(np.abs(xb).max(axis=1, keepdims=True), 1e-12)), -32, 31)
    d = float(np.float16(target / (16.0 * float(np.sum(q * xb)))))
    codes = (q + 32).astype(np.uint8)  # [block][256], value k = 128 half + 32 i + l
    out = np.zeros((K // 256, 210), np.uint8)
    c = codes.reshape(-1, 2, 4, 32)  # block, half, i, l
    for h in range(2):
        out[:, 64 * h:64 * h + 32] = (c[:, h, 0] & 15) | ((c[:, h, 2] & 15) << 4)
        out[:, 64 * h + 32:64 * h + 64] = (c[:, h, 1] & 15) | ((c[:, h, 3] & 15) << 4)
        out[:, 128 + 32 * h:160 + 32 * h] = ((c[:, h, 0] >> 4) | ((c[:, h, 1] >> 4) << 2) | ((c[:, h, 2] >> 4) << 4)
                                             | ((c[:, h, 3] >> 4) << 6))
    out[:, 192:208] = 16
    out[:, 208:210] = np.array([d], np.float16).view(np.uint8)
    return out.reshape(-1)


def lm_head_small_logits(rows: int, cols: int, seed: int) -> np.ndarray:
    """A Q6_K vocabulary tensor of random rows with fp16 d ~U[0.5e-5, 1.5e-5]:
    every random logit of an N(0, 1) input stays below about 1."""
    w = weights(TYPE_Q6_K, rows, cols, seed=seed).copy()
    nb = rows * (cols // 256)
    blk = w.reshape(nb, 210)
    d = rng(seed + 1).uniform(0.5e-5, 1.5e-5, nb).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return w


# The benchmark workloads: (type, rows N, cols K) per tensor.
GEMV_Q4K = dict(type=TYPE_Q4_K, N=9728, K=2560)
GEMV_Q6K_LMHEAD = dict(type=TYPE_Q6_K, N=151936, K=2560)
FFN = dict(gate=(TYPE_Q4_K, 9728, 2560), up=(TYPE_Q4_K, 9728, 2560), down=(TYPE_Q6_K, 2560, 9728))
TREE_VERIFY = dict(M=(8, 16, 32, 64), q4k=(TYPE_Q4_K, 9728, 2560), q5k=(TYPE_Q5_K, 4096, 2560),
                   q6k=(TYPE_Q6_K, 2560, 9728))
PREFILL_LAYER = dict(
    M=512,
    tensors=dict(qkv=(TYPE_Q5_K, 6144, 2560), o=(TYPE_Q4_K, 2560, 4096),
                 gate=(TYPE_Q4_K, 9728, 2560), up=(TYPE_Q4_K, 9728, 2560),
                 down=(TYPE_Q6_K, 2560, 9728), q8_0=(TYPE_Q8_0, 2560, 2560)),
)
