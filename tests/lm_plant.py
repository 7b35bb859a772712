"""LM-head weights with planted logits, for the chunked-scan tests.

A Q6_K vocabulary tensor whose random rows have a tiny scale (fp16 d about
1e-5, so every random logit stays below 1), and planted rows whose 6-bit
codes follow one token's activations, scaled so that their logit for that
token is close to a chosen value (the exact value is whatever the oracle
computes; the plan only needs it on the chosen side of each threshold).
"""
import numpy as np

import kquant_pack as kp
import synth
from oracle import TYPE_Q6_K

RB = 2100  # Q6_K row of K = 2560


def base_tensor(rows: int, K: int, seed: int) -> np.ndarray:
    """Random Q6_K rows with every block's d rescaled to ~1e-5."""
    w = synth.weights(TYPE_Q6_K, rows, K, seed=seed).copy()
    nb = rows * (K // 256)
    blk = w.reshape(nb, 210)
    d = np.random.default_rng(seed + 1).uniform(0.5e-5, 1.5e-5, nb).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return w


def aligned_row(x: np.ndarray, d: float) -> np.ndarray:
    """One Q6_K row (K = len(x)) whose codes follow x: q - 32 = round(31 x /
    max|x|) per block, every scale 16, fp16 scale d."""
    K = x.size
    blocks = []
    for b in range(K // 256):
        xs = x[256 * b:256 * (b + 1)].astype(np.float64)
        q = np.clip(np.rint(31.0 * xs / max(np.abs(xs).max(), 1e-12)), -32, 31).astype(int) + 32
        blocks.append(kp.pack_q6_k(d, np.full(16, 16), q))
    return np.concatenate(blocks)


def plant(w: np.ndarray, oracle, q8k, plan, K: int):
    """plan: list of (row, token, target logit). Each row gets codes that
    follow the token's activations and the d that brings its logit near the
    target; returns the achieved fp32 logits per plan entry."""
    d, qs, bs = q8k
    out = []
    for row, tok, target in plan:
        x = qs[tok].astype(np.float32) * np.repeat(d[tok], 256)
        unit = aligned_row(x, 1.0)
        v1 = oracle.dot_row(TYPE_Q6_K, unit, K, d[tok], qs[tok], bs[tok])
        scale = float(np.float16(target / v1))
        r = aligned_row(x, scale)
        w[row * RB:(row + 1) * RB] = r
        out.append(oracle.dot_row(TYPE_Q6_K, r, K, d[tok], qs[tok], bs[tok]))
    return out


CHUNK_THRESH = [19.5, 16.0, 13.5, 11.5, 10.5, 10.0, 10.0, 10.0, 10.0, -1e30]  # E:11245
