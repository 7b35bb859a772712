"""Writes tests/golden/golden_vectors.npz: known-answer vectors produced by
the reference's own scalar code compiled in place (oracle/_ref/libref.so,
built by oracle/Makefile from src/v182_r22_breakthrough_engine.c).

The reference ships no fixtures of its own for this path, so these are the
pins that travel with the repository: dequantized fp16 bits per type,
Q8_K / Q8_0 activation codes, fp32 row-dot sums (bit patterns), and the
SwiGLU requant. Inputs are seeded (Philox) synthetic blocks plus edge cases.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "npu880-mtk-npu-llm-runtime_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import kquant_pack as kp  # noqa: E402
import oracle as O  # noqa: E402
import synth  # noqa: E402

TYPES = {"q4_k": O.TYPE_Q4_K, "q5_k": O.TYPE_Q5_K, "q6_k": O.TYPE_Q6_K, "q8_0": O.TYPE_Q8_0}


def special_blocks(t):
    if t == O.TYPE_Q4_K:
        return [kp.pack_q4_k(0.0, 0.5, np.zeros(8, int), np.full(8, 63), np.full(256, 15)),
                kp.pack_q4_k(1.0, 0.25, np.arange(8) * 9, np.arange(8) * 7, np.arange(256) % 16)]
    if t == O.TYPE_Q5_K:
        return [kp.pack_q5_k(1.0, 0.0, np.ones(8, int), np.zeros(8, int), np.arange(256) % 32),
                kp.pack_q5_k(6e-5, 2.0, np.full(8, 63), np.full(8, 63), np.full(256, 31))]
    if t == O.TYPE_Q6_K:
        return [kp.pack_q6_k(1.0, np.full(16, -128), np.arange(256) % 64),
                kp.pack_q6_k(0.5, np.arange(16) - 8, np.full(256, 63))]
    return [kp.pack_q8_0(1.0, np.arange(-16, 16)), kp.pack_q8_0(0.125, np.full(32, -128))]


def main():
    ref = O.load_reference()
    if ref is None:
        sys.exit("oracle/_ref/libref.so missing: run make -C oracle")
    out = {}
    # fp16 casts
    g = np.random.default_rng(1234)
    f = np.concatenate([g.standard_normal(512).astype(np.float32) * 50,
                        np.array([0.0, -0.0, 65504, 65519.99, 65520, 6e-8, 2.98e-8, 1e-9,
                                  1.00048828125, 1.000732421875, -3.0517578e-05], np.float32)])
    out["fp16_in"] = f
    out["fp16_out"] = np.array([ref.f32_to_fp16(float(v)) for v in f], np.uint16)
    # dequant
    for name, t in TYPES.items():
        qk = 32 if t == O.TYPE_Q8_0 else 256
        w = np.concatenate([synth.blocks(t, 6, seed=900 + t).reshape(-1)] + special_blocks(t))
        n = w.size // O.BLOCK_BYTES[t]
        out[f"dq_{name}_w"] = w
        out[f"dq_{name}_y"] = ref.dequant_rows(t, w, n, qk)
    # quantizers
    rows = [g.standard_normal(512).astype(np.float32),
            (g.standard_normal(512) * 1e-3).astype(np.float32)]
    tie = np.zeros(512, np.float32)
    tie[:8] = [127, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5]
    tie[300] = -0.75
    rows.append(tie)
    x16 = np.stack([r.astype(np.float16).view(np.uint16) for r in rows])
    out["q_x16"] = x16
    kq = [ref.quantize_row_q8k_f16(r) for r in x16]
    out["q8k_d"] = np.stack([a[0] for a in kq])
    out["q8k_qs"] = np.stack([a[1] for a in kq])
    out["q8k_bs"] = np.stack([a[2] for a in kq])
    zq = [ref.quantize_row_q8_0_f16(r) for r in x16]
    out["q80_d"] = np.stack([a[0] for a in zq])
    out["q80_qs"] = np.stack([a[1] for a in zq])
    # dots: 3 rows x M=3 activations, K = 512
    K, M = 512, 3
    xf = synth.activations(M, K, seed=77)
    out["dot_x"] = xf
    d, qs, bs = (np.stack(v) for v in zip(*[ref.quantize_row_q8k_f16(r.astype(np.float16).view(np.uint16)) for r in xf]))
    d0, q0 = (np.stack(v) for v in zip(*[ref.quantize_row_q8_0_f16(r.astype(np.float16).view(np.uint16)) for r in xf]))
    for name, t in TYPES.items():
        w = synth.weights(t, 3, K, seed=500 + t)
        rb = w.size // 3
        out[f"dot_{name}_w"] = w
        ys = []
        for r in range(3):
            row = w[r * rb:(r + 1) * rb]
            if t == O.TYPE_Q8_0:
                ys.append(ref.dot_rows(t, row, K, d0, q0, None, batch_kernel=True))
            else:
                ys.append(ref.dot_rows(t, row, K, d, qs, bs))
        out[f"dot_{name}_y"] = np.stack(ys, axis=1)  # [M, rows]
    # swiglu + requant (fp16 gate/up as the reference takes them)
    gate = (g.standard_normal((2, 512)) * 3).astype(np.float16)
    up = g.standard_normal((2, 512)).astype(np.float16)
    h16, (sd, sqs, sbs) = ref.swiglu_q8k(gate.view(np.uint16), up.view(np.uint16))
    out.update(sw_gate=gate.view(np.uint16), sw_up=up.view(np.uint16), sw_h=h16,
               sw_d=sd, sw_qs=sqs, sw_bs=sbs)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
