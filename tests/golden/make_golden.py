"""Writes the committed fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference's own golden files (GGUF dumps of the PyTorch model, made by
convert/dump_dit_golden.py and convert/dump_dit_debug2.py) are not in the
reference tree, and ggml (where the path's arithmetic lives) is absent, so
these fixtures are computed here from the mathematics with exact rational
rounding (fractions.Fraction) and fp64 textbook formulas (tests/refmath.py),
independently of the oracle's C code. Seeds follow the reference's dumpers:
1234 for features/weights (convert/dump_dit_golden.py:30), 4242 for noise
(src/tools/generate.cpp:47).
"""
import os
import sys
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import refmath  # noqa: E402


def f32_bits(v):
    return np.array([v], dtype=np.float32).view(np.uint32)[0]


def conversions():
    vals = [0.0, -0.0, 1.0, -1.0, 0.1, 1 / 3, 65504.0, 65519.0, 65520.0, 1e5, -1e5,
            6.103515625e-05, 6.0e-05, 5.960464477539063e-08, 2.98e-08, 2.9802322387695312e-08,
            1e-10, 3.0e38, -3.4e38, 1.0009765625, 1.00048828125, 1.000732421875,
            1.0039062, 1.00390625, 1.005859375, 1.01171875, 2.0078125, 3.14159265, -2.71828,
            1.17549435e-38, 1e-40]
    rng = np.random.default_rng(1234)
    vals += list(rng.standard_normal(64).astype(np.float32) * 10.0)
    vals += list((rng.standard_normal(32) * 1e-5).astype(np.float32))
    x = np.array(vals, dtype=np.float32)
    f16 = np.array([refmath.to_f16_exact(float(v)) for v in x], dtype=np.float64)
    bf16 = np.array([refmath.to_bf16_exact(float(v)) for v in x], dtype=np.float64)
    f16_bits = f16.astype(np.float16).view(np.uint16)          # exact: values are on the grid
    bf16_bits = (bf16.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    np.savez(os.path.join(HERE, "conversions.npz"), x=x, f16_bits=f16_bits, bf16_bits=bf16_bits)


def _q8_expected(block, mode):
    """Exact-arithmetic Q8_0 quantization of one 32-float block.
    mode 0 = ggml-cpu x86 (d=amax/127, q=rne(fl(x*fl(127/amax)))),
    mode 1 = ggml scalar ref (q=half-away(fl(x*fl(1/d)))),
    mode 2 = gguf-py (q=half-away(fl(x/d)))."""
    f32 = refmath.to_f32_exact
    amax = max(abs(float(v)) for v in block)
    d = f32(Fraction(amax) / 127) if amax != 0 else 0.0
    qs = []
    for v in block:
        v = float(v)
        if amax == 0:
            qs.append(0)
            continue
        if mode == 0:
            t = Fraction(f32(Fraction(v) * Fraction(f32(Fraction(127) / Fraction(amax)))))
            q = round(t)                                   # Python round = half to even
        else:
            if mode == 1:
                t = Fraction(f32(Fraction(v) * Fraction(f32(1 / Fraction(d)))))
            else:
                t = Fraction(f32(Fraction(v) / Fraction(d)))
            a = abs(t)
            fl = a.numerator // a.denominator
            q = fl + (1 if a - fl >= Fraction(1, 2) else 0)
            q = -q if t < 0 else q
        qs.append(q)
    d_bits = np.array([refmath.to_f16_exact(d)], dtype=np.float64).astype(np.float16).view(np.uint16)[0]
    return d_bits, np.array(qs, dtype=np.int8)


def q8_0():
    # known-answer dequant blocks: (d, qs) -> d*q exactly
    kat_d = np.array([1.0, 0.0, 5.960464477539063e-08, 65504.0, 0.0078125, -0.5], dtype=np.float16)
    kat_q = np.zeros((len(kat_d), 32), dtype=np.int8)
    kat_q[0] = np.arange(-127, 128, 8)[:32]
    kat_q[1] = 77
    kat_q[2] = np.arange(32) - 16
    kat_q[3] = [127, -127, 1, -1] * 8
    kat_q[4] = np.arange(32) * 4 - 64
    kat_q[5] = -np.arange(32)
    blocks = np.zeros((len(kat_d), 34), dtype=np.uint8)
    blocks[:, :2] = kat_d.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = kat_q.view(np.uint8)
    deq = np.array([[float(Fraction(float(d)) * int(q)) for q in qrow]
                    for d, qrow in zip(kat_d, kat_q)], dtype=np.float32)
    # quantization inputs with ties at .5 and degenerate blocks
    rng = np.random.default_rng(1234)
    qin = [np.array([127.0] + [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5, 126.5] + [0.0] * 23, dtype=np.float32),
           np.zeros(32, dtype=np.float32),
           np.array([1e-3 * (i - 16) for i in range(32)], dtype=np.float32),
           np.array([(-1) ** i * 1e4 for i in range(32)], dtype=np.float32)]
    qin += [rng.standard_normal(32).astype(np.float32) * s for s in (0.02, 1.0, 30.0)]
    qin = np.stack(qin)
    d_bits = np.zeros((3, len(qin)), dtype=np.uint16)
    qs = np.zeros((3, len(qin), 32), dtype=np.int8)
    for mode in range(3):
        for i, blk in enumerate(qin):
            d_bits[mode, i], qs[mode, i] = _q8_expected(blk, mode)
    np.savez(os.path.join(HERE, "q8_0.npz"), kat_blocks=blocks, kat_deq=deq, q_in=qin,
             q_d_bits=d_bits, q_qs=qs)


def attention():
    rng = np.random.default_rng(1234)
    B, H, N, D = 1, 2, 9, 64
    q = rng.standard_normal((B, H, N, D)).astype(np.float32)
    k = rng.standard_normal((B, H, 11, D)).astype(np.float32)
    v = rng.standard_normal((B, H, 11, D)).astype(np.float32)
    mask = np.zeros((1, 1, 16, 11), dtype=np.float16)
    mask[..., 7:] = -np.inf
    mask[..., 3, 2] = -1.5
    o = refmath.attention(q, k, v, 0.125)                          # (B,H,N,D)
    om = refmath.attention(q, k, v, 0.125, mask[..., :N, :].astype(np.float64))
    np.savez(os.path.join(HERE, "attention.npz"), q=q, k=k, v=v, mask=mask,
             out=o.transpose(0, 2, 1, 3), out_mask=om.transpose(0, 2, 1, 3))


def rope_and_norms():
    rng = np.random.default_rng(1234)
    S, H, D = 7, 3, 64
    x = rng.standard_normal((1, S, H, D)).astype(np.float32)
    pos = np.array([0, 1, 2, 17, 193, 645, 1039], dtype=np.int32)
    y = refmath.rope_normal(x[0], pos, 64, 10000.0, 1.0)[None]
    y2 = refmath.rope_normal(x[0], pos, 64, 10000.0, 194.0 / 72.0)[None]
    w = (1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    rms = refmath.rms_norm(x, 1e-6, w)
    ln = refmath.layer_norm(x, 1e-5)
    np.savez(os.path.join(HERE, "rope_norm.npz"), x=x, pos=pos, rope=y, rope_clip=y2, w=w,
             rms=rms, ln=ln)


def mul_mat():
    rng = np.random.default_rng(1234)
    M, K, N = 24, 96, 5
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    w_bf16 = np.array([refmath.to_bf16_exact(float(v)) for v in w.ravel()], dtype=np.float32).reshape(M, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    x_bf16 = np.array([refmath.to_bf16_exact(float(v)) for v in x.ravel()], dtype=np.float64).reshape(N, K)
    y = x_bf16 @ w_bf16.astype(np.float64).T
    w_bits = (w_bf16.view(np.uint32) >> 16).astype(np.uint16)
    np.savez(os.path.join(HERE, "mul_mat_bf16.npz"), w_bits=w_bits, x=x, y=y)


if __name__ == "__main__":
    conversions()
    q8_0()
    attention()
    rope_and_norms()
    mul_mat()
    print("fixtures written to", HERE)
