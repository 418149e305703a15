"""Textbook fp64 / exact-arithmetic formulations used to pin the oracle.

Each function is written from the mathematics (not from the oracle's code):
explicit softmax matrices instead of online softmax, np.power angles instead
of ggml's running product, Fraction-exact rounding instead of bit tricks.
"""
from fractions import Fraction

import numpy as np


# ------------------------------------------------------------------ rounding
def _round_fraction_to_grid(x: Fraction, ulp: Fraction) -> Fraction:
    """Round x to the nearest multiple of ulp, ties to even multiple."""
    q = x / ulp
    lo = q.numerator // q.denominator
    rem = q - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    return lo * ulp


def round_to_format(v, mant_bits: int, emin: int, emax: int) -> float:
    """Exact round-to-nearest-even of a finite float or Fraction to a binary
    format with mant_bits explicit mantissa bits and normal exponent range
    [emin, emax]; returns +-inf on overflow. Exact rational arithmetic."""
    if not isinstance(v, Fraction):
        if v == 0 or not np.isfinite(v):
            return float(v)
    elif v == 0:
        return 0.0
    x = Fraction(v)
    s = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant_bits)
    r = _round_fraction_to_grid(x, ulp)
    max_finite = (2 - Fraction(2) ** (-mant_bits)) * Fraction(2) ** emax
    if r > max_finite:
        return s * float("inf")
    return s * float(r)


def to_bf16_exact(v):
    return round_to_format(float(v), 7, -126, 127)


def to_f16_exact(v):
    return round_to_format(float(v), 10, -14, 15)


def to_f32_exact(v):
    """Correctly rounded fp32 value of a float or Fraction."""
    return round_to_format(v, 23, -126, 127)


# ------------------------------------------------------------------ ops
def attention(q, k, v, scale, mask=None):
    """softmax(q k^T * scale + mask) v in fp64. q (..., Nq, D), k/v (..., Nkv, D)."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    s = np.einsum("...qd,...kd->...qk", q, k) * scale
    if mask is not None:
        s = s + mask.astype(np.float64)
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    den = p.sum(axis=-1, keepdims=True)
    den = np.where(den == 0, 1.0, den)
    return np.einsum("...qk,...kd->...qd", p / den, v)


def rms_norm(x, eps, w=None):
    x = x.astype(np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return y if w is None else y * np.asarray(w, dtype=np.float64)


def layer_norm(x, eps):
    x = x.astype(np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps)


def rope_normal(x, pos, n_dims, base=10000.0, fscale=1.0):
    """Rotate adjacent pairs (x_2i, x_2i+1) by pos*fscale*base^(-2i/n_dims),
    written as multiplication by a unit complex number. x (..., S, H, D)."""
    x = x.astype(np.float64)
    i = np.arange(n_dims // 2, dtype=np.float64)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * fscale * np.power(base, -2.0 * i / n_dims)
    z = x[..., :n_dims:2] + 1j * x[..., 1:n_dims:2]
    rot = np.exp(1j * ang)[:, None, :]          # (S, 1, n_dims/2) broadcast over heads
    z = z * rot
    out = x.copy()
    out[..., :n_dims:2] = z.real
    out[..., 1:n_dims:2] = z.imag
    return out


def gelu_tanh(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def q8_0_blocks_to_parts(blocks):
    """(rows, nb, 34) uint8 -> (d fp16 as float64 (rows, nb), qs int64 (rows, nb, 32))."""
    d = blocks[..., :2].copy().view(np.float16)[..., 0].astype(np.float64)
    qs = blocks[..., 2:].copy().view(np.int8).astype(np.int64)
    return d, qs


def q8_0_matmul_exact(wblocks, xblocks):
    """sum_b d_w d_x sum_j qw qx with exact integer block sums, fp64 scaling.
    wblocks (M, nb, 34), xblocks (N, nb, 34) -> (N, M)."""
    dw, qw = q8_0_blocks_to_parts(wblocks)
    dx, qx = q8_0_blocks_to_parts(xblocks)
    isum = np.einsum("mbj,nbj->nmb", qw, qx)          # exact int64
    return np.einsum("nmb,mb,nb->nm", isum.astype(np.float64), dw, dx)
