"""Pins of the oracle's convolution / SwiGLU restatement (oracle/tsk_oracle_conv.c)
against what the mathematics fixes, on the CPU:

- im2col against an independent numpy construction (pad, then strided taps);
- conv_cl against torch.nn.functional.conv1d in float64 -- the PyTorch op the
  reference graph's conv_cl reproduces (nn.Conv1d weights [OC, IC, KW] are
  ggml's [KW, IC, OC] kernel in the same memory), with stride, padding and
  dilation, F32 and BF16 kernels;
- the SwiGLU MLPs against torch's silu composed with the same convolutions.

A tap-order mistake (kernel flipped along KW) or an (ic, kw) flattening swap
would fail the torch comparison; test_conv_check_is_sensitive shows both
variants differ from torch by far more than the tolerance.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402

torch = pytest.importorskip("torch")
F = torch.nn.functional


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(((a - b) ** 2).sum() / max((b ** 2).sum(), 1e-300)))


def bf16_round(x):
    return oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.asarray(x, np.float32)))


def im2col_numpy(x, kw, s0, p0, d0):
    """x (N, IC, IW) -> (N, OW, IC*KW): zero-pad by p0, then tap kw of output ow
    reads padded position ow*s0 + kw*d0."""
    N, IC, IW = x.shape
    xp = np.zeros((N, IC, IW + 2 * p0 + d0 * kw + s0), np.float32)
    xp[:, :, p0:p0 + IW] = x
    ow = oracle.conv_len(IW, kw, s0, p0, d0)
    out = np.empty((N, ow, IC, kw), np.float32)
    for t in range(ow):
        for k in range(kw):
            out[:, t, :, k] = xp[:, :, t * s0 + k * d0]
    return out.reshape(N, ow, IC * kw)


@pytest.mark.parametrize("kw,s0,p0,d0", [(3, 1, 1, 1), (7, 1, 3, 1), (3, 2, 1, 1), (3, 1, 2, 2), (1, 1, 0, 1),
                                         (5, 3, 0, 2)])
def test_im2col_closed_form(kw, s0, p0, d0):
    rng = np.random.default_rng(kw * 100 + s0 * 10 + d0)
    x = rng.standard_normal((2, 5, 17)).astype(np.float32)
    got = oracle.im2col_1d(x, kw, s0, p0, d0)
    assert np.array_equal(got, im2col_numpy(x, kw, s0, p0, d0))


def torch_conv(w, x, bias, s0, p0, d0):
    """w (OC, IC, KW), x (B, IW, IC) -> (B, OW, OC), float64."""
    xt = torch.from_numpy(np.asarray(x, np.float64)).permute(0, 2, 1)
    wt = torch.from_numpy(np.asarray(w, np.float64))
    bt = torch.from_numpy(np.asarray(bias, np.float64)) if bias is not None else None
    return F.conv1d(xt, wt, bt, stride=s0, padding=p0, dilation=d0).permute(0, 2, 1).numpy()


@pytest.mark.parametrize("kw,s0,p0,d0", [(3, 1, 1, 1), (7, 1, 3, 1), (3, 2, 1, 1), (3, 1, 2, 2)])
def test_conv1d_f32_matches_torch(kw, s0, p0, d0):
    rng = np.random.default_rng(7 + kw + s0 + d0)
    B, IW, IC, OC = 2, 23, 16, 24
    w = (rng.standard_normal((OC, IC, kw)) * 0.1).astype(np.float32)
    b = rng.standard_normal(OC).astype(np.float32)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    got = oracle.conv1d(w, x, b, s0, p0, d0)
    ref = torch_conv(w, x, b, s0, p0, d0)
    assert got.shape == ref.shape
    # products of f32 values are exact in double: only the final f32 rounding differs
    assert rel(got, ref) < 1e-7


def test_conv1d_bf16_kernel_rounds_input():
    rng = np.random.default_rng(11)
    B, IW, IC, OC, KW = 2, 19, 32, 40, 3
    w = (rng.standard_normal((OC, IC, KW)) * 0.05).astype(np.float32)
    wb = oracle.f32_to_bf16_bits(w)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    got = oracle.conv1d(wb, x, None, 1, 1, 1, w_type=oracle.BF16)
    # ggml_mul_mat with a BF16 kernel rounds the im2col operand to bf16 (RNE)
    ref = torch_conv(oracle.bf16_bits_to_f32(wb), bf16_round(x), None, 1, 1, 1)
    assert rel(got, ref) < 1e-7
    # and without that rounding the result moves by ~1e-3
    assert rel(got, torch_conv(oracle.bf16_bits_to_f32(wb), x, None, 1, 1, 1)) > 1e-4


def test_conv_check_is_sensitive():
    rng = np.random.default_rng(3)
    B, IW, IC, OC, KW = 1, 15, 8, 8, 3
    w = rng.standard_normal((OC, IC, KW)).astype(np.float32)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    ref = torch_conv(w, x, None, 1, 1, 1)
    assert rel(oracle.conv1d(w, x), ref) < 1e-7
    flipped = oracle.conv1d(np.ascontiguousarray(w[:, :, ::-1]), x)
    swapped = oracle.conv1d(np.ascontiguousarray(w.reshape(OC, KW, IC).transpose(0, 2, 1)), x)
    assert rel(flipped, ref) > 0.1 and rel(swapped, ref) > 0.1


def test_swiglu_matches_torch():
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(4096) * 4).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    got = oracle.swiglu(a, b)
    ta = torch.from_numpy(a.astype(np.float64))
    ref = (F.silu(ta) * torch.from_numpy(b.astype(np.float64))).numpy()
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-30)) < 1e-6


def test_conv_mlp_swiglu_matches_torch():
    rng = np.random.default_rng(9)
    B, IW, IC, HID, OC = 2, 21, 16, 24, 16
    w1 = (rng.standard_normal((HID, IC, 3)) * 0.2).astype(np.float32)
    w3 = (rng.standard_normal((HID, IC, 3)) * 0.2).astype(np.float32)
    w2 = (rng.standard_normal((OC, HID, 3)) * 0.2).astype(np.float32)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    got = oracle.conv_mlp_swiglu(w1, w3, w2, x)
    h1 = torch.from_numpy(torch_conv(w1, x, None, 1, 1, 1))
    h3 = torch.from_numpy(torch_conv(w3, x, None, 1, 1, 1))
    ref = torch_conv(w2, (F.silu(h1) * h3).numpy(), None, 1, 1, 1)
    assert rel(got, ref) < 1e-6


def test_mlp_swiglu_matches_numpy():
    rng = np.random.default_rng(13)
    N, IC, HID, OC = 37, 16, 40, 24
    w1 = (rng.standard_normal((HID, IC)) * 0.2).astype(np.float32)
    w3 = (rng.standard_normal((HID, IC)) * 0.2).astype(np.float32)
    w2 = (rng.standard_normal((OC, HID)) * 0.2).astype(np.float32)
    x = rng.standard_normal((N, IC)).astype(np.float32)
    got = oracle.mlp_swiglu(w1, w3, w2, x)
    x64 = x.astype(np.float64)
    h1, h3 = x64 @ w1.T.astype(np.float64), x64 @ w3.T.astype(np.float64)
    ref = (h1 / (1 + np.exp(-h1)) * h3) @ w2.T.astype(np.float64)
    assert rel(got, ref) < 1e-6
