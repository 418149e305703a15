"""Convolution and SwiGLU nodes of the reference graph (src/mmdit.cpp:20-52) on
gfx950 through the C ABI, against the oracle (oracle/tsk_oracle_conv.c).

Tolerances (rel-L2 against the oracle, which sums in double):
- im2col: bit-exact (F32; F16 / BF16 = the RNE conversion of the F32 values);
- BF16 kernels: 2e-5 -- both sides round the input to bf16 and multiply
  exactly, only the fp32 summation order differs; a missing bf16 rounding
  of the input shows up at ~1e-3;
- F32 kernels: 1e-5 (all-fp32 products and sums);
- SwiGLU MLPs with BF16 kernels: 3e-4 -- the hidden state is rounded to bf16
  before w2 on both sides, and fp32-order differences of ~1e-6 flip that
  rounding by one bf16 ulp on a few elements in 10^4.
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env(orc):
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    return tsk, orc


def kernel(orc, rng, oc, ic, kw, scale=0.02, bf16=True):
    w = (rng.standard_normal((oc, ic, kw)) * scale).astype(np.float32)
    return orc.f32_to_bf16_bits(w) if bf16 else w


# ------------------------------------------------------------------ im2col
@pytest.mark.parametrize("kw,s0,p0,d0", [(3, 1, 1, 1), (7, 1, 3, 1), (3, 2, 1, 1), (3, 1, 2, 2)])
def test_im2col_bit_exact(env, kw, s0, p0, d0):
    tsk, orc = env
    rng = np.random.default_rng(kw * 10 + s0 + d0)
    N, IC, IW = 2, 64, 97
    x = rng.standard_normal((N, IC, IW)).astype(np.float32)
    ref = orc.im2col_1d(x, kw, s0, p0, d0)
    got = tsk.im2col_1d((8, IC, kw), tsk.to_device(x), s0, p0, d0).numpy()
    assert np.array_equal(got, ref)


def test_im2col_of_transposed_view_and_16bit_outputs(env):
    """conv1d_f32's operand: ggml_transpose of a channels-fastest [IC, S] tensor."""
    tsk, orc = env
    rng = np.random.default_rng(5)
    N, S, IC = 2, 194, 128
    xs = rng.standard_normal((N, S, IC)).astype(np.float32)      # channels fastest
    xd = tsk.to_device(xs)
    view = xd.view(0, (N, IC, S), (S * IC, 1, IC))                # (N, IC, IW) over the same memory
    ref = orc.im2col_1d(np.ascontiguousarray(xs.transpose(0, 2, 1)), 3)
    assert np.array_equal(tsk.im2col_1d((1, IC, 3), view).numpy(), ref)
    bf = tsk.im2col_1d((1, IC, 3), view, out_dtype="bf16").numpy()
    assert np.array_equal(bf, orc.f32_to_bf16_bits(ref))
    hf = tsk.im2col_1d((1, IC, 3), view, out_dtype="f16").numpy()
    assert np.array_equal(hf.view(np.uint16), ref.astype(np.float16).view(np.uint16))


# ------------------------------------------------------------------ conv_cl
# (B, IW, IC, OC, KW, s0, p0, d0): the reference graph's convolutions
# (latent/clip linear1 and convMLP k3, audio_input_proj k3 from 64 channels,
# sync / final-layer k7) plus stride, dilation and ragged edges
CONV_SHAPES = [
    (2, 194, 1024, 1024, 3, 1, 1, 1),
    (2, 646, 1024, 2816, 3, 1, 1, 1),
    (2, 194, 2816, 1024, 3, 1, 1, 1),
    (2, 194, 64, 1024, 3, 1, 1, 1),
    (2, 194, 1024, 64, 7, 1, 3, 1),
    (1, 72, 768, 1024, 7, 1, 3, 1),
    (2, 33, 40, 68, 3, 2, 1, 1),
    (1, 50, 16, 24, 3, 1, 2, 2),
    (3, 1, 8, 12, 3, 1, 1, 1),
    (1, 2, 8, 4, 3, 1, 1, 1),
]


@pytest.mark.parametrize("B,IW,IC,OC,KW,s0,p0,d0", CONV_SHAPES)
def test_conv1d_bf16(env, B, IW, IC, OC, KW, s0, p0, d0):
    tsk, orc = env
    rng = np.random.default_rng(B * 1000 + IW + OC + KW)
    w = kernel(orc, rng, OC, IC, KW)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    bias = rng.standard_normal(OC).astype(np.float32) if OC % 4 == 0 else None
    ref = orc.conv1d(w, x, bias, s0, p0, d0, w_type=orc.BF16)
    wd, xd = tsk.bf16_to_device(w), tsk.to_device(x)
    bd = tsk.to_device(bias) if bias is not None else None
    got = tsk.conv1d(wd, xd, bd, s0, p0, d0).numpy()          # ggml layout: packed per call
    assert got.shape == ref.shape
    assert rel_l2(got, ref) <= 2e-5
    packed = tsk.conv1d_pack_weight(wd)                       # kw-major: read in place
    got2 = tsk.conv1d(packed, xd, bd, s0, p0, d0).numpy()
    assert np.array_equal(got, got2)


def test_conv1d_bf16_io_and_determinism(env):
    tsk, orc = env
    rng = np.random.default_rng(21)
    B, IW, IC, OC = 2, 194, 1024, 1024
    w = kernel(orc, rng, OC, IC, 3)
    xb = orc.f32_to_bf16_bits(rng.standard_normal((B, IW, IC)).astype(np.float32))
    ref = orc.conv1d(w, orc.bf16_bits_to_f32(xb), None, w_type=orc.BF16)
    wd = tsk.conv1d_pack_weight(tsk.bf16_to_device(w))
    xd = tsk.bf16_to_device(xb)
    y = tsk.conv1d(wd, xd, out_dtype="bf16").numpy()
    assert rel_l2(orc.bf16_bits_to_f32(y), ref) <= 5e-3
    a = tsk.conv1d(wd, xd).numpy()
    b = tsk.conv1d(wd, xd).numpy()
    assert np.array_equal(a, b)
    assert rel_l2(a, ref) <= 2e-5


def test_conv1d_input_rounding_is_pinned(env):
    """The tolerance separates ggml's bf16 rounding of the input from none."""
    tsk, orc = env
    rng = np.random.default_rng(8)
    w = kernel(orc, rng, 256, 512, 3)
    x = rng.standard_normal((1, 100, 512)).astype(np.float32)
    got = tsk.conv1d(tsk.bf16_to_device(w), tsk.to_device(x)).numpy()
    unrounded = orc.conv1d(orc.bf16_bits_to_f32(w), x)       # F32 kernel: no input rounding
    assert rel_l2(got, unrounded) > 2e-4
    assert rel_l2(got, orc.conv1d(w, x, w_type=orc.BF16)) <= 2e-5


@pytest.mark.parametrize("B,IW,IC,OC,KW,s0,p0,d0", [(2, 194, 1024, 1024, 3, 1, 1, 1), (1, 60, 64, 1024, 3, 1, 1, 1),
                                                    (2, 50, 256, 64, 7, 1, 3, 1), (1, 33, 40, 68, 3, 2, 1, 2)])
def test_conv1d_f32_kernel(env, B, IW, IC, OC, KW, s0, p0, d0):
    """The Q8_0 DiT keeps its 3-D kernels in F32: all-fp32 arithmetic."""
    tsk, orc = env
    rng = np.random.default_rng(IW + OC)
    w = kernel(orc, rng, OC, IC, KW, bf16=False)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    bias = rng.standard_normal(OC).astype(np.float32) if OC % 4 == 0 else None
    ref = orc.conv1d(w, x, bias, s0, p0, d0)
    got = tsk.conv1d(tsk.to_device(w), tsk.to_device(x), tsk.to_device(bias) if bias is not None else None,
                     s0, p0, d0).numpy()
    assert rel_l2(got, ref) <= 1e-5


@pytest.mark.parametrize("N,K,M", [(388, 1024, 1024), (154, 1024, 2816), (77, 768, 1024), (7, 40, 12),
                                   (646, 3072, 1024)])
def test_mul_mat_f32_weights(env, N, K, M):
    tsk, orc = env
    rng = np.random.default_rng(N + K + M)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((N, K)).astype(np.float32)
    bias = rng.standard_normal(M).astype(np.float32) if M % 4 == 0 else None
    y = tsk.mul_mat(tsk.to_device(w), tsk.to_device(x), bias=tsk.to_device(bias) if bias is not None else None)
    ref = orc.mul_mat(w, x, bias=bias)
    assert rel_l2(y.numpy(), ref) <= 1e-5


# ------------------------------------------------------------------ SwiGLU
def test_swiglu_elementwise(env):
    tsk, orc = env
    rng = np.random.default_rng(3)
    a = (rng.standard_normal((646, 2816)) * 4).astype(np.float32)
    b = rng.standard_normal((646, 2816)).astype(np.float32)
    got = tsk.swiglu(tsk.to_device(a), tsk.to_device(b)).numpy()
    ref = orc.swiglu(a, b)
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-30)) <= 2e-6


@pytest.mark.parametrize("B,IW,IC,HID,OC", [(2, 194, 1024, 2816, 1024), (1, 72, 1024, 2816, 1024),
                                            (2, 37, 64, 40, 24)])
def test_conv_mlp_swiglu_bf16(env, B, IW, IC, HID, OC):
    tsk, orc = env
    rng = np.random.default_rng(IW + HID)
    w1, w3 = kernel(orc, rng, HID, IC, 3), kernel(orc, rng, HID, IC, 3)
    w2 = kernel(orc, rng, OC, HID, 3)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    ref = orc.conv_mlp_swiglu(w1, w3, w2, x, w_type=orc.BF16)
    d1, d3, d2 = (tsk.bf16_to_device(w) for w in (w1, w3, w2))
    xd = tsk.to_device(x)
    got = tsk.conv_mlp_swiglu(d1, d3, d2, xd).numpy()
    assert rel_l2(got, ref) <= 3e-4
    p1, p3, p2 = (tsk.conv1d_pack_weight(d) for d in (d1, d3, d2))
    assert np.array_equal(tsk.conv_mlp_swiglu(p1, p3, p2, xd).numpy(), got)


def test_conv_mlp_swiglu_128x128_tiles(env, monkeypatch):
    """The reference graph's 30 s convMLP (B = 2, 646 positions, 1024 -> 2816
    -> 1024, k3) runs its w1 / w3 GEMM on 128 x 128 tiles (484 of them): the
    oracle bound, and the same bits as 128 x 64 tiles (TSK_COOP_CFG=29: the
    tile shape changes no summation order)."""
    tsk, orc = env
    rng = np.random.default_rng(646)
    B, IW, IC, HID, OC = 2, 646, 1024, 2816, 1024
    w1, w3 = kernel(orc, rng, HID, IC, 3), kernel(orc, rng, HID, IC, 3)
    w2 = kernel(orc, rng, OC, HID, 3)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    ds = [tsk.conv1d_pack_weight(tsk.bf16_to_device(w)) for w in (w1, w3, w2)]
    xd = tsk.to_device(x)
    got = tsk.conv_mlp_swiglu(*ds, xd).numpy()
    try:
        monkeypatch.setenv("TSK_COOP_CFG", "29")
        tsk.init(0, reread=True)
        narrow = tsk.conv_mlp_swiglu(*ds, xd).numpy()
    finally:
        monkeypatch.delenv("TSK_COOP_CFG", raising=False)
        tsk.init(0, reread=True)
    assert np.array_equal(got, narrow)
    ref = orc.conv_mlp_swiglu(w1, w3, w2, x, w_type=orc.BF16)
    assert rel_l2(got, ref) <= 3e-4


def test_conv_mlp_swiglu_f32(env):
    tsk, orc = env
    rng = np.random.default_rng(17)
    B, IW, IC, HID, OC = 2, 100, 256, 512, 256
    w1, w3 = kernel(orc, rng, HID, IC, 3, bf16=False), kernel(orc, rng, HID, IC, 3, bf16=False)
    w2 = kernel(orc, rng, OC, HID, 3, bf16=False)
    x = rng.standard_normal((B, IW, IC)).astype(np.float32)
    ref = orc.conv_mlp_swiglu(w1, w3, w2, x)
    got = tsk.conv_mlp_swiglu(*(tsk.to_device(w) for w in (w1, w3, w2)), tsk.to_device(x)).numpy()
    assert rel_l2(got, ref) <= 1e-5


@pytest.mark.parametrize("bf16", [True, False])
def test_mlp_swiglu(env, bf16):
    """text stream: mlp over 2 x 77 tokens, 1024 -> 2816 -> 1024"""
    tsk, orc = env
    rng = np.random.default_rng(29 + bf16)
    N, IC, HID, OC = 154, 1024, 2816, 1024

    def mat(m, k):
        w = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
        return orc.f32_to_bf16_bits(w) if bf16 else w

    w1, w3, w2 = mat(HID, IC), mat(HID, IC), mat(OC, HID)
    x = rng.standard_normal((2, 77, IC)).astype(np.float32)
    ref = orc.mlp_swiglu(w1, w3, w2, x, w_type=orc.BF16 if bf16 else orc.F32)
    dev = tsk.bf16_to_device if bf16 else tsk.to_device
    got = tsk.mlp_swiglu(dev(w1), dev(w3), dev(w2), tsk.to_device(x)).numpy()
    assert got.shape == (2, 77, OC)
    assert rel_l2(got, ref) <= (3e-4 if bf16 else 1e-5)
