"""Pins the CPU oracle (oracle/tsk_oracle.c) against exact-arithmetic fixtures,
fp64 closed forms, special cases and brute force. CPU only."""
import os

import numpy as np
import pytest

import refmath
from conftest import rel_l2

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name))


# ---------------------------------------------------------------- conversions
def test_fp16_bf16_conversion_kat(orc):
    g = gold("conversions.npz")
    np.testing.assert_array_equal(orc.f32_to_f16_bits(g["x"]), g["f16_bits"])
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(g["x"]), g["bf16_bits"])
    # numpy's own IEEE half conversion agrees on every finite input
    np.testing.assert_array_equal(orc.f32_to_f16_bits(g["x"]), g["x"].astype(np.float16).view(np.uint16))


def test_fp16_roundtrip_all_codes(orc):
    codes = np.arange(65536, dtype=np.uint16)
    f = orc.f16_bits_to_f32(codes)
    finite = np.isfinite(f)
    np.testing.assert_array_equal(f[finite], codes[finite].view(np.float16).astype(np.float32))
    np.testing.assert_array_equal(orc.f32_to_f16_bits(f[finite]), codes[finite])


def test_bf16_roundtrip(orc):
    codes = np.arange(0, 65536, 7, dtype=np.uint16)
    f = orc.bf16_bits_to_f32(codes)
    finite = np.isfinite(f)
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(f[finite]), codes[finite])


# ---------------------------------------------------------------- Q8_0
def test_q8_0_dequant_kat(orc):
    g = gold("q8_0.npz")
    y = orc.dequantize_q8_0(g["kat_blocks"][:, None, :])
    np.testing.assert_array_equal(y, g["kat_deq"])


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_q8_0_quantize_kat(orc, mode):
    g = gold("q8_0.npz")
    blk = orc.quantize_q8_0(g["q_in"], mode)            # (rows, 1, 34)
    d_bits = blk[:, 0, :2].copy().view(np.uint16)[:, 0]
    qs = blk[:, 0, 2:].copy().view(np.int8)
    np.testing.assert_array_equal(d_bits, g["q_d_bits"][mode])
    np.testing.assert_array_equal(qs, g["q_qs"][mode])


def test_q8_0_modes_differ_only_on_ties(orc):
    g = gold("q8_0.npz")
    q0 = orc.quantize_q8_0(g["q_in"], 0)[:, 0, 2:].view(np.int8)
    q1 = orc.quantize_q8_0(g["q_in"], 1)[:, 0, 2:].view(np.int8)
    # block 0 holds exact .5 ties at d = 1: rne vs half-away
    assert list(q0[0, 1:5]) == [2, -2, 0, 0] and list(q1[0, 1:5]) == [3, -3, 1, -1]


def test_q8_0_mul_mat_brute_force(orc):
    rng = np.random.default_rng(7)
    M, K, N = 40, 256, 13
    w = (rng.standard_normal((M, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal((N, K)).astype(np.float32)
    wb = orc.quantize_q8_0(w, orc.Q8_GGUF_PY)
    y = orc.mul_mat(wb, x, a_type=orc.Q8_0)
    xb = orc.quantize_q8_0(x, orc.Q8_CPU_SIMD)
    exact = refmath.q8_0_matmul_exact(wb, xb)
    assert rel_l2(y, exact) < 1e-6
    # a mistake such as a transposed operand or dropped block scale fails this
    assert rel_l2(y, x @ w.T) < 2e-2


# ---------------------------------------------------------------- mul_mat
def test_mul_mat_bf16_fixture(orc):
    g = gold("mul_mat_bf16.npz")
    y = orc.mul_mat(g["w_bits"], g["x"], a_type=orc.BF16)
    assert rel_l2(y, g["y"]) < 1e-7


def test_mul_mat_f32_bias_and_batch(orc):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((17, 40)).astype(np.float32)
    x = rng.standard_normal((2, 3, 5, 40)).astype(np.float32)
    b = rng.standard_normal(17).astype(np.float32)
    y = orc.mul_mat(w, x, bias=b)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert rel_l2(y, ref) < 1e-7


def test_mul_mat_identity(orc):
    x = np.random.default_rng(4).standard_normal((6, 32)).astype(np.float32)
    eye = np.eye(32, dtype=np.float32)
    np.testing.assert_array_equal(orc.mul_mat(eye, x), x)
    eye_bf = (eye.view(np.uint32) >> 16).astype(np.uint16)
    y = orc.mul_mat(eye_bf, x, a_type=orc.BF16)
    np.testing.assert_array_equal(y, orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(x)))


# ---------------------------------------------------------------- attention
def test_attention_fixture_f32(orc):
    g = gold("attention.npz")
    o = orc.flash_attn_ext(g["q"], g["k"], g["v"], scale=0.125)
    assert rel_l2(o, g["out"]) < 1e-6


def test_attention_fixture_mask(orc):
    g = gold("attention.npz")
    o = orc.flash_attn_ext(g["q"], g["k"], g["v"], mask=g["mask"], scale=0.125)
    assert rel_l2(o, g["out_mask"]) < 1e-6


def test_attention_special_cases(orc):
    rng = np.random.default_rng(5)
    v = rng.standard_normal((1, 2, 1, 64)).astype(np.float32)
    q = rng.standard_normal((1, 2, 3, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 1, 64)).astype(np.float32)
    o = orc.flash_attn_ext(q, k, v)                           # one key: O = V
    np.testing.assert_allclose(o, np.broadcast_to(v.transpose(0, 2, 1, 3), o.shape), rtol=1e-6)
    k = rng.standard_normal((1, 2, 50, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 50, 64)).astype(np.float32)
    o = orc.flash_attn_ext(np.zeros_like(q), k, v)            # q = 0: mean of V
    np.testing.assert_allclose(o[0, 0], v[0].mean(axis=1), rtol=1e-5, atol=1e-6)
    o = orc.flash_attn_ext(q, k, np.ones_like(v))             # V = 1: O = 1
    np.testing.assert_allclose(o, 1.0, rtol=1e-6)
    perm = rng.permutation(50)                                # key permutation invariance
    o1 = orc.flash_attn_ext(q, k, v)
    o2 = orc.flash_attn_ext(q, k[:, :, perm], v[:, :, perm])
    np.testing.assert_allclose(o1, o2, rtol=1e-5, atol=1e-6)


def test_attention_f16_kv_and_gqa(orc):
    rng = np.random.default_rng(6)
    q = rng.standard_normal((2, 4, 33, 64)).astype(np.float32)
    k = rng.standard_normal((2, 2, 40, 64)).astype(np.float16)
    v = rng.standard_normal((2, 2, 40, 64)).astype(np.float16)
    o = orc.flash_attn_ext(q, k, v, scale=0.125)
    # ggml-cpu converts Q to F16 when K is F16; heads 0,1 share kv head 0
    qh = q.astype(np.float16).astype(np.float64)
    kk = np.repeat(k.astype(np.float64), 2, axis=1)
    vv = np.repeat(v.astype(np.float64), 2, axis=1)
    ref = refmath.attention(qh, kk, vv, 0.125).transpose(0, 2, 1, 3)
    assert rel_l2(o, ref) < 1e-6
    # the fp16 V accumulator of ggml-cpu stays within its fp16 error budget
    o16 = orc.flash_attn_ext(q, k, v, scale=0.125, vacc_f16=True)
    assert 1e-5 < rel_l2(o16, ref) < 3e-3


def test_attention_bf16_softcap_alibi(orc):
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 4, 10, 64)).astype(np.float32)
    kf = rng.standard_normal((1, 4, 12, 64)).astype(np.float32)
    vf = rng.standard_normal((1, 4, 12, 64)).astype(np.float32)
    kb, vb = orc.f32_to_bf16_bits(kf), orc.f32_to_bf16_bits(vf)
    mask = (rng.standard_normal((1, 1, 10, 12))).astype(np.float16)
    o = orc.flash_attn_ext(q, kb, vb, mask=mask, scale=0.125, max_bias=8.0, softcap=20.0,
                           kv_bf16=True)
    qd = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(q)).astype(np.float64)
    kd = orc.bf16_bits_to_f32(kb).astype(np.float64)
    vd = orc.bf16_bits_to_f32(vb).astype(np.float64)
    # ALiBi slopes for 4 heads, max_bias 8: 2^-2, 2^-4, 2^-6, 2^-8
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / 4) for h in range(4)])
    s = np.einsum("bhqd,bhkd->bhqk", qd, kd) * 0.125
    s = 20.0 * np.tanh(s / 20.0) + slopes[None, :, None, None] * mask.astype(np.float64)
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = np.einsum("bhqk,bhkd->bhqd", p / p.sum(-1, keepdims=True), vd).transpose(0, 2, 1, 3)
    assert rel_l2(o, ref) < 1e-6


def test_attention_fully_masked_row_is_zero(orc):
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 1, 2, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, 4, 64)).astype(np.float32)
    mask = np.zeros((1, 1, 2, 4), dtype=np.float16)
    mask[0, 0, 1, :] = -np.inf
    o = orc.flash_attn_ext(q, k, k, mask=mask)
    assert np.all(o[0, 1] == 0.0) and np.all(np.isfinite(o))


# ---------------------------------------------------------------- norms / rope
def test_rms_norm_and_norm_fixture(orc):
    g = gold("rope_norm.npz")
    assert rel_l2(orc.rms_norm_mul(g["x"], g["w"], 1e-6), g["rms"]) < 1e-6
    assert rel_l2(orc.norm(g["x"], 1e-5), g["ln"]) < 1e-6
    y = orc.rms_norm_mul(g["x"], None, 1e-6)                  # unit RMS
    np.testing.assert_allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, -1)), 1.0, rtol=1e-5)


def test_rope_fixture(orc):
    g = gold("rope_norm.npz")
    x, pos = g["x"], g["pos"]
    y = orc.rope_ext(x, pos, 64)
    # ggml's running-product angle vs the exact angle: |dtheta| <= ~(i+2) ulp(theta)
    # at |theta| <= 1039 rad, i.e. <= 2e-4 absolute per rotated value here.
    np.testing.assert_allclose(y, g["rope"], atol=3e-4 * np.abs(x).max())
    assert rel_l2(y, g["rope"]) < 2e-5
    yc = orc.rope_ext(x, pos, 64, freq_scale=194.0 / 72.0)
    assert rel_l2(yc, g["rope_clip"]) < 4e-5
    np.testing.assert_array_equal(y[0, 0], x[0, 0])           # position 0: identity
    pair = lambda a: np.hypot(a[..., 0::2].astype(np.float64), a[..., 1::2])
    np.testing.assert_allclose(pair(y), pair(x), rtol=2e-6)   # rotations keep pair norms


def test_rope_partial_dims_copy(orc):
    x = np.random.default_rng(2).standard_normal((1, 3, 2, 64)).astype(np.float32)
    y = orc.rope_ext(x, np.array([5, 6, 7], dtype=np.int32), 32)
    np.testing.assert_array_equal(y[..., 32:], x[..., 32:])
    assert not np.array_equal(y[..., :32], x[..., :32])


def test_gelu_closed_form():
    # fixed points of GELU(tanh): 0 -> 0; large x -> x; the value at 1 is known
    assert refmath.gelu_tanh(0.0) == 0.0
    assert abs(refmath.gelu_tanh(1.0) - 0.8411919906082768) < 1e-12


# ---------------------------------------------------------------- T5 (config 4)
def test_t5_bucket_closed_forms(orc):
    """src/t5_encoder.cpp:14-26 with 32 buckets, max distance 128: exact
    buckets below 8, one bucket per sign half, log-spaced above, clamped."""
    assert orc.t5_bucket(0) == 0
    for n in range(1, 8):
        assert orc.t5_bucket(-n) == n and orc.t5_bucket(n) == 16 + n
    # |rel| = 8 * 2^j lies exactly on bucket 8 + 2j (log(2^j) / log(16) = j / 4)
    for j in range(4):
        n = 8 << j
        assert orc.t5_bucket(-n) == 8 + 2 * j and orc.t5_bucket(n) == 24 + 2 * j
    for n in (128, 129, 1000, 10 ** 6):
        assert orc.t5_bucket(-n) == 15 and orc.t5_bucket(n) == 31


def test_t5_bucket_exact_integer_brute_force(orc):
    """for 8 <= n < 128 the log bucket is 8 + max{j : 16^j <= (n / 8)^8},
    decided here in exact integer arithmetic"""
    for n in range(8, 400):
        j = 0
        while 16 ** (j + 1) * 8 ** 8 <= n ** 8:
            j += 1
        want = min(8 + j, 15)
        assert orc.t5_bucket(-n) == want, n
        assert orc.t5_bucket(n) == 16 + want, n


def test_t5_attention_explicit_path_vs_fp64(orc):
    """the reference's scores / add / soft_max / P.V chain (t5_encoder.cpp:68-75)
    against an fp64 softmax with the same additive mask; padded keys get no weight"""
    rng = np.random.default_rng(44)
    n, H, D = 37, 3, 64
    q, k, v = (rng.standard_normal((n, H, D)).astype(np.float32) * 0.3 for _ in range(3))
    rel_bias = rng.standard_normal((32, H)).astype(np.float32)
    ids = np.ones(n, np.int32)
    ids[-5:] = 0
    mask = orc.t5_attention_mask(rel_bias, ids)
    # mask structure: bias depends only on k - q, padded keys are -inf
    assert np.all(np.isneginf(mask[:, :, -5:]))
    assert mask[1, 3, 7] == rel_bias[orc.t5_bucket(4), 1] and mask[2, 10, 2] == rel_bias[orc.t5_bucket(-8), 2]
    o = orc.t5_attention(q, k, v, mask)
    s = np.einsum("qhd,khd->hqk", q.astype(np.float64), k.astype(np.float64)) + mask.astype(np.float64)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("hqk,khd->qhd", p, v.astype(np.float64))
    assert rel_l2(o, ref) <= 1e-6
    # keys past the padding never contribute: changing them changes nothing
    v2 = v.copy()
    v2[-5:] = 1e3
    np.testing.assert_array_equal(orc.t5_attention(q, k, v2, mask), o)
