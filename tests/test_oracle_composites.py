"""Independent pins of the oracle's composite functions: the flow step and
sampler (orc_dit_forward / orc_dit_sample, restating src/mmdit.cpp:119-376)
and the T5 encoder layers (orc_t5_encode_range, src/t5_encoder.cpp:40-104),
each against the fp64 restatement in refmath.py written from the reference's
graph, plus orc_gelu_tanh against its closed form.

The oracle runs here in its all-fp32 mode (F32 activations, F32 K / V, F32
weights), so oracle and restatement differ only by fp32 rounding of
intermediates (~6e-8 per operation; measured 1e-7 .. 5e-7): tolerance
1e-6 rel-L2. Each structural mistake a composition could make -- shift / scale chunks swapped, a text
stream that is never updated, the wrong gate on the MLP branch, RoPE on the
text tokens, the step size of the wrong sign, a missing relative-position
bias -- moves the result by more than 1e-2, so it cannot pass. (The last
joint block's text stream is pre_only: its output is never read again, so
its post-attention half has no observable effect and no weights.)"""
import numpy as np
import pytest

import refmath
from conftest import rel_l2

TOL = 1e-6
SMALL = dict(hidden=128, n_head=2, head_dim=64, depth=3, fused_depth=1, latent_dim=16, text_seq=9,
             mlp_hidden=256, max_batch=2, max_latent=32, rope_theta=10000.0, t_max_period=1.0,
             ln_eps=1e-5, qk_eps=1e-6)


def weights(names, seed, std=0.05):
    """random weights (matrices std, biases std, norm weights 1 + std) so that
    every block moves the residual streams measurably"""
    out = {}
    for i, (name, ne) in enumerate(names):
        rng = np.random.default_rng([seed, i])
        w = (rng.standard_normal(int(ne[0]) * int(ne[1])) * std).astype(np.float32)
        if name.endswith("norm.weight"):
            w += 1.0
        out[name] = w.reshape(int(ne[1]), int(ne[0])) if ne[1] > 1 else w
    return out


@pytest.fixture(scope="module")
def small_dit(orc):
    cfg = orc.dit_config(**{k: v for k, v in SMALL.items()})
    od = orc.OracleDiT(cfg)
    W = weights(od.tensors(), 7)
    for k, v in W.items():
        od.set_tensor(k, v)
    return od, W


def inputs(T=17, seed=3):
    rng = np.random.default_rng(seed)
    lat = rng.standard_normal((T, SMALL["latent_dim"])).astype(np.float32)
    txt = rng.standard_normal((SMALL["text_seq"], SMALL["hidden"])).astype(np.float32)
    return lat, txt


def test_gelu_tanh_closed_form(orc):
    x = np.linspace(-10.0, 10.0, 4001).astype(np.float32)
    got = orc.gelu_tanh(x).astype(np.float64)
    want = refmath.gelu_tanh(x.astype(np.float64))
    err = np.abs(got - want) / np.maximum(np.abs(want), 1e-30)
    big = np.abs(want) > 1e-3
    assert err[big].max() < 2e-6, err[big].max()
    assert np.abs(got - want).max() < 1e-6
    # odd part and limits: gelu(x) - gelu(-x) = x, gelu(10) = 10, gelu(-10) = 0
    assert np.allclose(got - orc.gelu_tanh(-x).astype(np.float64), x, atol=4e-6)
    assert got[-1] == np.float32(10.0) and abs(got[0]) < 1e-20


@pytest.mark.parametrize("t", [1.0, 0.37, 0.0])
def test_dit_forward_matches_fp64_restatement(small_dit, t):
    od, W = small_dit
    lat, txt = inputs()
    got = od.forward(lat[None], np.array([t], np.float32), txt[None], act_bf16=False, kv_f16=False)[0]
    want = refmath.dit_forward_ref(W, SMALL, lat, t, txt)
    e = rel_l2(got, want)
    print(f"oracle flow step vs fp64 restatement (t = {t}): rel-L2 {e:.2e}")
    assert e <= TOL


def test_dit_forward_batch_rows_independent(small_dit):
    od, W = small_dit
    lat, txt = inputs()
    lat2, txt2 = inputs(seed=4)
    got = od.forward(np.stack([lat, lat2]), np.array([0.8, 0.2], np.float32), np.stack([txt, txt2]),
                     act_bf16=False, kv_f16=False)
    assert rel_l2(got[1], refmath.dit_forward_ref(W, SMALL, lat2, 0.2, txt2)) <= TOL


@pytest.mark.parametrize("mistake", [dict(swap_shift_scale=True), dict(text_frozen=True),
                                     dict(gate_mlp_index=2), dict(rope_text=True)])
def test_dit_restatement_detects_structural_mistakes(small_dit, mistake):
    """each planted mistake moves the fp64 restatement far outside TOL from the oracle"""
    od, W = small_dit
    lat, txt = inputs()
    got = od.forward(lat[None], np.array([0.6], np.float32), txt[None], act_bf16=False, kv_f16=False)[0]
    wrong = refmath.dit_forward_ref(W, SMALL, lat, 0.6, txt, **mistake)
    e = rel_l2(got, wrong)
    print(f"planted {mistake}: rel-L2 {e:.2e}")
    assert e > 100 * TOL


def test_dit_sample_matches_fp64_restatement(small_dit):
    od, W = small_dit
    rng = np.random.default_rng(11)
    noise = rng.standard_normal((13, SMALL["latent_dim"])).astype(np.float32)
    tc = rng.standard_normal((SMALL["text_seq"], SMALL["hidden"])).astype(np.float32)
    tu = rng.standard_normal((SMALL["text_seq"], SMALL["hidden"])).astype(np.float32)
    x, f0 = od.sample(noise, tc, tu, steps=3, cfg_scale=5.0, act_bf16=False, kv_f16=False)
    rx, rf0 = refmath.dit_sample_ref(W, SMALL, noise, tc, tu, 3, 5.0)
    e0, ex = rel_l2(f0, rf0), rel_l2(x, rx)
    print(f"oracle sampler vs fp64 restatement: flow0 {e0:.2e}, latent {ex:.2e}")
    assert e0 <= TOL and ex <= TOL
    # an Euler step of the wrong sign is far off
    wrong = np.asarray(noise, np.float64) - (rx - noise)
    assert rel_l2(x, wrong) > 100 * TOL


T5_SMALL = dict(d_model=128, d_ff=192, n_layers=2, n_heads=2, d_kv=64, rel_buckets=32, rel_max_dist=128,
                max_tokens=160, eps=1e-6)


def test_t5_bucket_restatement_matches_oracle(orc):
    for r in range(-400, 401):
        assert orc.t5_bucket(r) == refmath.t5_bucket_ref(r), r


@pytest.mark.parametrize("n", [40, 150])
def test_t5_encode_matches_fp64_restatement(orc, n):
    cfg = orc.t5_config(weight_type=orc.F32, **T5_SMALL)
    ot = orc.OracleT5(cfg)
    rng = np.random.default_rng(n)
    W = {}
    for name, ne, ty in ot.tensors():
        if name == "rel_bias":
            w = rng.standard_normal((ne[1], ne[0])).astype(np.float32)
        elif name.endswith("norm"):
            w = (1.0 + 0.1 * rng.standard_normal(ne[0])).astype(np.float32)
        else:
            w = (rng.standard_normal((ne[1], ne[0])) / np.sqrt(ne[0])).astype(np.float32)
            if name.endswith(".q") or name.endswith(".k"):
                w *= np.float32(8.0 ** -0.5)
        W[name] = w
        ot.set_tensor(name, w)
    x = rng.standard_normal((n, T5_SMALL["d_model"])).astype(np.float32)
    ids = np.arange(1, n + 1, dtype=np.int32)
    ids[-n // 5:] = 0
    got = ot.encode(x, ids)
    want = refmath.t5_encode_ref(W, T5_SMALL, x, ids)
    e = rel_l2(got, want)
    print(f"oracle T5 (n = {n}) vs fp64 restatement: rel-L2 {e:.2e}")
    assert e <= TOL
    # without the relative-position bias the result is far off
    Wz = dict(W, rel_bias=np.zeros_like(W["rel_bias"]))
    assert rel_l2(got, refmath.t5_encode_ref(Wz, T5_SMALL, x, ids)) > 100 * TOL
