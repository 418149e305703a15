"""The Oobleck VAE decoder on gfx950 (tsk_vae_*, ts_vae::decode,
src/vae_decoder.cpp:62-124) against the oracle's restatement (pinned against
torch's Conv1d / ConvTranspose1d in test_oracle_vae.py).

Every convolution is F32 on both sides, and the device runs the transposed
convolutions as 3-tap phase convolutions instead of the reference's
zero-stuffed ones -- the same nonzero products. The two differ by fp32
rounding only: the device accumulates each output in one fp32 chain of MFMA
steps (K up to 7 x 2048 = 14336 terms, 3584 steps), the oracle sums in
double. At the reference's channel counts that is a few 1e-5 of the audio
(torch's own fp32 decode on the CPU differs from fp64 by 2.0e-5 on the same
weights and latent; the device measured 5.9e-5); with 4 .. 12 channels
~1e-5. Bound 2e-4 rel-L2; a wrong phase, tap or padding of a transposed
convolution moves the audio by more than 0.3 (test_oracle_vae.py). Snake
parameters N(0, 0.1): larger ones amplify fp32 rounding further."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 2e-4


@pytest.fixture(scope="module")
def env(orc):
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    return tsk, orc


def build_pair(tsk, orc, seed=77, **kw):
    v = tsk.Vae(tsk.vae_config(**kw))
    ov = orc.OracleVae(orc.vae_config(**kw))
    assert v.tensors() == ov.tensors()
    W = tsk.vae_synthetic_weights(v.tensors(), seed=seed, snake_std=0.1)
    for k, w in W.items():
        v.set_tensor(k, w)
        ov.set_tensor(k, w)
    return v, ov


@pytest.mark.parametrize("T", [1, 2, 5])
def test_vae_small_channels(env, T):
    """narrow channels (4 .. 12), the reference's strides"""
    tsk, orc = env
    v, ov = build_pair(tsk, orc, latent_dim=8, channels=4, c_mults=[1, 2, 2, 3, 3], max_latent=8)
    lat = np.random.default_rng(T).standard_normal((8, T)).astype(np.float32)
    a = v.decode(lat)
    r = ov.decode(lat)
    e = rel_l2(a, r)
    print(f"VAE (channels 4..12) T={T}: rel-L2 {e:.3e}", flush=True)
    assert a.shape == (2, T * 2048) and e <= TOL
    v.close()


def test_vae_reference_channels(env):
    """the reference's decoder (64 -> 2048 -> 1024 -> 512 -> 256 -> 128 -> 128
    channels, strides 8 8 4 4 2) on 3 latent frames (6144 samples)"""
    tsk, orc = env
    v, ov = build_pair(tsk, orc, max_latent=16)
    lat = np.random.default_rng(3).standard_normal((64, 3)).astype(np.float32)
    a = v.decode(lat)
    r = ov.decode(lat)
    e = rel_l2(a, r)
    print(f"VAE (reference channels) T=3: rel-L2 {e:.3e}, audio rms {np.sqrt((r ** 2).mean()):.3f}", flush=True)
    assert a.shape == (2, 6144) and e <= TOL
    # device entry point: the same bits
    lat_d = tsk.to_device(lat)
    out = tsk.empty((2, 6144))
    v.decode_device(lat_d, out)
    tsk.synchronize()
    assert np.array_equal(out.numpy(), a)
    # a longer latent (16 frames, 32768 samples): finite, deterministic, and
    # its first frames' audio independent of what follows only through the
    # receptive field -- checked against the oracle on the same input
    lat16 = np.random.default_rng(4).standard_normal((64, 16)).astype(np.float32)
    a16 = v.decode(lat16)
    assert np.isfinite(a16).all() and np.array_equal(v.decode(lat16), a16)
    e16 = rel_l2(a16, ov.decode(lat16))
    print(f"VAE (reference channels) T=16: rel-L2 {e16:.3e}", flush=True)
    assert e16 <= TOL
    with pytest.raises(tsk.TskError):
        v.decode(np.zeros((64, 17), np.float32))          # beyond max_latent
    v.close()


def test_vae_split_products(env, monkeypatch):
    """The opt-in split products (TSK_VAE_SPLIT=1 when the model is created:
    every convolution but the output one as three bf16 products over weight
    planes [hi | lo | hi] and input planes [hi | hi | lo], which the previous
    convolution's epilogue writes with its SnakeBeta): about 2^-17 of |x w|
    per term, which the decoder amplifies 50-100 times on its way to the audio
    (fp32 products: ~6e-5 from the oracle), so the audio is held to 1e-3;
    TSK_VAE_SPLIT=0 on the same model (read on every call) is the fp32 path
    again, held to TOL. The split planes' layout is checked by the same
    comparison: a plane in the wrong place moves the audio by O(1)."""
    tsk, orc = env
    monkeypatch.setenv("TSK_VAE_SPLIT", "1")
    tsk.init(0, reread=True)
    try:
        v, ov = build_pair(tsk, orc, max_latent=16)
        for T, seed in ((3, 3), (16, 4)):
            lat = np.random.default_rng(seed).standard_normal((64, T)).astype(np.float32)
            r = ov.decode(lat)
            a = v.decode(lat)
            assert np.isfinite(a).all() and np.array_equal(v.decode(lat), a)
            e = rel_l2(a, r)
            monkeypatch.setenv("TSK_VAE_SPLIT", "0")
            tsk.init(0, reread=True)
            ex = rel_l2(v.decode(lat), r)
            monkeypatch.setenv("TSK_VAE_SPLIT", "1")
            tsk.init(0, reread=True)
            print(f"VAE (reference channels) T={T}: split products rel-L2 {e:.3e}, fp32 products {ex:.3e}",
                  flush=True)
            assert e <= 1e-3 and ex <= TOL
        v.close()
    finally:
        monkeypatch.delenv("TSK_VAE_SPLIT", raising=False)
        tsk.init(0, reread=True)
