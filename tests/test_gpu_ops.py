"""rms_norm*w, norm, rope_ext and the fused QK-RMSNorm+RoPE prologue on
gfx950 vs the oracle (fp32 paths rel-L2 <= 1e-5)."""
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


def test_rms_norm_mul(env):
    tsk, orc = env
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 420, 16, 64)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(64)).astype(np.float32)
    y = tsk.rms_norm_mul(tsk.to_device(x), tsk.to_device(w), 1e-6).numpy()
    assert rel_l2(y, orc.rms_norm_mul(x, w, 1e-6)) <= 1e-6
    x2 = rng.standard_normal((5, 1024)).astype(np.float32) * 3 + 1
    w2 = np.ones(1024, np.float32)
    y2 = tsk.rms_norm_mul(tsk.to_device(x2), tsk.to_device(w2), 1e-6).numpy()
    assert rel_l2(y2, orc.rms_norm_mul(x2, w2, 1e-6)) <= 1e-6


def test_norm(env):
    tsk, orc = env
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((388, 1024)) * 2 + 0.5).astype(np.float32)
    x[3] = 0.25                                                # constant row (padding token case)
    y = tsk.norm(tsk.to_device(x), 1e-5).numpy()
    assert rel_l2(y, orc.norm(x, 1e-5)) <= 1e-5


@pytest.mark.parametrize("S,fscale", [(646, 1.0), (194, 1.0), (72, 194.0 / 72.0), (1040, 1.0)])
def test_rope_ext(env, S, fscale):
    tsk, orc = env
    rng = np.random.default_rng(S)
    x = rng.standard_normal((1, S, 16, 64)).astype(np.float32)
    pos = np.arange(S, dtype=np.int32)
    y = tsk.rope_ext(tsk.to_device(x), tsk.to_device(pos), 64, freq_scale=fscale)
    assert rel_l2(y.numpy(), orc.rope_ext(x, pos, 64, freq_scale=fscale)) <= 1e-5


def test_qk_norm_rope(env):
    tsk, orc = env
    rng = np.random.default_rng(3)
    S = 646
    x = rng.standard_normal((2, S, 16, 64)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(64)).astype(np.float32)
    pos = np.arange(S, dtype=np.int32)
    y = tsk.qk_norm_rope(tsk.to_device(x), tsk.to_device(w),
                         tsk.to_device(pos)).numpy()
    ref = orc.rope_ext(orc.rms_norm_mul(x, w, 1e-6), pos, 64)
    assert rel_l2(y, ref) <= 1e-5
    # text stream: no rope (pos == NULL)
    y2 = tsk.qk_norm_rope(tsk.to_device(x), tsk.to_device(w), None).numpy()
    assert rel_l2(y2, orc.rms_norm_mul(x, w, 1e-6)) <= 1e-6
    # bf16 in / out
    xbits = orc.f32_to_bf16_bits(x)
    yb = orc.bf16_bits_to_f32(tsk.qk_norm_rope(tsk.bf16_to_device(xbits), tsk.to_device(w), tsk.to_device(pos)).numpy())
    refb = orc.rope_ext(orc.rms_norm_mul(orc.bf16_bits_to_f32(xbits), w, 1e-6), pos, 64)
    assert rel_l2(yb, refb) <= 5e-3
