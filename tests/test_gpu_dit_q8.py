"""The Q8_0 MM-DiT driver (tsk_dit_config.weight_type = Q8_0): the block
projections (attn.qkv, linear1, ffn.fc1, ffn.fc2) are ggml Q8_0 weights and
every activation they read is quantized to Q8_0 first, so each product is
ggml's Q8_0 x Q8_0 vec_dot (exact int32 block sums, fp32 scaling); the rest
of the step is the BF16 driver's. Compared with the oracle's restatement run
with the same Q8_0 blocks.

Both sides quantize activations with the x86 rule (d = amax / 127 as fp16,
q = rne(x 127 / amax)); an activation that lands within an ulp of a rounding
boundary can round differently when its fp32 value differs by summation
order, so each flow step is checked against max(2e-3, 2 x the oracle's own
change under a one-ulp (1e-7 relative) change of its input latent)."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
Q8_0 = 8


@pytest.fixture(scope="module")
def env(orc):
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    return tsk, orc


def build_q8_pair(tsk, orc, seed=1234, raw=True, **kw):
    """driver + oracle with the same weights; the Q8_0 projections as ggml
    blocks from ggml's reference quantizer (raw) or quantized by each side from
    the same f32 values"""
    kw = dict(kw, weight_type=Q8_0)
    dit = tsk.Dit(tsk.dit_config(**kw))
    od = orc.OracleDiT(orc.dit_config(**kw))
    names = dit.tensors()
    assert names == od.tensors()
    types = dit.tensor_types()
    W = tsk.synthetic_weights(names, seed=seed)
    for k, v in W.items():
        if types[k] == Q8_0 and raw:
            blocks = orc.quantize_q8_0(v, orc.Q8_CPU_REF)
            dit.set_tensor_q8_0(k, blocks)
            od.set_tensor_q8_0(k, blocks)
        else:
            dit.set_tensor(k, v)
            od.set_tensor(k, v)
    return dit, od, W, types


def inputs(B, T, seed=4242, t=0.5):
    rng = np.random.default_rng(seed)
    lat = rng.standard_normal((B, T, 64), dtype=np.float32)
    txt = rng.standard_normal((B, 77, 1024), dtype=np.float32)
    return lat, np.full(B, t, np.float32), txt


def cm(lat):
    return np.ascontiguousarray(lat.transpose(0, 2, 1))


def one_ulp_sensitivity(od, lat, t, txt, seed=99):
    rng = np.random.default_rng(seed)
    ref = od.forward(lat, t, txt, act_bf16=True, kv_f16=True)
    pert = (lat * (1 + 1e-7 * rng.standard_normal(lat.shape))).astype(np.float32)
    return ref, rel_l2(od.forward(pert, t, txt, act_bf16=True, kv_f16=True), ref)


def test_q8_types_and_host_quantizer(env):
    """exactly the four block projections are Q8_0, and tsk_dit_set_tensor's
    host quantization of f32 weights is ggml's reference quantizer bit for
    bit (same forward output as uploading its blocks)"""
    tsk, orc = env
    kw = dict(depth=2, fused_depth=1, max_latent=64)
    a, _, W, types = build_q8_pair(tsk, orc, raw=True, **kw)
    b, _, _, _ = build_q8_pair(tsk, orc, raw=False, **kw)
    q8 = sorted(k for k, ty in types.items() if ty == Q8_0)
    assert q8 and all(any(k.endswith(s) for s in (".attn.qkv.weight", ".linear1.weight", ".ffn.fc1.weight",
                                                   ".ffn.fc2.weight")) for k in q8)
    assert len(q8) == 4 + 1 + 4              # joint latent, joint text (pre_only: qkv only), fused
    lat, t, txt = inputs(2, 40)
    assert np.array_equal(a.forward(cm(lat), t, txt), b.forward(cm(lat), t, txt))
    with pytest.raises(tsk.TskError):
        a.set_tensor_q8_0("t_embed.mlp.0.weight", np.zeros((1024, 32, 34), np.uint8))
    a.close()
    b.close()


def test_q8_small_forward(env):
    tsk, orc = env
    dit, od, _, _ = build_q8_pair(tsk, orc, depth=3, fused_depth=1, max_latent=64)
    lat, t, txt = inputs(2, 50)
    f = dit.forward(cm(lat), t, txt)
    ref, sens = one_ulp_sensitivity(od, lat, t, txt)
    e = rel_l2(f, ref)
    print(f"Q8_0 small DiT vs oracle Q8_0 path: rel-L2 {e:.3e} (oracle one-ulp sensitivity {sens:.3e})", flush=True)
    assert e <= max(2e-3, 2 * sens)
    dit.close()


def test_q8_config2_flow_step(env):
    """configuration 2's step (9 s, 194 + 77 tokens, CFG batch 2, 21 blocks)
    with Q8_0 block projections"""
    tsk, orc = env
    dit, od, _, _ = build_q8_pair(tsk, orc)
    lat, t, txt = inputs(2, 194)
    f = dit.forward(cm(lat), t, txt)
    ref, sens = one_ulp_sensitivity(od, lat, t, txt)
    e = rel_l2(f, ref)
    print(f"Q8_0 config 2 step vs oracle Q8_0 path: rel-L2 {e:.3e} (oracle one-ulp sensitivity {sens:.3e})",
          flush=True)
    assert e <= max(2e-3, 2 * sens)
    assert np.array_equal(dit.forward(cm(lat), t, txt), f)          # deterministic
    f1 = dit.forward(cm(lat[1:]), t[1:], txt[1:])
    assert np.array_equal(f1[0], f[1])                              # batch rows independent
    dit.close()


def test_q8_sampler(env):
    """ts_dit::sample with the Q8_0 driver: 3 steps, CFG 5, against the
    oracle's sampler with the same Q8_0 blocks. flow0 = u + 5 (c - u)
    multiplies the independent rounding noise of the two forwards by ~6.4, so
    flow0 and the latent are held to max(5e-3, 2.5 x the oracle sampler's own
    change under a one-ulp change of its noise, the larger of two draws)."""
    tsk, orc = env
    dit, od, _, _ = build_q8_pair(tsk, orc, depth=2, fused_depth=1, max_latent=64)
    rng = np.random.default_rng(4242)
    noise = rng.standard_normal((40, 64), dtype=np.float32)
    tc = rng.standard_normal((77, 1024), dtype=np.float32)
    tu = rng.standard_normal((77, 1024), dtype=np.float32)
    x, flow0 = dit.sample(noise.T, tc, tu, steps=3, cfg_scale=5.0)
    rx, rflow0 = od.sample(noise, tc, tu, steps=3, cfg_scale=5.0, act_bf16=True, kv_f16=True)
    s0 = sx = 0.0
    for _ in range(2):
        pert = (noise * (1 + 1e-7 * rng.standard_normal(noise.shape))).astype(np.float32)
        px, pflow0 = od.sample(pert, tc, tu, steps=3, cfg_scale=5.0, act_bf16=True, kv_f16=True)
        s0, sx = max(s0, rel_l2(pflow0, rflow0)), max(sx, rel_l2(px, rx))
    e0, ex = rel_l2(flow0.T, rflow0), rel_l2(x.T, rx)
    print(f"Q8_0 sampler: flow0 {e0:.3e}, latent {ex:.3e} (oracle one-ulp sensitivity {s0:.3e}, {sx:.3e})",
          flush=True)
    assert e0 <= max(5e-3, 2.5 * s0) and ex <= max(5e-3, 2.5 * sx)
    dit.close()


def test_q8_load_gguf(env, tmp_path):
    """a GGUF file with Q8_0 block projections (the q8 converter's output) loads
    bit for bit: the same forward as uploading the blocks directly"""
    import gguf_writer as gw
    tsk, orc = env
    kw = dict(depth=2, fused_depth=1, max_latent=64)
    a, _, W, types = build_q8_pair(tsk, orc, **kw)
    tensors = []
    for name, w in W.items():
        if types[name] == Q8_0:
            tensors.append(gw.q8_0_tensor(name, orc.quantize_q8_0(w, orc.Q8_CPU_REF), w.shape[1]))
        elif w.ndim == 2:
            tensors.append(gw.bf16_tensor(name, orc.f32_to_bf16_bits(w)))
        else:
            tensors.append(gw.f32_tensor(name, w))
    path = tmp_path / "dit_q8.gguf"
    gw.write_gguf(path, {"dit.depth": (gw.U32, 2), "dit.fused_depth": (gw.U32, 1)}, tensors)
    g = tsk.Gguf(path)
    b = tsk.Dit(tsk.dit_config(weight_type=Q8_0, **kw))
    g.load_into(b)
    lat, t, txt = inputs(2, 40, seed=5)
    assert np.array_equal(a.forward(cm(lat), t, txt), b.forward(cm(lat), t, txt))
    g.close()
    a.close()
    b.close()


def test_stream_pairs_change_no_bits(env, monkeypatch):
    """A joint block's two Q8_0 projections run as one launch (both streams'
    tiles in one grid); each output is summed in the same order as when the
    streams run as two launches (TSK_Q8_PAIR=0): the flow is bit-equal, at 9 s
    and at a length where the tile shape changes (T = 400), over joint blocks
    with a pre_only text stream and fused blocks."""
    tsk, orc = env
    dit, _, _, _ = build_q8_pair(tsk, orc, depth=3, fused_depth=1, max_latent=400)
    try:
        for T in (194, 400):
            lat, t, txt = inputs(2, T, seed=T + 3)
            ref = dit.forward(cm(lat), t, txt)
            monkeypatch.setenv("TSK_Q8_PAIR", "0")
            tsk.init(0, reread=True)
            f = dit.forward(cm(lat), t, txt)
            monkeypatch.delenv("TSK_Q8_PAIR")
            tsk.init(0, reread=True)
            assert np.isfinite(ref).all() and np.array_equal(f, ref), T
    finally:
        monkeypatch.delenv("TSK_Q8_PAIR", raising=False)
        tsk.init(0, reread=True)
        dit.close()


@pytest.mark.parametrize("T,cfg", [(194, None), (40, "43"), (40, "24"), (40, "14"), (40, "25")])
def test_attention_q8_output_bits(env, T, cfg):
    """the attention writing linear1's Q8_0 planes itself (the default) gives
    the bits of its f32 output quantized by the separate kernel
    (TSK_ATTN_Q8=0): joint blocks with a pre_only text stream and the
    automatic 4 x 1 / 4 x 2 launch shapes (T = 194), and forced 4 x 3, 2 x 4,
    1 x 4 and 2 x 5 shapes (key ranges x query blocks: the Q8_0 block's amax
    across two waves, one wave's lane pair, a lane pair per 32 dims)"""
    import os
    tsk, _ = env
    lat, t, txt = inputs(2, T)
    out = {}
    keys = ("TSK_ATTN_Q8", "TSK_ATTN_CFG")
    old = {k: os.environ.get(k) for k in keys}
    try:
        if cfg:
            os.environ["TSK_ATTN_CFG"] = cfg
        for flag in ("0", "1"):
            os.environ["TSK_ATTN_Q8"] = flag
            tsk.init(0, reread=True)
            dit = tsk.Dit(tsk.dit_config(weight_type=Q8_0, max_batch=2, max_latent=T))
            for k, v in tsk.synthetic_weights(dit.tensors(), seed=99).items():
                dit.set_tensor(k, v)
            out[flag] = dit.forward(cm(lat), t, txt)
            dit.close()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        tsk.init(0, reread=True)
    assert np.isfinite(out["1"]).all()
    assert np.array_equal(out["0"], out["1"])


@pytest.mark.parametrize("T,B", [(194, 2), (40, 2), (23, 1)])
def test_qkv_epilogue_bits(env, T, B):
    """the Q8_0 QKV GEMM writing the attention operands in its epilogue (the
    default) gives the bits of its f32 rows scattered by the separate kernel
    (TSK_Q8_QKV_FUSED=0): joint blocks (two streams in one launch, a pre_only
    text stream) and fused blocks, token counts that leave partial 64-token
    tiles, one and two batch items"""
    import os
    tsk, _ = env
    lat, t, txt = inputs(B, T)
    out = {}
    old = os.environ.get("TSK_Q8_QKV_FUSED")
    try:
        for flag in ("0", "1"):
            os.environ["TSK_Q8_QKV_FUSED"] = flag
            tsk.init(0, reread=True)
            dit = tsk.Dit(tsk.dit_config(weight_type=Q8_0, max_batch=B, max_latent=T))
            for k, v in tsk.synthetic_weights(dit.tensors(), seed=99).items():
                dit.set_tensor(k, v)
            out[flag] = dit.forward(cm(lat), t, txt)
            dit.close()
    finally:
        if old is None:
            os.environ.pop("TSK_Q8_QKV_FUSED", None)
        else:
            os.environ["TSK_Q8_QKV_FUSED"] = old
        tsk.init(0, reread=True)
    assert np.isfinite(out["1"]).all()
    assert np.array_equal(out["0"], out["1"])


@pytest.mark.parametrize("fused", ["0", "1"])
def test_v_rows_layout_bits(env, fused):
    """V written as rows [B][H][Ntot][64] (the default) or as V^T rows
    (TSK_ATTN_VROWS=0) by the Q8_0 QKV epilogue (fused) or the scatter kernel:
    the attention reads the same fp16 values either way, and the Q8_0 step's
    output is the same bit for bit"""
    import os
    tsk, _ = env
    lat, t, txt = inputs(2, 194)
    out = {}
    keys = ("TSK_ATTN_VROWS", "TSK_Q8_QKV_FUSED")
    old = {k: os.environ.get(k) for k in keys}
    try:
        os.environ["TSK_Q8_QKV_FUSED"] = fused
        for flag in ("0", "1"):
            os.environ["TSK_ATTN_VROWS"] = flag
            tsk.init(0, reread=True)
            dit = tsk.Dit(tsk.dit_config(weight_type=Q8_0, max_batch=2, max_latent=194))
            for k, v in tsk.synthetic_weights(dit.tensors(), seed=99).items():
                dit.set_tensor(k, v)
            out[flag] = dit.forward(cm(lat), t, txt)
            dit.close()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        tsk.init(0, reread=True)
    assert np.isfinite(out["1"]).all()
    assert np.array_equal(out["0"], out["1"])
