"""The reference graph (tsk_mmdit, src/mmdit.cpp:119-376) in the weight types
of every converter output, against the oracle's restatement holding the same
types, and the GGUF loader (ts_dit::load, src/mmdit.cpp:104-116):

- Q8_0 (convert/quantize_gguf.py:9-15): 2-D linears with ne0 % 32 == 0 as
  Q8_0 x Q8_0 products (qkv, every adaLN, the text stream's linear1 / MLP,
  the input and conditioning linears), the 3-D convolution kernels and the
  t_embed MLP F32 (the convolutions as three bf16 products each by default,
  the t_embed MLP as fp32 products);
- F32 (the F32 GGUF, the "GGML F32 path" of the accuracy targets);
- files read by tsk_mmdit_create_from_gguf: a Q8_0 GGUF and a BF16 GGUF give
  the bits of a model holding the same values through set_tensor; a Q8_0
  t_embed MLP (convert/convert_thinksound.py --quant q8_0 quantizes it; the
  quantize_gguf.py rule keeps it F32) runs as Q8_0;
- the on-device sampler (conditioning once, CFG / Euler on the device)
  against a host loop over tsk_mmdit_forward, bit for bit.

Bounds: a forward is held to max(2e-3, 2 x the oracle's own sensitivity)
against the oracle with the same weight types. The sensitivity is the larger
of two changes of the oracle's output: when its attention takes K / V in F32
instead of the reference's F16 cast, and when its inputs move by 2^-20
relative (random signs), the size of the differences fp32 summation order
makes in the F32 products (the F32 stages here and in the oracle differ by
1-2e-6). With Q8_0 activations such a change flips some quantization
roundings; a flip in the conditioning vectors (two rows, every token's
modulation) spreads to every token, so the oracle's own response to that
perturbation is 7-9e-3 on these models, whatever did the perturbing. The F32
model has no such rounding and is held to 2e-3 against the F32 path
outright."""
import numpy as np
import pytest

import gguf_writer as gw
from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32, Q8_0, BF16 = 0, 8, 30
SMALL = dict(depth=3, fused_depth=1, max_latent=64, max_clip=16, max_sync=48)


@pytest.fixture(scope="module")
def env(orc):
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    return tsk, orc


def build_typed(tsk, orc, wt, seed=1234, **kw):
    m = tsk.MMDit(tsk.mmdit_config(weight_type=wt, **kw))
    od = orc.OracleMMDiT(orc.mmdit_config(weight_type=wt, **kw))
    names = m.tensors()
    assert names == od.tensors()
    W = tsk.mmdit_synthetic_weights(names, seed=seed)
    for k, v in W.items():
        m.set_tensor(k, v)
        od.set_tensor(k, v)
    return m, od, W


def inputs(B, T, Sc, Ss, seed=4242):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32)
    return f(B, 64, T), f(B, Sc, 1024), f(B, Ss, 768), f(B, 77, 1024), f(B, 77, 2048), f(B, 1024)


def jittered(args, seed=7, rel=2.0 ** -20):
    """every float input times (1 +- rel), random signs (t kept)"""
    rng = np.random.default_rng(seed)
    j = lambda a: (a * (1 + np.float32(rel) * rng.choice(np.array([-1, 1], np.float32), a.shape))).astype(np.float32)
    return (j(args[0]), args[1]) + tuple(j(a) for a in args[2:])


def check(m, od, args, label):
    f = m.forward(*args)
    assert np.isfinite(f).all()
    ref = od.forward(*args)
    floor_kv = rel_l2(od.forward(*args, kv_f16=False), ref)
    floor_j = rel_l2(od.forward(*jittered(args)), ref)
    e = rel_l2(f, ref)
    e32 = rel_l2(f, od.forward(*args, act_bf16=False, kv_f16=False))
    print(f"{label}: rel-L2 {e:.3e} vs the oracle with the same types (its own change: K/V F16-vs-F32 "
          f"{floor_kv:.3e}, inputs x (1 +- 2^-20) {floor_j:.3e}); {e32:.3e} vs the F32 path", flush=True)
    assert e <= max(2e-3, 2 * max(floor_kv, floor_j))
    return f


def test_q8_0_rule_types(env):
    """the quantize_gguf.py rule: 2-D linears Q8_0, convolutions / t_embed /
    vectors / empties F32"""
    tsk, orc = env
    m = tsk.MMDit(tsk.mmdit_config(weight_type=Q8_0, **SMALL))
    ty = {n: t for n, _, t in m.tensors()}
    assert ty["joint_blocks.0.latent_block.attn.qkv.weight"] == Q8_0
    assert ty["joint_blocks.0.latent_block.adaLN_modulation.1.weight"] == Q8_0
    assert ty["joint_blocks.0.text_block.ffn.w2.weight"] == Q8_0
    assert ty["clip_input_proj.0.weight"] == Q8_0 and ty["global_cond_mlp.w1.weight"] == Q8_0
    assert ty["joint_blocks.0.latent_block.linear1.weight"] == F32
    assert ty["audio_input_proj.2.w2.weight"] == F32 and ty["final_layer.conv.weight"] == F32
    assert ty["t_embed.mlp.0.weight"] == F32 and ty["sync_pos_emb"] == F32 and ty["empty_t5_feat"] == F32
    m.close()


def test_q8_0_graph_forward(env):
    """3 blocks (the second pre_only for clip / text) + 1 fused, B = 2, a
    different t per row; batch rows independent"""
    tsk, orc = env
    m, od, _ = build_typed(tsk, orc, Q8_0, **SMALL)
    args = inputs(2, 40, 10, 32)
    args = (args[0], np.array([0.8, 0.3], np.float32)) + args[1:]
    f = check(m, od, args, "Q8_0 graph, 3 blocks, T=40")
    f1 = m.forward(*(a[1:] for a in args))
    assert np.array_equal(f1[0], f[1])
    m.close()


def test_q8_0_graph_9s_shapes(env):
    """2 joint + 2 fused blocks at the 9 s token counts (194 / 72 / 216)"""
    tsk, orc = env
    m, od, _ = build_typed(tsk, orc, Q8_0, depth=4, fused_depth=2, max_latent=194, max_clip=72, max_sync=216)
    args = inputs(2, 194, 72, 216, seed=9)
    check(m, od, (args[0], np.full(2, 0.6, np.float32)) + args[1:], "Q8_0 graph, 4 blocks, 9 s shapes")
    m.close()


def test_f32_graph_forward(env):
    """the all-F32 model (dit-f32.gguf) against the oracle's F32 path"""
    tsk, orc = env
    m, od, _ = build_typed(tsk, orc, F32, **SMALL)
    assert all(t == F32 for _, _, t in m.tensors())
    lat, clip, sync, text, t5, g = inputs(2, 40, 10, 32, seed=13)
    args = (lat, np.array([0.5, 0.9], np.float32), clip, sync, text, t5, g)
    f = m.forward(*args)
    ref = od.forward(*args, act_bf16=False, kv_f16=True)
    e = rel_l2(f, ref)
    print(f"F32 graph vs the oracle's F32 path: rel-L2 {e:.3e}", flush=True)
    assert e <= 2e-3
    m.close()


def test_f32_split_products(env, monkeypatch):
    """F32 matrices as three bf16 products (the default, TSK_F32_SPLIT=1: the
    weight's planes [hi | lo | hi] against the rows' [hi | hi | lo]) against
    fp32 MFMA products (TSK_F32_SPLIT=0, read on every call) in the same
    model, at the 9 s token counts. The latent input projection (x_in: a k3
    convolution and a convMLP, every kernel F32 in both GGUFs, no attention)
    moves by the dropped x_lo w_lo terms and the lo roundings only: held to
    1e-4 of the oracle's F32 stage, where fp32 products agree to 1e-5 and a
    split that lost its lo planes would be ~2e-3 off. The flows carry the
    attention's F16 K / V roundings, which such small moves flip here and
    there (the two modes' flows differ by ~2e-4): the F32 model's flow is
    held to 2e-3 of the F32 path in both modes, the Q8_0 model's (whose Q8_0
    activations flip as well) to the oracle's bound in both modes."""
    tsk, orc = env
    kw = dict(depth=4, fused_depth=2, max_latent=194, max_clip=72, max_sync=216)
    args = inputs(2, 194, 72, 216, seed=21)
    args = (args[0], np.array([0.7, 0.2], np.float32)) + args[1:]
    for wt in (F32, Q8_0):
        m, od, _ = build_typed(tsk, orc, wt, **kw)
        m.debug(True)
        try:
            f_split = m.forward(*args)
            x_split = m.stage("x_in")
            monkeypatch.setenv("TSK_F32_SPLIT", "0")
            tsk.init(0, reread=True)
            f_exact = m.forward(*args)
            x_exact = m.stage("x_in")
        finally:
            monkeypatch.delenv("TSK_F32_SPLIT", raising=False)
            tsk.init(0, reread=True)
        m.debug(False)
        assert np.isfinite(f_split).all() and np.isfinite(f_exact).all()
        ref = od.forward(*args, act_bf16=False, kv_f16=True)
        x_ref = od.stage("x_in")
        xs, xx = rel_l2(x_split, x_ref), rel_l2(x_exact, x_ref)
        d = rel_l2(f_split, f_exact)
        print(f"type {wt}, 9 s shapes: x_in vs the oracle's F32 stage: split {xs:.3e}, fp32 products {xx:.3e}; "
              f"flows split vs fp32 products {d:.3e}", flush=True)
        assert xs <= 1e-4 and xx <= 1e-5
        if wt == F32:
            e_s, e_x = rel_l2(f_split, ref), rel_l2(f_exact, ref)
            print(f"F32 model: flow vs the F32 path: split {e_s:.3e}, fp32 products {e_x:.3e}", flush=True)
            assert e_s <= 2e-3 and e_x <= 2e-3
        else:
            check(m, od, args, "Q8_0 graph, 9 s shapes, split F32 products")
            monkeypatch.setenv("TSK_F32_SPLIT", "0")
            tsk.init(0, reread=True)
            try:
                check(m, od, args, "Q8_0 graph, 9 s shapes, fp32 products")
            finally:
                monkeypatch.delenv("TSK_F32_SPLIT", raising=False)
                tsk.init(0, reread=True)
        m.close()


GGUF_KW = dict(depth=3, fused_depth=1, mlp_hidden=512, max_latent=64, max_clip=16, max_sync=48)


def dit_keys(c):
    """the keys convert/convert_thinksound.py:38-45 writes"""
    u = lambda v: (gw.U32, v)
    return {"dit.latent_dim": u(c.latent_dim), "dit.clip_dim": u(c.clip_dim), "dit.sync_dim": u(c.sync_dim),
            "dit.text_dim": u(c.t5_dim), "dit.hidden_dim": u(c.hidden), "dit.depth": u(c.depth),
            "dit.fused_depth": u(c.fused_depth), "dit.num_heads": u(c.n_head), "dit.text_seq_len": u(c.text_seq),
            "dit.kernel_size": u(3), "dit.sync_kernel": u(7), "dit.rope_theta": (gw.F32, 10000.0),
            "dit.t_embed_max_period": (gw.F32, 1.0), "dit.sample_rate": u(44100),
            "dit.diffusion_objective": (gw.STRING, "rectified_flow")}


def file_tensors(orc, W, types):
    """GGUF tensors: Q8_0 blocks (ggml's reference quantizer), BF16 bits or F32"""
    out = []
    for name, w in W.items():
        t = types[name]
        if t == Q8_0:
            out.append(gw.q8_0_tensor(name, orc.quantize_q8_0(w, orc.Q8_CPU_REF), w.shape[-1]))
        elif t == BF16:
            out.append(gw.bf16_tensor(name, orc.f32_to_bf16_bits(w)))
        else:
            out.append(gw.f32_tensor(name, w))
    return out


def test_gguf_q8_0_graph(env, tmp_path):
    """A Q8_0 GGUF (quantize_gguf.py's types) loads into the model's types bit
    for bit: tsk_mmdit_create_from_gguf gives the forward bits of a model that
    quantized the same f32 weights itself; the file's sizes and weight type
    come from its dit.* keys. A file whose t_embed MLP is Q8_0 too (the
    converter's --quant q8_0 rule) runs it as Q8_0, held to the oracle with
    the same types."""
    tsk, orc = env
    a = tsk.MMDit(tsk.mmdit_config(weight_type=Q8_0, **GGUF_KW))
    names = a.tensors()
    types = {n: t for n, _, t in names}
    W = tsk.mmdit_synthetic_weights(names, seed=71)
    for k, v in W.items():
        a.set_tensor(k, v)
    path = tmp_path / "dit-q8.gguf"
    gw.write_gguf(path, dit_keys(a.cfg), file_tensors(orc, W, types))
    g = tsk.Gguf(path)
    c = g.mmdit_config(max_latent=64, max_clip=16, max_sync=48)
    assert (c.depth, c.fused_depth, c.mlp_hidden, c.weight_type) == (3, 1, 512, Q8_0)
    b = tsk.MMDit(c, gguf=g)
    assert b.tensors() == names
    lat, clip, sync, text, t5, gt = inputs(2, 37, 12, 40, seed=3)
    args = (lat, np.array([0.7, 0.2], np.float32), clip, sync, text, t5, gt)
    np.testing.assert_array_equal(b.forward(*args), a.forward(*args))
    # a BF16 model cannot hold the file's Q8_0 tensors
    bf = tsk.MMDit(tsk.mmdit_config(weight_type=BF16, **GGUF_KW))
    with pytest.raises(tsk.TskError) as ei:
        bf.load_gguf(g)
    assert ei.value.status == -2
    g.close()
    bf.close()
    b.close()
    a.close()
    # the t_embed MLP as Q8_0
    t2 = dict(types)
    for n in ("t_embed.mlp.0.weight", "t_embed.mlp.2.weight"):
        t2[n] = Q8_0
    path2 = tmp_path / "dit-q8-temb.gguf"
    ft = file_tensors(orc, W, t2)
    gw.write_gguf(path2, dit_keys(c), ft)
    g2 = tsk.Gguf(path2)
    m = tsk.MMDit(g2.mmdit_config(max_latent=64, max_clip=16, max_sync=48), gguf=g2)
    assert {n: t for n, _, t in m.tensors()}["t_embed.mlp.2.weight"] == Q8_0
    od = orc.OracleMMDiT(orc.mmdit_config(weight_type=Q8_0, **GGUF_KW))
    for n in ("t_embed.mlp.0.weight", "t_embed.mlp.2.weight"):
        od.set_type(n, Q8_0)
    for name, ne, gtype, raw in ft:
        if gtype == gw.GGML_Q8_0:
            od.set_tensor_q8_0(name, raw)
        else:
            od.set_tensor(name, W[name])
    check(m, od, args, "Q8_0 GGUF with a Q8_0 t_embed MLP")
    g2.close()
    m.close()


def test_gguf_bf16_graph(env, tmp_path):
    """a BF16 GGUF (quantize_gguf.py --type bf16: BF16 linears and
    convolutions, F32 t_embed MLP and vectors) gives the bits of the
    synthetic-weight model; an F32 file matrix is refused by a BF16 model"""
    tsk, orc = env
    a = tsk.MMDit(tsk.mmdit_config(**GGUF_KW))
    names = a.tensors()
    types = {n: t for n, _, t in names}
    W = tsk.mmdit_synthetic_weights(names, seed=72)
    for k, v in W.items():
        a.set_tensor(k, v)
    path = tmp_path / "dit-bf16.gguf"
    gw.write_gguf(path, dit_keys(a.cfg), file_tensors(orc, W, types))
    g = tsk.Gguf(path)
    c = g.mmdit_config(max_latent=64, max_clip=16, max_sync=48)
    assert c.weight_type == BF16
    b = tsk.MMDit(c, gguf=g)
    lat, clip, sync, text, t5, gt = inputs(2, 33, 9, 24, seed=4)
    args = (lat, np.array([0.4, 0.4], np.float32), clip, sync, text, t5, gt)
    np.testing.assert_array_equal(b.forward(*args), a.forward(*args))
    g.close()
    path32 = tmp_path / "dit-f32.gguf"
    gw.write_gguf(path32, dit_keys(a.cfg), file_tensors(orc, W, {n: F32 for n in types}))
    g32 = tsk.Gguf(path32)
    assert g32.mmdit_config().weight_type == F32
    with pytest.raises(tsk.TskError) as ei:
        a.load_gguf(g32)
    assert ei.value.status == -2
    g32.close()
    a.close()
    b.close()


@pytest.mark.parametrize("wt", [BF16, Q8_0])
def test_sampler_on_device_matches_host_loop(env, wt):
    """tsk_mmdit_sample (conditioning once, x on the device, CFG / Euler on
    the device) against ts_dit::sample's loop written on the host over
    tsk_mmdit_forward (src/mmdit.cpp:358-373: t = 1 - s / steps, one B = 2
    forward with the unconditional row on the learned empties and a zero
    global text feature, v = u + cfg (c - u), x += dt v in fp32): the same
    bits, latent and flow0"""
    tsk, orc = env
    m = tsk.MMDit(tsk.mmdit_config(weight_type=wt, **SMALL))
    W = tsk.mmdit_synthetic_weights(m.tensors(), seed=8)
    for k, v in W.items():
        m.set_tensor(k, v)
    lat, clip, sync, text, t5, g = inputs(1, 40, 10, 32, seed=21)
    steps, cfg = 3, np.float32(5.0)
    x, flow0 = m.sample(lat[0], clip[0], sync[0], text[0], t5[0], g[0], steps=steps, cfg_scale=5.0)
    hx = lat[0].copy()                                   # (L, T)
    es = W["empty_string_feat"].reshape(77, 1024)
    et = W["empty_t5_feat"].reshape(77, 2048)
    h0 = None
    for s in range(steps):
        t_curr = np.float32(1) - np.float32(s) / np.float32(steps)
        t_prev = np.float32(1) - np.float32(s + 1) / np.float32(steps)
        dt = np.float32(t_prev - t_curr)
        f = m.forward(np.stack([hx, hx]), np.array([t_curr, t_curr], np.float32), np.concatenate([clip, clip]),
                      np.concatenate([sync, sync]), np.stack([text[0], es]), np.stack([t5[0], et]),
                      np.stack([g[0], np.zeros(1024, np.float32)]))
        fc, fu = f[0].T, f[1].T                           # (L, T)
        v = fu + (fc - fu) * cfg
        if s == 0:
            h0 = v.copy()
        hx = hx + dt * v
    assert np.array_equal(flow0, h0)
    assert np.array_equal(x, hx)
    m.close()
