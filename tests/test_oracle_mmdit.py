"""Independent pin of the oracle's restatement of the reference's MM-DiT graph
(orc_mmdit_forward / orc_mmdit_sample, src/mmdit.cpp:119-376) against the fp64
formulation refmath.mmdit_forward_ref / mmdit_sample_ref, written from the
graph's structure with convolutions as sums of shifted matrix products.

The oracle runs in its all-fp32 mode (F32 weights and activations, F32 K /
V), so the two differ only by fp32 rounding of intermediates: tolerance 1e-6
rel-L2 (measured ~1e-7). Each structural mistake a composition could make --
shift / scale swapped, the clip RoPE without its T / S_c scale, the sync
index without the half-step of nearest-exact, text_f padded on the wrong
side, the latent adaLN from global_c instead of extended_c, a clip stream that is
never updated, the wrong gate on the MLP branch -- moves the restatement by
far more than 100 x the tolerance, so none can pass. (The order of the text
tokens is not observable: they carry no position and attention is invariant
under a permutation of its keys.)"""
import numpy as np
import pytest

import refmath
from conftest import rel_l2

TOL = 1e-6
SMALL = dict(hidden=128, n_head=2, head_dim=64, depth=3, fused_depth=1, latent_dim=32, text_seq=5, clip_dim=64,
             sync_dim=64, t5_dim=128, mlp_hidden=96, max_batch=2, max_latent=32, max_clip=16, max_sync=48,
             rope_theta=10000.0, t_max_period=1.0)


def weights(tensors, seed, std=0.05):
    """random F32 weights in PyTorch order (ne reversed), norm weights 1 + std,
    the learned empty features N(0, 1)"""
    out = {}
    for i, (name, ne, _) in enumerate(tensors):
        rng = np.random.default_rng([seed, i])
        shape = tuple(int(x) for x in reversed(ne))
        while len(shape) > 1 and shape[0] == 1:
            shape = shape[1:]
        w = rng.standard_normal(shape) * (1.0 if name.startswith("empty_") else std)
        if name.endswith("norm.weight"):
            w += 1.0
        out[name] = w.astype(np.float32)
    return out


@pytest.fixture(scope="module")
def small(orc):
    od = orc.OracleMMDiT(orc.mmdit_config(**SMALL))
    W = weights(od.tensors(), 11)
    for k, v in W.items():
        od.set_tensor(k, v)
    return od, W


def inputs(B=1, T=12, Sc=5, Ss=16, seed=3):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    return (f(B, SMALL["latent_dim"], T), f(B, Sc, SMALL["clip_dim"]), f(B, Ss, SMALL["sync_dim"]),
            f(B, SMALL["text_seq"], SMALL["clip_dim"]), f(B, SMALL["text_seq"], SMALL["t5_dim"]),
            f(B, SMALL["clip_dim"]))


def test_tensor_inventory(small):
    """the converter's names: 7 joint x 3 streams + fused blocks; the last
    joint block's clip / text streams pre_only (adaLN of 2 H, no linear1 /
    ffn); t_embed and the vectors F32, every other matrix BF16"""
    od, W = small
    names = {n: (ne, ty) for n, ne, ty in od.tensors()}
    H = SMALL["hidden"]
    assert names["joint_blocks.1.clip_block.adaLN_modulation.1.weight"][0] == (H, 2 * H, 1)
    assert "joint_blocks.1.clip_block.linear1.weight" not in names
    assert names["joint_blocks.0.clip_block.linear1.weight"][0] == (3, H, H)
    assert names["joint_blocks.0.text_block.linear1.weight"][0] == (H, H, 1)
    assert names["final_layer.conv.weight"][0] == (7, H, SMALL["latent_dim"])
    assert names["sync_input_proj.0.weight"][0] == (7, SMALL["sync_dim"], H)
    assert names["t_embed.mlp.0.weight"][1] == 0 and names["clip_cond_proj.weight"][1] == 30
    assert all(ty == 0 for n, (ne, ty) in names.items() if ne[1] == 1 and ne[2] == 1)


@pytest.mark.parametrize("t,T,Sc,Ss", [(0.5, 12, 5, 16), (0.9, 20, 7, 24), (0.1, 9, 9, 8)])
def test_mmdit_forward_matches_fp64_restatement(small, t, T, Sc, Ss):
    od, W = small
    lat, clip, sync, text, t5, g = inputs(1, T, Sc, Ss)
    got = od.forward(lat, np.array([t], np.float32), clip, sync, text, t5, g, act_bf16=False, kv_f16=False)[0]
    ref = refmath.mmdit_forward_ref(W, SMALL, lat[0], t, clip[0], sync[0], text[0], t5[0], g[0])
    e = rel_l2(got, ref)
    print(f"orc_mmdit_forward vs fp64 (T={T}, clip {Sc}, sync {Ss}): rel-L2 {e:.2e}")
    assert e <= TOL


def test_mmdit_forward_batch_rows_independent(small):
    od, W = small
    lat, clip, sync, text, t5, g = inputs(2, seed=5)
    got = od.forward(lat, np.array([0.3, 0.7], np.float32), clip, sync, text, t5, g, act_bf16=False, kv_f16=False)
    ref = refmath.mmdit_forward_ref(W, SMALL, lat[1], 0.7, clip[1], sync[1], text[1], t5[1], g[1])
    assert rel_l2(got[1], ref) <= TOL


@pytest.mark.parametrize("mistake", [dict(swap_shift_scale=True), dict(clip_rope_unscaled=True),
                                     dict(sync_index_no_half=True), dict(text_pad_left=True),
                                     dict(latent_cond_global=True), dict(clip_frozen=True),
                                     dict(gate_mlp_index=2)])
def test_mmdit_restatement_detects_structural_mistakes(small, mistake):
    od, W = small
    lat, clip, sync, text, t5, g = inputs(1, 12, 5, 16)
    got = od.forward(lat, np.array([0.5], np.float32), clip, sync, text, t5, g, act_bf16=False, kv_f16=False)[0]
    wrong = refmath.mmdit_forward_ref(W, SMALL, lat[0], 0.5, clip[0], sync[0], text[0], t5[0], g[0], **mistake)
    e = rel_l2(got, wrong)
    print(f"planted {mistake}: rel-L2 {e:.2e}")
    assert e > 100 * TOL


def test_mmdit_sample_matches_fp64_restatement(small):
    """3 Euler steps with CFG 5; the unconditional branch on the learned empties"""
    od, W = small
    lat, clip, sync, text, t5, g = inputs(1, 10, 5, 16, seed=9)
    x, flow0 = od.sample(lat[0], clip[0], sync[0], text[0], t5[0], g[0], steps=3, cfg_scale=5.0, act_bf16=False,
                         kv_f16=False)
    rx, rflow0 = refmath.mmdit_sample_ref(W, SMALL, lat[0], clip[0], sync[0], text[0], t5[0], g[0], 3, 5.0)
    e0, ex = rel_l2(flow0, rflow0), rel_l2(x, rx)
    print(f"orc_mmdit_sample vs fp64: flow0 {e0:.2e}, latent {ex:.2e}")
    assert e0 <= TOL and ex <= TOL
    # the unconditional branch matters: the sampler with cond == uncond inputs differs
    Wu = dict(W, empty_string_feat=text[0], empty_t5_feat=t5[0])
    wx, _ = refmath.mmdit_sample_ref(Wu, SMALL, lat[0], clip[0], sync[0], text[0], t5[0], g[0], 3, 5.0)
    assert rel_l2(x, wx) > 100 * TOL


def test_q8_0_types_and_dequantized_f32_path(orc):
    """weight_type Q8_0 (convert/quantize_gguf.py:9-15): the 2-D linears with
    ne0 % 32 == 0 are held as Q8_0 (ggml's reference quantizer), the
    convolutions, the t_embed MLP and every vector F32. The oracle's F32 path
    then runs on the dequantized values: it matches the fp64 restatement fed
    those values (pins the quantizer round trip and the inventory), and the
    Q8_0 path -- the same weights with every Q8_0 product's input quantized
    per 32 values (orc_mul_mat, pinned by brute force) -- differs from it by
    the activation quantization only."""
    od = orc.OracleMMDiT(orc.mmdit_config(**dict(SMALL, weight_type=orc.Q8_0)))
    ty = {n: t for n, _, t in od.tensors()}
    assert ty["joint_blocks.0.latent_block.attn.qkv.weight"] == orc.Q8_0
    assert ty["text_input_proj.2.w2.weight"] == orc.Q8_0
    assert ty["joint_blocks.0.latent_block.ffn.w1.weight"] == orc.F32
    assert ty["t_embed.mlp.0.weight"] == orc.F32 and ty["empty_string_feat"] == orc.F32
    W = weights(od.tensors(), 12)
    Wq = {}
    for k, v in W.items():
        od.set_tensor(k, v)
        if ty[k] == orc.Q8_0:
            Wq[k] = orc.dequantize_q8_0(orc.quantize_q8_0(v, orc.Q8_CPU_REF)).reshape(v.shape)
        else:
            Wq[k] = v
    lat, clip, sync, text, t5, g = inputs(1, 12, 5, 16, seed=7)
    t = np.array([0.6], np.float32)
    got = od.forward(lat, t, clip, sync, text, t5, g, act_bf16=False, kv_f16=False)[0]
    ref = refmath.mmdit_forward_ref(Wq, SMALL, lat[0], 0.6, clip[0], sync[0], text[0], t5[0], g[0])
    e = rel_l2(got, ref)
    assert e <= TOL, e
    # the undequantized weights are another model
    assert rel_l2(got, refmath.mmdit_forward_ref(W, SMALL, lat[0], 0.6, clip[0], sync[0], text[0], t5[0],
                                                 g[0])) > 100 * TOL
    q = od.forward(lat, t, clip, sync, text, t5, g, act_bf16=True, kv_f16=False)[0]
    eq = rel_l2(q, got)
    print(f"Q8_0 oracle: F32 path on dequantized weights vs fp64 {e:.2e}; Q8_0 products vs F32 path {eq:.2e}")
    assert 1e-4 < eq < 5e-2


def test_q8_0_blocks_equal_quantized_values(orc):
    """orc_mmdit_set_tensor_q8_0 with the blocks of ggml's reference
    quantizer gives the bits of set_tensor on the f32 values; set_type makes
    a single tensor Q8_0 (the converter's --quant q8_0 t_embed)"""
    cfg = orc.mmdit_config(**dict(SMALL, weight_type=orc.Q8_0))
    a, b = orc.OracleMMDiT(cfg), orc.OracleMMDiT(cfg)
    for o in (a, b):
        o.set_type("t_embed.mlp.0.weight", orc.Q8_0)
    ty = {n: t for n, _, t in a.tensors()}
    assert ty["t_embed.mlp.0.weight"] == orc.Q8_0
    W = weights(a.tensors(), 13)
    for k, v in W.items():
        a.set_tensor(k, v)
        if ty[k] == orc.Q8_0:
            b.set_tensor_q8_0(k, orc.quantize_q8_0(v, orc.Q8_CPU_REF).tobytes())
        else:
            b.set_tensor(k, v)
    lat, clip, sync, text, t5, g = inputs(1, 10, 5, 16, seed=8)
    t = np.array([0.4], np.float32)
    fa = a.forward(lat, t, clip, sync, text, t5, g)
    assert np.array_equal(fa, b.forward(lat, t, clip, sync, text, t5, g))
    assert np.isfinite(fa).all()
