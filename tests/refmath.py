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


# ------------------------------------------------------------------ composites
# fp64 restatements of the composite functions the oracle builds from its ops,
# written from the reference's graph (src/mmdit.cpp, src/t5_encoder.cpp) and
# the benchmarked block shape: the structure (block order, adaLN chunk order,
# gate placement, the pre_only stream, the final layer, the CFG / Euler
# update, the T5 layer) is what these pin. Two places follow the reference's
# own fp32 host / ggml evaluation because fp64 would move their results by
# far more than the comparison resolves: the timestep-embedding arguments
# t * f_k (fp32 products fed to cosf / sinf, mmdit.cpp:305-314; |t f| reaches
# 10^4, where an fp32 argument differs from the fp64 one by ~1e-3) and the
# RoPE angles (ggml's running product theta *= theta_scale in fp32, the
# rope_ext semantics the single-op pins check).

def _f32(x):
    return np.float32(x)


def timestep_embedding_ref(t, H, max_period):
    """[cos(t f_k), sin(t f_k)], f_k = (1e4 / max_period) * 1e4^(-2k / H), the
    products rounded to fp32 as the reference's host code evaluates them."""
    half = H // 2
    k = np.arange(half, dtype=np.float64)
    p = (np.power(10000.0, (-2.0 * k / H).astype(np.float32).astype(np.float64))).astype(np.float32)
    fr = (np.float64(_f32(10000.0 / max_period)) * p.astype(np.float64)).astype(np.float32)
    arg = (np.float64(_f32(t)) * fr.astype(np.float64)).astype(np.float32).astype(np.float64)
    return np.concatenate([np.cos(arg), np.sin(arg)])


def rope_angles_ggml(npos, n_dims, base=10000.0, fscale=1.0):
    """(npos, n_dims/2) angles of ggml's rope cache: theta_scale = base^(-2/n),
    theta starts at p and is multiplied by theta_scale per pair, in fp32."""
    ts = _f32(np.power(np.float64(_f32(base)), np.float64(_f32(-2.0 / n_dims))))
    out = np.empty((npos, n_dims // 2), np.float64)
    for p in range(npos):
        theta = _f32(p)
        for i in range(n_dims // 2):
            out[p, i] = np.float64(_f32(np.float64(theta) * np.float64(_f32(fscale))))
            theta = _f32(np.float64(theta) * np.float64(ts))
    return out


def rope_apply(x, ang):
    """rotate adjacent pairs of x (S, H, D) by ang (S, D/2)"""
    out = x.copy()
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def silu(x):
    return x / (1.0 + np.exp(-x))


def _lin(W, name, x, bias=True):
    y = np.asarray(x, np.float64) @ np.asarray(W[name + ".weight"], np.float64).T
    if bias:
        y = y + np.asarray(W[name + ".bias"], np.float64)
    return y


def dit_forward_ref(W, cfg, latent, t, text, swap_shift_scale=False, text_frozen=False, gate_mlp_index=5,
                    rope_text=False):
    """One flow evaluation of the benchmarked MM-DiT (fp64), B = 1:
    latent (T, L), t scalar, text (S, H) -> flow (T, L).

    Structure (src/mmdit.cpp): t-embedding -> t_embed MLP (:158-161);
    every block's adaLN on silu(c) -> 6 chunks shift/scale/gate (msa),
    shift/scale/gate (mlp) (:209-216; 2 for a pre_only stream);
    x_mod = LN(x, 1e-5) (1 + scale) + shift (:55-59, :218); qkv with channel
    3 (h d_h + d) + j (:67-76); RMSNorm(1e-6) * w on q, k (:78-80, :221-222);
    RoPE on the latent only (:223); attention over latent | text (:251-256);
    x += linear1(o) gate_msa; x += mlp(LN(x)(1 + scale_mlp) + shift_mlp)
    gate_mlp (:226-235); the last joint block's text stream pre_only (:240);
    fused blocks on the latent (:275-281); final adaLN (2 chunks), LN /
    modulate and the output projection (:285-289).
    The switches plant structural mistakes for the sensitivity checks:
    shift / scale swapped, the text stream never updated (as if every joint
    block were pre_only), the wrong gate on the MLP branch, RoPE on text."""
    H, nh, hd = cfg["hidden"], cfg["n_head"], cfg["head_dim"]
    nj = cfg["depth"] - cfg["fused_depth"]
    ln_eps, qk_eps = cfg["ln_eps"], cfg["qk_eps"]
    temb = timestep_embedding_ref(t, H, cfg["t_max_period"])
    c = _lin(W, "t_embed.mlp.2", silu(_lin(W, "t_embed.mlp.0", temb)))
    sc = silu(c)
    lat = _lin(W, "audio_input_proj", latent)
    txt = np.asarray(text, np.float64)
    T, St = lat.shape[0], txt.shape[0]
    ang = rope_angles_ggml(T, hd, cfg["rope_theta"])

    def layer_norm(x):
        mu = x.mean(-1, keepdims=True)
        var = ((x - mu) ** 2).mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(var + ln_eps)

    def pre_attn(p, x, rope, pre_only):
        mod = _lin(W, p + ".adaLN_modulation.1", sc)
        ch = [mod[i * H:(i + 1) * H] for i in range(2 if pre_only else 6)]
        shift, scale = (ch[1], ch[0]) if swap_shift_scale else (ch[0], ch[1])
        xn = layer_norm(x) * (1.0 + scale) + shift
        qkv = _lin(W, p + ".attn.qkv", xn).reshape(x.shape[0], nh, hd, 3)
        q, k, v = qkv[..., 0], qkv[..., 1], qkv[..., 2]
        qn = np.asarray(W[p + ".attn.q_norm.weight"], np.float64)
        kn = np.asarray(W[p + ".attn.k_norm.weight"], np.float64)
        q = q / np.sqrt((q * q).mean(-1, keepdims=True) + qk_eps) * qn
        k = k / np.sqrt((k * k).mean(-1, keepdims=True) + qk_eps) * kn
        if rope:
            q, k = rope_apply(q, ang[:x.shape[0]]), rope_apply(k, ang[:x.shape[0]])
        return q, k, v, ch

    def attend(qs, ks, vs):
        q, k, v = (np.concatenate(a, axis=0) for a in (qs, ks, vs))       # (N, nh, hd)
        s = np.einsum("qhd,khd->hqk", q, k) / np.sqrt(hd)
        s = s - s.max(-1, keepdims=True)
        pr = np.exp(s)
        pr /= pr.sum(-1, keepdims=True)
        return np.einsum("hqk,khd->qhd", pr, v).reshape(q.shape[0], H)

    def post_attn(p, x, o, ch):
        x = x + _lin(W, p + ".linear1", o) * ch[2]
        r = layer_norm(x) * (1.0 + ch[4]) + ch[3]
        f = _lin(W, p + ".ffn.fc2", gelu_tanh(_lin(W, p + ".ffn.fc1", r)))
        return x + f * ch[gate_mlp_index]

    for i in range(nj):
        pre_only = i == nj - 1
        pl, pt = f"joint_blocks.{i}.latent_block", f"joint_blocks.{i}.text_block"
        ql, kl, vl, chl = pre_attn(pl, lat, True, False)
        qt, kt, vt, cht = pre_attn(pt, txt, rope_text, pre_only)
        o = attend([ql, qt], [kl, kt], [vl, vt])
        lat = post_attn(pl, lat, o[:T], chl)
        if not pre_only and not text_frozen:
            txt = post_attn(pt, txt, o[T:T + St], cht)
    for i in range(cfg["fused_depth"]):
        p = f"fused_blocks.{i}"
        q, k, v, ch = pre_attn(p, lat, True, False)
        lat = post_attn(p, lat, attend([q], [k], [v]), ch)
    fm = _lin(W, "final_layer.adaLN_modulation.1", sc)
    fx = layer_norm(lat) * (1.0 + fm[H:2 * H]) + fm[:H]
    return _lin(W, "final_layer.linear", fx)


def dit_sample_ref(W, cfg, noise, text_cond, text_uncond, steps, cfg_scale):
    """ts_dit::sample (src/mmdit.cpp:344-376) in fp64: t = 1 - s / steps,
    velocity v = u + cfg (c - u) of a conditional and an unconditional
    forward, Euler x += (t_{s+1} - t_s) v. noise (T, L) -> (x, flow0).
    The step times and dt are the reference's fp32 host values (:360-362)."""
    x = np.asarray(noise, np.float64).copy()
    flow0 = None
    f = np.float32
    for s in range(steps):
        t_curr = float(f(1.0) - f(s) / f(steps))
        t_next = float(f(1.0) - f(s + 1) / f(steps))
        t_next = t_curr + float(f(f(t_next) - f(t_curr)))
        fc = dit_forward_ref(W, cfg, x, t_curr, text_cond)
        fu = dit_forward_ref(W, cfg, x, t_curr, text_uncond)
        v = fu + (fc - fu) * cfg_scale
        if s == 0:
            flow0 = v
        x = x + (t_next - t_curr) * v
    return x, flow0


def t5_bucket_ref(rel, num_buckets=32, max_dist=128):
    """src/t5_encoder.cpp:14-26 restated with exact integer arithmetic: half
    the buckets per sign, |rel| < nb/4 exact, then nb/4 + max{j : (max_dist /
    max_exact)^(j / (nb/2 - max_exact)) <= |rel| / max_exact}, clamped. Exact
    for these parameters (max_dist / max_exact = 16 = 2^4, 8 log buckets): the
    log bucket is 8 + max{j : 16^j 8^8 <= n^8} (n^8 and 16^j 8^8 are integers)."""
    nb = num_buckets // 2
    ret = nb if rel > 0 else 0
    n = abs(rel)
    max_exact = nb // 2
    if n < max_exact:
        return ret + n
    assert max_dist // max_exact == 16 and nb - max_exact == 8, "closed form for 32 buckets / 128 only"
    j = 0
    while 16 ** (j + 1) * max_exact ** 8 <= n ** 8:
        j += 1
    return ret + min(max_exact + j, nb - 1)


def t5_encode_ref(W, cfg, x, ids, layers=None, final_norm=True):
    """ts_t5::encode's layers (src/t5_encoder.cpp:56-88) in fp64 with F32
    weights: h = rmsnorm(x) w_attn; q, k, v = h W^T; scores = q k^T (no
    scale) + rel_bias[bucket(k - q)][head] + (-inf on padded keys);
    softmax; o = P v; x += o W_o^T; h = rmsnorm(x) w_ffn;
    x += (gelu(h W_i0^T) * (h W_i1^T)) W_o'^T; out_norm at the end."""
    d, nh, dk = cfg["d_model"], cfg["n_heads"], cfg["d_kv"]
    eps = cfg["eps"]
    x = np.asarray(x, np.float64).copy()
    n = x.shape[0]
    rel = np.arange(n)[None, :] - np.arange(n)[:, None]                 # k - q
    bk = np.vectorize(lambda r: t5_bucket_ref(int(r), cfg["rel_buckets"], cfg["rel_max_dist"]))(rel)
    rb = np.asarray(W["rel_bias"], np.float64)                           # (buckets, heads)
    bias = rb[bk].transpose(2, 0, 1)                                     # (heads, q, k)
    pad = np.where(np.asarray(ids) != 0, 0.0, -np.inf)[None, None, :]

    def rms(v, w):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)

    def mm(name, v):
        return v @ np.asarray(W[name], np.float64).T

    b, e = layers if layers is not None else (0, cfg["n_layers"])
    for i in range(b, e):
        p = f"blk.{i}"
        h = rms(x, W[p + ".attn_norm"])
        q, k, v = (mm(p + s, h).reshape(n, nh, dk) for s in (".q", ".k", ".v"))
        s = np.einsum("qhd,khd->hqk", q, k) + bias + pad
        m = s.max(-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        pr = np.exp(s - m)
        den = pr.sum(-1, keepdims=True)
        pr = pr / np.where(den == 0, 1.0, den)
        o = np.einsum("hqk,khd->qhd", pr, v).reshape(n, nh * dk)
        x = x + mm(p + ".o", o)
        h = rms(x, W[p + ".ffn_norm"])
        x = x + mm(p + ".wo", gelu_tanh(mm(p + ".wi_0", h)) * mm(p + ".wi_1", h))
    return rms(x, W["out_norm"]) if final_norm else x


def conv1d_ref(W, name, x, pad, bias=True):
    """y[t] = sum_kw W[:, :, kw] x[t + kw - pad] (+ b), zero outside the
    sequence: PyTorch Conv1d(stride 1) with W (OC, IC, KW), x (S, IC)."""
    w = np.asarray(W[name + ".weight"], np.float64)
    oc, ic, kw = w.shape
    x = np.asarray(x, np.float64)
    S = x.shape[0]
    xp = np.concatenate([np.zeros((pad, ic)), x, np.zeros((pad, ic))])
    y = np.zeros((S + 2 * pad - kw + 1, oc))
    for j in range(kw):
        y += xp[j:j + y.shape[0]] @ w[:, :, j].T
    if bias:
        y = y + np.asarray(W[name + ".bias"], np.float64)
    return y


def mmdit_forward_ref(W, cfg, latent, t, clip, sync, text, t5, g, swap_shift_scale=False, clip_rope_unscaled=False,
                      sync_index_no_half=False, text_pad_left=False, latent_cond_global=False, clip_frozen=False,
                      gate_mlp_index=5):
    """The reference's MM-DiT graph (src/mmdit.cpp:119-342) in fp64, B = 1:
    latent (L, T), t scalar, clip (S_c, clip_dim), sync (S_s, sync_dim),
    text (text_seq, clip_dim), t5 (text_seq, t5_dim), g (clip_dim,) ->
    flow (T, L). Written from the graph's structure:
      x = convmlp(silu(conv_k3(latent^T)));  c_t = mlp_t(temb(t))
      clip = convmlp(silu(W clip + b));  sync = convmlp(silu(conv_k7(sync + pos)))
      text = mlp(silu(W [text | 0 ; t5] + b))           (154 tokens)
      global = c_t + swiglu_mlp(W_c mean(clip) + b_c + W_t g + b_t)
      ext[t] = sync[floor((t + 0.5) S_s / T)] + global
    joint blocks: the latent stream's adaLN from ext (one modulation per
    token), clip / text from global; RoPE on latent (scale 1) and clip
    (scale T / S_c); attention over latent | clip | text; linear1 and the
    MLP are k3 convolutions on latent / clip, linear on text; the last
    block's clip / text pre_only. Fused blocks on the latent with ext; final
    adaLN(ext), LN / modulate, conv k7.
    Switches plant the structural mistakes the pin must catch."""
    H, nh, hd = cfg["hidden"], cfg["n_head"], cfg["head_dim"]
    nj = cfg["depth"] - cfg["fused_depth"]
    X = 2 * cfg["text_seq"]

    def swiglu_conv(p, x):
        return conv1d_ref(W, p + ".w2", silu(conv1d_ref(W, p + ".w1", x, 1, False)) *
                          conv1d_ref(W, p + ".w3", x, 1, False), 1, False)

    def swiglu_lin(p, x):
        return _lin(W, p + ".w2", silu(_lin(W, p + ".w1", x, False)) * _lin(W, p + ".w3", x, False), False)

    def layer_norm(x):
        mu = x.mean(-1, keepdims=True)
        var = ((x - mu) ** 2).mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(var + 1e-5)

    lat = np.asarray(latent, np.float64).T
    T = lat.shape[0]
    lat = swiglu_conv("audio_input_proj.2", silu(conv1d_ref(W, "audio_input_proj.0", lat, 1)))
    te = _lin(W, "t_embed.mlp.2", silu(_lin(W, "t_embed.mlp.0", timestep_embedding_ref(t, H, cfg["t_max_period"]))))
    clip = swiglu_conv("clip_input_proj.2", silu(_lin(W, "clip_input_proj.0", clip)))
    Sc = clip.shape[0]
    sync = np.asarray(sync, np.float64)
    Ss = sync.shape[0]
    pos = np.asarray(W["sync_pos_emb"], np.float64)                   # (8, sync_dim)
    sync = sync + pos[np.arange(Ss) % 8]
    sync = swiglu_conv("sync_input_proj.2", silu(conv1d_ref(W, "sync_input_proj.0", sync, 3)))
    txt_pad = np.zeros((cfg["text_seq"], cfg["t5_dim"]))
    if text_pad_left:
        txt_pad[:, cfg["t5_dim"] - cfg["clip_dim"]:] = text
    else:
        txt_pad[:, :cfg["clip_dim"]] = text
    seq = [txt_pad, np.asarray(t5, np.float64)]
    txt = swiglu_lin("text_input_proj.2", silu(_lin(W, "text_input_proj.0", np.concatenate(seq))))
    gvec = _lin(W, "clip_cond_proj", clip.mean(0)) + _lin(W, "text_cond_proj", g)
    gc = swiglu_lin("global_cond_mlp", gvec) + te
    idx = (np.floor(np.arange(T) * Ss / T) if sync_index_no_half else np.floor((np.arange(T) + 0.5) * Ss / T)).astype(int)
    ext = sync[idx] + gc
    s_ext, s_gc = silu(ext), silu(gc)
    ang_l = rope_angles_ggml(T, hd, cfg["rope_theta"])
    ang_c = rope_angles_ggml(Sc, hd, cfg["rope_theta"], 1.0 if clip_rope_unscaled else T / Sc)

    def pre_attn(p, x, cond, ang, pre_only):
        mod = _lin(W, p + ".adaLN_modulation.1", cond)          # (S or 1, n H)
        mod = np.broadcast_to(mod.reshape(-1, mod.shape[-1]), (x.shape[0], mod.shape[-1]))
        ch = [mod[:, i * H:(i + 1) * H] for i in range(2 if pre_only else 6)]
        shift, scale = (ch[1], ch[0]) if swap_shift_scale else (ch[0], ch[1])
        xn = layer_norm(x) * (1.0 + scale) + shift
        qkv = _lin(W, p + ".attn.qkv", xn).reshape(x.shape[0], nh, hd, 3)
        q, k, v = qkv[..., 0], qkv[..., 1], qkv[..., 2]
        q = q / np.sqrt((q * q).mean(-1, keepdims=True) + 1e-6) * np.asarray(W[p + ".attn.q_norm.weight"], np.float64)
        k = k / np.sqrt((k * k).mean(-1, keepdims=True) + 1e-6) * np.asarray(W[p + ".attn.k_norm.weight"], np.float64)
        if ang is not None:
            q, k = rope_apply(q, ang), rope_apply(k, ang)
        return q, k, v, ch

    def attend(qs, ks, vs):
        q, k, v = (np.concatenate(a, axis=0) for a in (qs, ks, vs))
        s = np.einsum("qhd,khd->hqk", q, k) / np.sqrt(hd)
        s = s - s.max(-1, keepdims=True)
        pr = np.exp(s)
        pr /= pr.sum(-1, keepdims=True)
        return np.einsum("hqk,khd->qhd", pr, v).reshape(q.shape[0], H)

    def post_attn(p, x, o, ch, conv):
        l1 = conv1d_ref(W, p + ".linear1", o, 1) if conv else _lin(W, p + ".linear1", o)
        x = x + l1 * ch[2]
        r = layer_norm(x) * (1.0 + ch[4]) + ch[3]
        f = swiglu_conv(p + ".ffn", r) if conv else swiglu_lin(p + ".ffn", r)
        return x + f * ch[gate_mlp_index]

    lat_cond = s_gc[None, :] if latent_cond_global else s_ext
    for i in range(nj):
        pre_only = i == nj - 1
        pl, pc, pt = (f"joint_blocks.{i}.{s}_block" for s in ("latent", "clip", "text"))
        ql, kl, vl, chl = pre_attn(pl, lat, lat_cond, ang_l, False)
        qc, kc, vc, chc = pre_attn(pc, clip, s_gc[None, :], ang_c, pre_only)
        qt, kt, vt, cht = pre_attn(pt, txt, s_gc[None, :], None, pre_only)
        o = attend([ql, qc, qt], [kl, kc, kt], [vl, vc, vt])
        lat = post_attn(pl, lat, o[:T], chl, True)
        if not pre_only:
            if not clip_frozen:
                clip = post_attn(pc, clip, o[T:T + Sc], chc, True)
            txt = post_attn(pt, txt, o[T + Sc:T + Sc + X], cht, False)
    for i in range(cfg["fused_depth"]):
        p = f"fused_blocks.{i}"
        q, k, v, ch = pre_attn(p, lat, lat_cond, ang_l, False)
        lat = post_attn(p, lat, attend([q], [k], [v]), ch, True)
    fm = _lin(W, "final_layer.adaLN_modulation.1", lat_cond)
    fm = np.broadcast_to(fm.reshape(-1, 2 * H), (T, 2 * H))
    fx = layer_norm(lat) * (1.0 + fm[:, H:]) + fm[:, :H]
    return conv1d_ref(W, "final_layer.conv", fx, 3)


def mmdit_sample_ref(W, cfg, noise, clip, sync, text, t5, g, steps, cfg_scale):
    """ts_dit::sample (src/mmdit.cpp:344-376) over mmdit_forward_ref: the
    unconditional forward on the learned empties (stored (clip_dim, 77) /
    (t5_dim, 77) in ggml order, i.e. token rows) and a zero global text
    feature; noise (L, T) -> (x (L, T), flow0 (L, T))."""
    x = np.asarray(noise, np.float64).copy()
    es = np.asarray(W["empty_string_feat"], np.float64)
    et = np.asarray(W["empty_t5_feat"], np.float64)
    zg = np.zeros(cfg["clip_dim"])
    f = np.float32
    flow0 = None
    for s in range(steps):
        t_curr = float(f(1.0) - f(s) / f(steps))
        t_next = float(f(1.0) - f(s + 1) / f(steps))
        dt = float(f(f(t_next) - f(t_curr)))
        fc = mmdit_forward_ref(W, cfg, x, t_curr, clip, sync, text, t5, g).T
        fu = mmdit_forward_ref(W, cfg, x, t_curr, clip, sync, es, et, zg).T
        v = fu + (fc - fu) * cfg_scale
        if s == 0:
            flow0 = v
        x = x + dt * v
    return x, flow0
