/*
 * tsk_oracle_dit.c — CPU restatement of one MM-DiT flow evaluation and of the
 * CFG Euler sampler, composed from the ggml-semantics ops of tsk_oracle.c.
 * TEST INFRASTRUCTURE ONLY (checker + timed CPU baseline).
 *
 * Follows the structure of ts_dit::forward (src/mmdit.cpp:119-342):
 *   t-embedding (host sin/cos, :305-314) -> t_embed MLP (:158-160);
 *   per block pre_attn (:203-225): adaLN lin on silu(cond) -> chunk (:209-216)
 *     -> LayerNorm eps 1e-5 (:59) * (1+scale) + shift (:55-57, :218)
 *     -> qkv lin (:219) -> split_qkv with channel 3*(h*64+d)+j (:67-76)
 *     -> rms_norm*w on q,k (:221-222) -> rope NORMAL on non-text (:223);
 *   joint attention over concat(latent, text) (:251-256), split back (:258-260);
 *   post_attn (:226-235): x += linear1(o)*gate_msa; x += mlp(mod(LN(x)))*gate_mlp;
 *   last joint block: text stream pre_only (:240, :262);
 *   fused blocks on the latent stream (:275-281); final layer (:285-289);
 *   sampler (:344-376): t = 1 - s/steps, v = u + cfg*(c - u), x += dt*v.
 * with the benchmarked block shape: linear projections, GELU(tanh) MLP of
 * width mlp_hidden, two streams (latent, text), adaLN conditioned on the
 * timestep embedding.
 */
#include "tsk_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* a weight: f32 values, or (q8) ggml Q8_0 blocks [ne1][ne0 / 32] */
typedef struct { char name[96]; int64_t ne[2]; float *data; uint8_t *q8; } orc_w;

/* the Q8_0 driver's Q8_0 matrices: the block projections */
static int is_block_proj(const char *name) {
    return strstr(name, ".attn.qkv.weight") || strstr(name, ".linear1.weight") || strstr(name, ".ffn.fc1.weight") ||
           strstr(name, ".ffn.fc2.weight");
}

struct orc_dit {
    tsk_dit_config cfg;
    int nw, capw;
    orc_w *w;
};

static void add_w(orc_dit *d, const char *name, int64_t ne0, int64_t ne1) {
    if (d->nw == d->capw) {
        d->capw = d->capw ? 2 * d->capw : 64;
        d->w = (orc_w *) realloc(d->w, sizeof(orc_w) * d->capw);
    }
    orc_w *w = &d->w[d->nw++];
    snprintf(w->name, sizeof(w->name), "%s", name);
    w->ne[0] = ne0; w->ne[1] = ne1;
    w->data = (float *) calloc((size_t) (ne0 * ne1), sizeof(float));
    w->q8 = d->cfg.weight_type == TSK_TYPE_Q8_0 && is_block_proj(name)
                ? (uint8_t *) calloc((size_t) (ne0 / 32 * ne1), 34) : NULL;
}

static void add_block(orc_dit *d, const char *p, int pre_only) {
    const tsk_dit_config *c = &d->cfg;
    const int H = c->hidden;
    char nm[96];
#define W2(suffix, a, b) do { snprintf(nm, sizeof(nm), "%s.%s", p, suffix); add_w(d, nm, a, b); } while (0)
    W2("adaLN_modulation.1.weight", H, (pre_only ? 2 : 6) * H);
    W2("adaLN_modulation.1.bias", (pre_only ? 2 : 6) * H, 1);
    W2("attn.qkv.weight", H, 3 * H);
    W2("attn.qkv.bias", 3 * H, 1);
    W2("attn.q_norm.weight", c->head_dim, 1);
    W2("attn.k_norm.weight", c->head_dim, 1);
    if (!pre_only) {
        W2("linear1.weight", H, H);
        W2("linear1.bias", H, 1);
        W2("ffn.fc1.weight", H, c->mlp_hidden);
        W2("ffn.fc1.bias", c->mlp_hidden, 1);
        W2("ffn.fc2.weight", c->mlp_hidden, H);
        W2("ffn.fc2.bias", H, 1);
    }
#undef W2
}

orc_dit *orc_dit_create(const tsk_dit_config *cfg) {
    orc_dit *d = (orc_dit *) calloc(1, sizeof(orc_dit));
    d->cfg = *cfg;
    const int H = cfg->hidden, nj = cfg->depth - cfg->fused_depth;
    add_w(d, "audio_input_proj.weight", cfg->latent_dim, H);
    add_w(d, "audio_input_proj.bias", H, 1);
    add_w(d, "t_embed.mlp.0.weight", H, H);
    add_w(d, "t_embed.mlp.0.bias", H, 1);
    add_w(d, "t_embed.mlp.2.weight", H, H);
    add_w(d, "t_embed.mlp.2.bias", H, 1);
    char p[96];
    for (int i = 0; i < nj; ++i) {
        snprintf(p, sizeof(p), "joint_blocks.%d.latent_block", i); add_block(d, p, 0);
        snprintf(p, sizeof(p), "joint_blocks.%d.text_block", i);   add_block(d, p, i == nj - 1);
    }
    for (int i = 0; i < cfg->fused_depth; ++i) {
        snprintf(p, sizeof(p), "fused_blocks.%d", i); add_block(d, p, 0);
    }
    add_w(d, "final_layer.adaLN_modulation.1.weight", H, 2 * H);
    add_w(d, "final_layer.adaLN_modulation.1.bias", 2 * H, 1);
    add_w(d, "final_layer.linear.weight", H, cfg->latent_dim);
    add_w(d, "final_layer.linear.bias", cfg->latent_dim, 1);
    return d;
}

void orc_dit_destroy(orc_dit *d) {
    if (!d) return;
    for (int i = 0; i < d->nw; ++i) { free(d->w[i].data); free(d->w[i].q8); }
    free(d->w); free(d);
}

int orc_dit_n_tensors(const orc_dit *d) { return d->nw; }

int orc_dit_tensor_info(const orc_dit *d, int i, const char **name, int64_t *ne0, int64_t *ne1) {
    if (i < 0 || i >= d->nw) return TSK_ERR_INVALID_ARG;
    *name = d->w[i].name;
    *ne0 = d->w[i].ne[0];
    *ne1 = d->w[i].ne[1];
    return TSK_OK;
}

static orc_w *find_w(orc_dit *d, const char *name) {
    for (int i = 0; i < d->nw; ++i) if (!strcmp(d->w[i].name, name)) return &d->w[i];
    fprintf(stderr, "orc_dit: missing tensor %s\n", name);
    abort();
}

/* f32 values; a Q8_0 weight is quantized with ggml's reference quantizer
 * (quantize_row_q8_0_ref: id = 1 / d, round half away) */
int orc_dit_set_tensor(orc_dit *d, const char *name, const float *src, int64_t n) {
    for (int i = 0; i < d->nw; ++i) {
        if (strcmp(d->w[i].name, name)) continue;
        if (n != d->w[i].ne[0] * d->w[i].ne[1]) return TSK_ERR_SHAPE;
        memcpy(d->w[i].data, src, sizeof(float) * (size_t) n);
        if (d->w[i].q8) orc_quantize_q8_0(src, d->w[i].q8, n, ORC_Q8_CPU_REF);
        return TSK_OK;
    }
    return TSK_ERR_INVALID_ARG;
}

/* ggml Q8_0 blocks of a Q8_0 weight, as stored */
int orc_dit_set_tensor_q8_0(orc_dit *d, const char *name, const void *blocks, size_t nbytes) {
    for (int i = 0; i < d->nw; ++i) {
        if (strcmp(d->w[i].name, name)) continue;
        if (!d->w[i].q8) return TSK_ERR_TYPE;
        if (nbytes != (size_t) (d->w[i].ne[0] / 32 * d->w[i].ne[1]) * 34) return TSK_ERR_SHAPE;
        memcpy(d->w[i].q8, blocks, nbytes);
        return TSK_OK;
    }
    return TSK_ERR_INVALID_ARG;
}

/* y[N, M] = W[K, M] x[N, K] + b  (ggml_mul_mat + ggml_add, mmdit.cpp:12-16).
 * act_bf16 rounds x to bf16 first, as ggml does for a BF16 weight, for the
 * per-block projections (attn.qkv, linear1, ffn.fc1, ffn.fc2). The thin
 * conditioning / input / output projections keep F32 activations: that is
 * the precision policy of the device path (their bf16 rounding alone moves a
 * 21-block step by ~2.9e-3 rel-L2 from the F32 path with random weights). */
static void lin(orc_dit *d, const char *wname, const char *bname, const float *x, int64_t N,
                float *y, int act_bf16) {
    orc_w *w = find_w(d, wname);
    orc_w *b = bname ? find_w(d, bname) : NULL;
    const int64_t K = w->ne[0], M = w->ne[1];
    tsk_tensor ta = { TSK_TYPE_F32, {K, M, 1, 1}, {4, 4 * K, 4 * K * M, 4 * K * M}, w->data };
    tsk_tensor tb = { TSK_TYPE_F32, {K, N, 1, 1}, {4, 4 * K, 4 * K * N, 4 * K * N}, (void *) x };
    tsk_tensor td = { TSK_TYPE_F32, {M, N, 1, 1}, {4, 4 * M, 4 * M * N, 4 * M * N}, y };
    tsk_tensor tbias = { TSK_TYPE_F32, {M, 1, 1, 1}, {4, 4 * M, 4 * M, 4 * M}, b ? b->data : NULL };
    float *xr = NULL;
    const int block_proj = strstr(wname, ".attn.qkv.") || strstr(wname, ".linear1.") || strstr(wname, ".ffn.fc");
    if (w->q8) {
        /* Q8_0 weight: ggml_mul_mat quantizes x to Q8_0 (the x86 path) */
        ta.type = TSK_TYPE_Q8_0;
        ta.nb[0] = 34; ta.nb[1] = (size_t) (K / 32) * 34; ta.nb[2] = ta.nb[3] = ta.nb[1] * (size_t) M;
        ta.data = w->q8;
    } else if (act_bf16 && block_proj) {
        xr = (float *) malloc(sizeof(float) * (size_t) (K * N));
        for (int64_t i = 0; i < K * N; ++i) xr[i] = orc_bf16_to_fp32(orc_fp32_to_bf16(x[i]));
        tb.data = xr;
    }
    orc_mul_mat(&ta, &tb, b ? &tbias : NULL, &td);
    free(xr);
}

/* LayerNorm eps (mmdit.cpp:59) then modulate x*(1+scale)+shift (mmdit.cpp:55-57);
 * shift/scale rows are per batch item (rows_per_b rows each). */
static void ln_modulate(const float *x, int64_t rows, int64_t H, int64_t rows_per_b,
                        const float *mod, int64_t mod_stride, int shift_i, int scale_i,
                        float eps, float *y) {
    tsk_tensor tx = { TSK_TYPE_F32, {H, rows, 1, 1}, {4, 4 * H, 4 * H * rows, 4 * H * rows}, (void *) x };
    tsk_tensor ty = { TSK_TYPE_F32, {H, rows, 1, 1}, {4, 4 * H, 4 * H * rows, 4 * H * rows}, y };
    orc_norm(&tx, eps, &ty);
    for (int64_t r = 0; r < rows; ++r) {
        const float *m = mod + (r / rows_per_b) * mod_stride;
        const float *sh = m + shift_i * H, *sc = m + scale_i * H;
        for (int64_t i = 0; i < H; ++i) y[r * H + i] = y[r * H + i] * (sc[i] + 1.0f) + sh[i];
    }
}

typedef struct {
    float *q, *k, *v;       /* [rows, n_head, head_dim] after norm/rope */
    float *mod;             /* [B, nmod*H] */
    int nmod;
} stream_state;

/* pre_attn (mmdit.cpp:203-225) for one stream of `rows` = B*S rows */
static void pre_attn(orc_dit *d, const char *p, const float *x, int B, int S, const float *silu_c,
                     int rope, int pre_only, stream_state *st, int act_bf16) {
    const tsk_dit_config *c = &d->cfg;
    const int64_t H = c->hidden, nh = c->n_head, hd = c->head_dim, rows = (int64_t) B * S;
    char wn[128], bn[128];
    st->nmod = pre_only ? 2 : 6;
    st->mod = (float *) malloc(sizeof(float) * (size_t) (B * st->nmod * H));
    snprintf(wn, sizeof(wn), "%s.adaLN_modulation.1.weight", p);
    snprintf(bn, sizeof(bn), "%s.adaLN_modulation.1.bias", p);
    lin(d, wn, bn, silu_c, B, st->mod, act_bf16);
    float *xn = (float *) malloc(sizeof(float) * (size_t) (rows * H));
    ln_modulate(x, rows, H, S, st->mod, st->nmod * H, 0, 1, c->ln_eps, xn);
    float *qkv = (float *) malloc(sizeof(float) * (size_t) (rows * 3 * H));
    snprintf(wn, sizeof(wn), "%s.attn.qkv.weight", p);
    snprintf(bn, sizeof(bn), "%s.attn.qkv.bias", p);
    lin(d, wn, bn, xn, rows, qkv, act_bf16);
    st->q = (float *) malloc(sizeof(float) * (size_t) (rows * H));
    st->k = (float *) malloc(sizeof(float) * (size_t) (rows * H));
    st->v = (float *) malloc(sizeof(float) * (size_t) (rows * H));
    /* split_qkv: channel 3*(h*hd+d)+j (mmdit.cpp:67-76) */
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < H; ++i) {
            st->q[r * H + i] = qkv[r * 3 * H + 3 * i + 0];
            st->k[r * H + i] = qkv[r * 3 * H + 3 * i + 1];
            st->v[r * H + i] = qkv[r * 3 * H + 3 * i + 2];
        }
    free(qkv); free(xn);
    snprintf(wn, sizeof(wn), "%s.attn.q_norm.weight", p);
    orc_w *qn = find_w(d, wn);
    snprintf(wn, sizeof(wn), "%s.attn.k_norm.weight", p);
    orc_w *kn = find_w(d, wn);
    /* [hd, nh, S] per batch item for rms_norm / rope */
    int32_t *pos = (int32_t *) malloc(sizeof(int32_t) * (size_t) S);
    for (int i = 0; i < S; ++i) pos[i] = i;
    for (int b = 0; b < B; ++b) {
        float *bufs[2] = { st->q + (int64_t) b * S * H, st->k + (int64_t) b * S * H };
        float *ws[2] = { qn->data, kn->data };
        for (int j = 0; j < 2; ++j) {
            tsk_tensor t = { TSK_TYPE_F32, {hd, nh, S, 1}, {4, 4 * hd, 4 * H, 4 * H * S}, bufs[j] };
            orc_rms_norm_mul(&t, ws[j], c->qk_eps, &t);
            if (rope) orc_rope_ext(&t, pos, (int) hd, c->rope_theta, 1.0f, &t);
        }
    }
    free(pos);
}

/* attention over the concatenation of nseg streams for every batch item
 * (mmdit.cpp:85-95, :251-256): K/V cast to F16 when kv_f16. Output rows are
 * written back per stream into o[s] ([B*S_s, H]). */
static void joint_attention(orc_dit *d, int B, int nseg, const int *S, stream_state **st, float **o,
                            int kv_f16) {
    const tsk_dit_config *c = &d->cfg;
    const int64_t H = c->hidden, nh = c->n_head, hd = c->head_dim;
    int64_t N = 0;
    for (int s = 0; s < nseg; ++s) N += S[s];
    float *Q = (float *) malloc(sizeof(float) * (size_t) (N * H));
    float *K = (float *) malloc(sizeof(float) * (size_t) (N * H));
    float *V = (float *) malloc(sizeof(float) * (size_t) (N * H));
    uint16_t *K16 = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) (N * H));
    uint16_t *V16 = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) (N * H));
    float *O = (float *) malloc(sizeof(float) * (size_t) (N * H));
    for (int b = 0; b < B; ++b) {
        /* permute to [hd, N, nh] (mmdit.cpp:88-90) */
        int64_t off = 0;
        for (int s = 0; s < nseg; ++s) {
            for (int64_t n = 0; n < S[s]; ++n)
                for (int64_t h = 0; h < nh; ++h)
                    for (int64_t e = 0; e < hd; ++e) {
                        const int64_t src = ((int64_t) b * S[s] + n) * H + h * hd + e;
                        const int64_t dst = (h * N + off + n) * hd + e;
                        Q[dst] = st[s]->q[src]; K[dst] = st[s]->k[src]; V[dst] = st[s]->v[src];
                    }
            off += S[s];
        }
        tsk_tensor tq = { TSK_TYPE_F32, {hd, N, nh, 1}, {4, 4 * hd, 4 * hd * N, 4 * hd * N * nh}, Q };
        tsk_tensor tk = { TSK_TYPE_F32, {hd, N, nh, 1}, {4, 4 * hd, 4 * hd * N, 4 * hd * N * nh}, K };
        tsk_tensor tv = tk; tv.data = V;
        if (kv_f16) {
            orc_fp32_to_fp16_row(K, K16, N * H);
            orc_fp32_to_fp16_row(V, V16, N * H);
            tk.type = TSK_TYPE_F16; tk.nb[0] = 2; tk.nb[1] = 2 * hd; tk.nb[2] = 2 * hd * N; tk.nb[3] = 2 * hd * N * nh; tk.data = K16;
            tv = tk; tv.data = V16;
        }
        tsk_tensor to = { TSK_TYPE_F32, {hd, nh, N, 1}, {4, 4 * hd, 4 * H, 4 * H * N}, O };
        orc_flash_attn_ext(&tq, &tk, &tv, NULL, 1.0f / sqrtf((float) hd), 0.0f, 0.0f, 0, &to);
        off = 0;
        for (int s = 0; s < nseg; ++s) {
            memcpy(o[s] + (int64_t) b * S[s] * H, O + off * H, sizeof(float) * (size_t) (S[s] * H));
            off += S[s];
        }
    }
    free(Q); free(K); free(V); free(K16); free(V16); free(O);
}

/* post_attn (mmdit.cpp:226-235) with linear projections and GELU(tanh) MLP */
static void post_attn(orc_dit *d, const char *p, float *x, int B, int S, const float *o,
                      const stream_state *st, int act_bf16) {
    const tsk_dit_config *c = &d->cfg;
    const int64_t H = c->hidden, F = c->mlp_hidden, rows = (int64_t) B * S, ms = 6 * H;
    char wn[128], bn[128];
    float *l1 = (float *) malloc(sizeof(float) * (size_t) (rows * H));
    snprintf(wn, sizeof(wn), "%s.linear1.weight", p);
    snprintf(bn, sizeof(bn), "%s.linear1.bias", p);
    lin(d, wn, bn, o, rows, l1, act_bf16);
    for (int64_t r = 0; r < rows; ++r) {
        const float *g = st->mod + (r / S) * ms + 2 * H;
        for (int64_t i = 0; i < H; ++i) x[r * H + i] += l1[r * H + i] * g[i];
    }
    float *rn = l1;
    ln_modulate(x, rows, H, S, st->mod, ms, 3, 4, c->ln_eps, rn);
    float *h = (float *) malloc(sizeof(float) * (size_t) (rows * F));
    snprintf(wn, sizeof(wn), "%s.ffn.fc1.weight", p);
    snprintf(bn, sizeof(bn), "%s.ffn.fc1.bias", p);
    lin(d, wn, bn, rn, rows, h, act_bf16);
    for (int64_t i = 0; i < rows * F; ++i) h[i] = orc_gelu_tanh(h[i]);
    float *f = (float *) malloc(sizeof(float) * (size_t) (rows * H));
    snprintf(wn, sizeof(wn), "%s.ffn.fc2.weight", p);
    snprintf(bn, sizeof(bn), "%s.ffn.fc2.bias", p);
    lin(d, wn, bn, h, rows, f, act_bf16);
    for (int64_t r = 0; r < rows; ++r) {
        const float *g = st->mod + (r / S) * ms + 5 * H;
        for (int64_t i = 0; i < H; ++i) x[r * H + i] += f[r * H + i] * g[i];
    }
    free(l1); free(h); free(f);
}

static void free_stream(stream_state *s) { free(s->q); free(s->k); free(s->v); free(s->mod); }

int orc_dit_forward(orc_dit *d, int B, int T, const float *latent, const float *t,
                    const float *text, float *flow, int act_bf16, int kv_f16) {
    const tsk_dit_config *c = &d->cfg;
    const int64_t H = c->hidden, L = c->latent_dim, St = c->text_seq;
    const int nj = c->depth - c->fused_depth;
    /* timestep frequency embedding (mmdit.cpp:305-314) */
    float *temb = (float *) malloc(sizeof(float) * (size_t) (B * H));
    const int half = (int) H / 2;
    const float fscale_t = 10000.0f / c->t_max_period;
    for (int b = 0; b < B; ++b)
        for (int kk = 0; kk < half; ++kk) {
            const float fr = fscale_t * powf(10000.0f, -2.0f * (float) kk / (float) H);
            temb[b * H + kk] = cosf(t[b] * fr);
            temb[b * H + half + kk] = sinf(t[b] * fr);
        }
    float *te = (float *) malloc(sizeof(float) * (size_t) (B * H));
    float *cvec = (float *) malloc(sizeof(float) * (size_t) (B * H));
    lin(d, "t_embed.mlp.0.weight", "t_embed.mlp.0.bias", temb, B, te, act_bf16);
    for (int64_t i = 0; i < B * H; ++i) te[i] = orc_silu(te[i]);
    lin(d, "t_embed.mlp.2.weight", "t_embed.mlp.2.bias", te, B, cvec, act_bf16);
    /* adaLN input: silu(cond) (mmdit.cpp:209) */
    float *sc = te;
    for (int64_t i = 0; i < B * H; ++i) sc[i] = orc_silu(cvec[i]);

    float *lat = (float *) malloc(sizeof(float) * (size_t) (B * T * H));
    lin(d, "audio_input_proj.weight", "audio_input_proj.bias", latent, (int64_t) B * T, lat, act_bf16);
    float *txt = (float *) malloc(sizeof(float) * (size_t) (B * St * H));
    memcpy(txt, text, sizeof(float) * (size_t) (B * St * H));

    char p[96];
    for (int i = 0; i < nj; ++i) {
        const int pre_only = i == nj - 1;
        stream_state sl, stt;
        snprintf(p, sizeof(p), "joint_blocks.%d.latent_block", i);
        pre_attn(d, p, lat, B, T, sc, 1, 0, &sl, act_bf16);
        snprintf(p, sizeof(p), "joint_blocks.%d.text_block", i);
        pre_attn(d, p, txt, B, (int) St, sc, 0, pre_only, &stt, act_bf16);
        float *ol = (float *) malloc(sizeof(float) * (size_t) (B * T * H));
        float *ot = (float *) malloc(sizeof(float) * (size_t) (B * St * H));
        int S2[2] = { T, (int) St };
        stream_state *ss[2] = { &sl, &stt };
        float *os[2] = { ol, ot };
        joint_attention(d, B, 2, S2, ss, os, kv_f16);
        snprintf(p, sizeof(p), "joint_blocks.%d.latent_block", i);
        post_attn(d, p, lat, B, T, ol, &sl, act_bf16);
        if (!pre_only) {
            snprintf(p, sizeof(p), "joint_blocks.%d.text_block", i);
            post_attn(d, p, txt, B, (int) St, ot, &stt, act_bf16);
        }
        free(ol); free(ot); free_stream(&sl); free_stream(&stt);
    }
    for (int i = 0; i < c->fused_depth; ++i) {
        stream_state s1;
        snprintf(p, sizeof(p), "fused_blocks.%d", i);
        pre_attn(d, p, lat, B, T, sc, 1, 0, &s1, act_bf16);
        float *o1 = (float *) malloc(sizeof(float) * (size_t) (B * T * H));
        int S1[1] = { T };
        stream_state *ss[1] = { &s1 };
        float *os[1] = { o1 };
        joint_attention(d, B, 1, S1, ss, os, kv_f16);
        post_attn(d, p, lat, B, T, o1, &s1, act_bf16);
        free(o1); free_stream(&s1);
    }
    /* final layer (mmdit.cpp:285-289) with a linear output projection */
    float *fmod = (float *) malloc(sizeof(float) * (size_t) (B * 2 * H));
    lin(d, "final_layer.adaLN_modulation.1.weight", "final_layer.adaLN_modulation.1.bias", sc, B, fmod, act_bf16);
    float *fx = (float *) malloc(sizeof(float) * (size_t) (B * T * H));
    ln_modulate(lat, (int64_t) B * T, H, T, fmod, 2 * H, 0, 1, c->ln_eps, fx);
    lin(d, "final_layer.linear.weight", "final_layer.linear.bias", fx, (int64_t) B * T, flow, act_bf16);
    (void) L;
    free(temb); free(te); free(cvec); free(lat); free(txt); free(fmod); free(fx);
    return TSK_OK;
}

/* ts_dit::sample (mmdit.cpp:344-376) with cond/uncond batched as B=2. */
int orc_dit_sample(orc_dit *d, int T, const float *noise, const float *text_cond,
                   const float *text_uncond, int steps, float cfg_scale, float *out,
                   float *flow0, int act_bf16, int kv_f16) {
    const tsk_dit_config *c = &d->cfg;
    const int64_t L = c->latent_dim, TL = (int64_t) T * L, TX = (int64_t) c->text_seq * c->hidden;
    float *x2 = (float *) malloc(sizeof(float) * (size_t) (2 * TL));
    float *tx2 = (float *) malloc(sizeof(float) * (size_t) (2 * TX));
    float *f2 = (float *) malloc(sizeof(float) * (size_t) (2 * TL));
    memcpy(out, noise, sizeof(float) * (size_t) TL);
    memcpy(tx2, text_cond, sizeof(float) * (size_t) TX);
    memcpy(tx2 + TX, text_uncond, sizeof(float) * (size_t) TX);
    for (int s = 0; s < steps; ++s) {
        const float t_curr = 1.0f - (float) s / (float) steps;
        const float t_prev = 1.0f - (float) (s + 1) / (float) steps;
        const float dt = t_prev - t_curr;
        memcpy(x2, out, sizeof(float) * (size_t) TL);
        memcpy(x2 + TL, out, sizeof(float) * (size_t) TL);
        float tt[2] = { t_curr, t_curr };
        orc_dit_forward(d, 2, T, x2, tt, tx2, f2, act_bf16, kv_f16);
        for (int64_t i = 0; i < TL; ++i) {
            const float fc = f2[i], fu = f2[TL + i];
            const float v = fu + (fc - fu) * cfg_scale;
            if (s == 0 && flow0) flow0[i] = v;
            out[i] += dt * v;
        }
    }
    free(x2); free(tx2); free(f2);
    return TSK_OK;
}
