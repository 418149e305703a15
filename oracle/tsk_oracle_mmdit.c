/*
 * tsk_oracle_mmdit.c — CPU restatement of the reference's MM-DiT graph,
 * ts_dit::forward and ts_dit::sample (src/mmdit.cpp:119-376), node by node
 * with the ggml-semantics ops of tsk_oracle.c / tsk_oracle_conv.c.
 * TEST INFRASTRUCTURE ONLY: the checker of tsk_mmdit_forward /
 * tsk_mmdit_sample. One batch row per forward, as the reference runs it.
 *
 *   lat = convmlp(silu(conv_cl(audio_input_proj.0, latent^T)))       :150-155
 *   te  = lin(t_embed.mlp.2, silu(lin(t_embed.mlp.0, temb)))         :157-161
 *   clip = convmlp(silu(lin(clip_input_proj.0, clip_f)))             :163-167
 *   sync = convmlp(silu(conv_cl k7 p3(sync_f + pos_emb[s % 8])))     :168-177
 *   text = mlp(silu(lin(text_input_proj.0, [pad(text_f) | t5])))     :179-183
 *   gc = mlp(global_cond_mlp, lin(clip_cond, mean(clip)) + lin(text_cond, g)) + te
 *   extended_c = sync[nearest-exact(t)] + gc                         :184-196
 *   joint blocks (latent / clip / text; last clip, text pre_only), fused
 *   blocks, final layer                                              :203-289
 *   sampler: v = u + cfg (c - u), x += dt v                          :344-376
 *
 * Each weight has a stored type, as the converters write the files
 * (convert/quantize_gguf.py:9-15): under weight_type BF16 every matrix is
 * BF16 but the t_embed MLP ("_emb" names) F32; under Q8_0 the 2-D linears
 * with ne0 % 32 == 0 and no "_emb" / "norm" / "empty" in their names are
 * Q8_0 and the convolutions F32; under F32 all are F32 (orc_mmdit_set_type
 * overrides one tensor's type, as a GGUF file may). With act_bf16 the
 * products run in the stored types (ggml_mul_mat converts its src1 to the
 * weight's vec_dot type: bf16 rounding, Q8_0 quantization); without, every
 * product is F32 on the same weight values (the "GGML F32 path"; a Q8_0
 * weight as its dequantized values).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tsk_oracle.h"

enum { MK_LIN = 0, MK_CONV = 1, MK_VEC = 2 };

typedef struct {
    char name[200];
    int64_t ne[3];
    int kind, type;    /* type: TSK_TYPE_F32 / BF16 / Q8_0 as stored */
    float *data;       /* f32 values in ggml order (a Q8_0 tensor's dequantized values) */
    uint16_t *bf;      /* bf16 copy of a BF16 matrix */
    uint8_t *q8;       /* Q8_0 blocks of a Q8_0 matrix, ne[1] rows of ne[0] / 32 */
} mw;

/* stage outputs of the last forward, concatenated over its batch rows (the
 * reference's dbg map, mmdit.cpp:333-336) */
#define ORC_NSTAGE 16
typedef struct { char name[24]; float *data; int64_t n; } stage;

struct orc_mmdit {
    tsk_mmdit_config cfg;
    int nw, capw;
    mw *w;
    int nst;
    stage st[ORC_NSTAGE];
};

static void stage_reset(orc_mmdit *m) {
    for (int i = 0; i < m->nst; ++i) free(m->st[i].data);
    m->nst = 0;
}

/* append n floats to stage `name` */
static void stage_add(orc_mmdit *m, const char *name, const float *x, int64_t n) {
    stage *e = NULL;
    for (int i = 0; i < m->nst; ++i) if (!strcmp(m->st[i].name, name)) e = &m->st[i];
    if (!e) {
        if (m->nst == ORC_NSTAGE) return;
        e = &m->st[m->nst++];
        snprintf(e->name, sizeof(e->name), "%s", name);
        e->data = NULL;
        e->n = 0;
    }
    e->data = (float *) realloc(e->data, sizeof(float) * (size_t) (e->n + n));
    memcpy(e->data + e->n, x, sizeof(float) * (size_t) n);
    e->n += n;
}

int64_t orc_mmdit_stage_size(const orc_mmdit *m, const char *name) {
    for (int i = 0; i < m->nst; ++i) if (!strcmp(m->st[i].name, name)) return m->st[i].n;
    return -1;
}

int orc_mmdit_stage(const orc_mmdit *m, const char *name, float *out, int64_t n) {
    for (int i = 0; i < m->nst; ++i) {
        if (strcmp(m->st[i].name, name)) continue;
        if (n != m->st[i].n) return TSK_ERR_SHAPE;
        memcpy(out, m->st[i].data, sizeof(float) * (size_t) n);
        return TSK_OK;
    }
    return TSK_ERR_INVALID_ARG;
}

/* the stored type of a weight under a model-wide weight type (the
 * converters' rule, convert/quantize_gguf.py:9-15) */
static int rule_type(int wt, const mw *x) {
    if (x->kind == MK_VEC || wt == TSK_TYPE_F32) return TSK_TYPE_F32;
    const int emb = strstr(x->name, "_emb") != NULL;
    if (wt == TSK_TYPE_BF16) return emb ? TSK_TYPE_F32 : TSK_TYPE_BF16;
    if (x->kind == MK_CONV || emb || strstr(x->name, "norm") || strstr(x->name, "empty") || x->ne[0] % 32)
        return TSK_TYPE_F32;
    return TSK_TYPE_Q8_0;
}

static int64_t nel(const mw *x) { return x->ne[0] * x->ne[1] * x->ne[2]; }

/* (re)allocate the typed copy of a weight */
static void set_type(mw *x, int type) {
    free(x->bf); free(x->q8);
    x->bf = NULL; x->q8 = NULL;
    x->type = type;
    if (type == TSK_TYPE_BF16) x->bf = (uint16_t *) calloc((size_t) nel(x), sizeof(uint16_t));
    if (type == TSK_TYPE_Q8_0) x->q8 = (uint8_t *) calloc((size_t) (nel(x) / 32), 34);
}

static void addw(orc_mmdit *m, const char *name, int64_t a, int64_t b, int64_t c, int kind) {
    if (m->nw == m->capw) {
        m->capw = m->capw ? 2 * m->capw : 128;
        m->w = (mw *) realloc(m->w, sizeof(mw) * (size_t) m->capw);
    }
    mw *x = &m->w[m->nw++];
    memset(x, 0, sizeof(*x));
    snprintf(x->name, sizeof(x->name), "%s", name);
    x->ne[0] = a; x->ne[1] = b; x->ne[2] = c;
    x->kind = kind;
    x->data = (float *) calloc((size_t) (a * b * c), sizeof(float));
    set_type(x, rule_type(m->cfg.weight_type, x));
}

static void add_lin(orc_mmdit *m, const char *p, int in, int out, int bias) {
    char nm[200];
    snprintf(nm, sizeof(nm), "%s.weight", p); addw(m, nm, in, out, 1, MK_LIN);
    if (bias) { snprintf(nm, sizeof(nm), "%s.bias", p); addw(m, nm, out, 1, 1, MK_VEC); }
}

static void add_conv(orc_mmdit *m, const char *p, int kw, int in, int out, int bias) {
    char nm[200];
    snprintf(nm, sizeof(nm), "%s.weight", p); addw(m, nm, kw, in, out, MK_CONV);
    if (bias) { snprintf(nm, sizeof(nm), "%s.bias", p); addw(m, nm, out, 1, 1, MK_VEC); }
}

static void add_block(orc_mmdit *m, const char *p, int pre_only, int conv) {
    const int H = m->cfg.hidden, F = m->cfg.mlp_hidden;
    char nm[160];
    snprintf(nm, sizeof(nm), "%s.adaLN_modulation.1", p); add_lin(m, nm, H, (pre_only ? 2 : 6) * H, 1);
    snprintf(nm, sizeof(nm), "%s.attn.qkv", p); add_lin(m, nm, H, 3 * H, 1);
    snprintf(nm, sizeof(nm), "%s.attn.q_norm.weight", p); addw(m, nm, m->cfg.head_dim, 1, 1, MK_VEC);
    snprintf(nm, sizeof(nm), "%s.attn.k_norm.weight", p); addw(m, nm, m->cfg.head_dim, 1, 1, MK_VEC);
    if (pre_only) return;
    if (conv) {
        snprintf(nm, sizeof(nm), "%s.linear1", p); add_conv(m, nm, 3, H, H, 1);
        snprintf(nm, sizeof(nm), "%s.ffn.w1", p); add_conv(m, nm, 3, H, F, 0);
        snprintf(nm, sizeof(nm), "%s.ffn.w3", p); add_conv(m, nm, 3, H, F, 0);
        snprintf(nm, sizeof(nm), "%s.ffn.w2", p); add_conv(m, nm, 3, F, H, 0);
    } else {
        snprintf(nm, sizeof(nm), "%s.linear1", p); add_lin(m, nm, H, H, 1);
        snprintf(nm, sizeof(nm), "%s.ffn.w1", p); add_lin(m, nm, H, F, 0);
        snprintf(nm, sizeof(nm), "%s.ffn.w3", p); add_lin(m, nm, H, F, 0);
        snprintf(nm, sizeof(nm), "%s.ffn.w2", p); add_lin(m, nm, F, H, 0);
    }
}

/* the converter's names and shapes (convert/convert_thinksound.py:32,
 * docs/ARCHITECTURE.md section 6.1) */
orc_mmdit *orc_mmdit_create(const tsk_mmdit_config *cfg) {
    orc_mmdit *m = (orc_mmdit *) calloc(1, sizeof(orc_mmdit));
    m->cfg = *cfg;
    const int H = cfg->hidden, F = cfg->mlp_hidden, nj = cfg->depth - cfg->fused_depth;
    add_conv(m, "audio_input_proj.0", 3, cfg->latent_dim, H, 1);
    add_conv(m, "audio_input_proj.2.w1", 3, H, F, 0);
    add_conv(m, "audio_input_proj.2.w3", 3, H, F, 0);
    add_conv(m, "audio_input_proj.2.w2", 3, F, H, 0);
    add_lin(m, "clip_input_proj.0", cfg->clip_dim, H, 1);
    add_conv(m, "clip_input_proj.2.w1", 3, H, F, 0);
    add_conv(m, "clip_input_proj.2.w3", 3, H, F, 0);
    add_conv(m, "clip_input_proj.2.w2", 3, F, H, 0);
    add_conv(m, "sync_input_proj.0", 7, cfg->sync_dim, H, 1);
    add_conv(m, "sync_input_proj.2.w1", 3, H, F, 0);
    add_conv(m, "sync_input_proj.2.w3", 3, H, F, 0);
    add_conv(m, "sync_input_proj.2.w2", 3, F, H, 0);
    add_lin(m, "text_input_proj.0", cfg->t5_dim, H, 1);
    add_lin(m, "text_input_proj.2.w1", H, F, 0);
    add_lin(m, "text_input_proj.2.w3", H, F, 0);
    add_lin(m, "text_input_proj.2.w2", F, H, 0);
    add_lin(m, "text_cond_proj", cfg->clip_dim, H, 1);
    add_lin(m, "clip_cond_proj", H, H, 1);
    add_lin(m, "global_cond_mlp.w1", H, F, 0);
    add_lin(m, "global_cond_mlp.w3", H, F, 0);
    add_lin(m, "global_cond_mlp.w2", F, H, 0);
    addw(m, "sync_pos_emb", cfg->sync_dim, 8, 1, MK_VEC);
    add_lin(m, "t_embed.mlp.0", H, H, 1);
    add_lin(m, "t_embed.mlp.2", H, H, 1);
    char p[96];
    for (int i = 0; i < nj; ++i) {
        snprintf(p, sizeof(p), "joint_blocks.%d.latent_block", i); add_block(m, p, 0, 1);
        snprintf(p, sizeof(p), "joint_blocks.%d.clip_block", i);   add_block(m, p, i == nj - 1, 1);
        snprintf(p, sizeof(p), "joint_blocks.%d.text_block", i);   add_block(m, p, i == nj - 1, 0);
    }
    for (int i = 0; i < cfg->fused_depth; ++i) {
        snprintf(p, sizeof(p), "fused_blocks.%d", i); add_block(m, p, 0, 1);
    }
    add_lin(m, "final_layer.adaLN_modulation.1", H, 2 * H, 1);
    add_conv(m, "final_layer.conv", 7, H, cfg->latent_dim, 1);
    addw(m, "empty_string_feat", cfg->clip_dim, cfg->text_seq, 1, MK_VEC);
    addw(m, "empty_t5_feat", cfg->t5_dim, cfg->text_seq, 1, MK_VEC);
    return m;
}

void orc_mmdit_destroy(orc_mmdit *m) {
    if (!m) return;
    for (int i = 0; i < m->nw; ++i) { free(m->w[i].data); free(m->w[i].bf); free(m->w[i].q8); }
    stage_reset(m);
    free(m->w);
    free(m);
}

int orc_mmdit_n_tensors(const orc_mmdit *m) { return m->nw; }

int orc_mmdit_tensor_info(const orc_mmdit *m, int i, const char **name, int64_t ne[3], int *type) {
    if (i < 0 || i >= m->nw) return TSK_ERR_INVALID_ARG;
    *name = m->w[i].name;
    for (int j = 0; j < 3; ++j) ne[j] = m->w[i].ne[j];
    *type = m->w[i].type;
    return TSK_OK;
}

static mw *find_w(orc_mmdit *m, const char *name) {
    for (int i = 0; i < m->nw; ++i) if (!strcmp(m->w[i].name, name)) return &m->w[i];
    fprintf(stderr, "orc_mmdit: missing tensor %s\n", name);
    abort();
}

static mw *lookup(orc_mmdit *m, const char *name) {
    for (int i = 0; i < m->nw; ++i) if (!strcmp(m->w[i].name, name)) return &m->w[i];
    return NULL;
}

/* f32 values; a Q8_0 tensor is quantized with ggml's reference quantizer
 * (quantize_row_q8_0_ref) and keeps its dequantized values as data */
int orc_mmdit_set_tensor(orc_mmdit *m, const char *name, const float *src, int64_t n) {
    mw *x = lookup(m, name);
    if (!x) return TSK_ERR_INVALID_ARG;
    if (n != nel(x)) return TSK_ERR_SHAPE;
    if (x->type == TSK_TYPE_Q8_0) {
        orc_quantize_q8_0(src, x->q8, n, ORC_Q8_CPU_REF);
        orc_dequantize_q8_0(x->q8, x->data, n);
        return TSK_OK;
    }
    memcpy(x->data, src, sizeof(float) * (size_t) n);
    if (x->bf) orc_fp32_to_bf16_row(src, x->bf, n);
    return TSK_OK;
}

/* Q8_0 blocks as a GGUF file holds them */
int orc_mmdit_set_tensor_q8_0(orc_mmdit *m, const char *name, const void *blocks, size_t nbytes) {
    mw *x = lookup(m, name);
    if (!x) return TSK_ERR_INVALID_ARG;
    if (x->type != TSK_TYPE_Q8_0) return TSK_ERR_TYPE;
    if (nbytes != (size_t) (nel(x) / 32) * 34) return TSK_ERR_SHAPE;
    memcpy(x->q8, blocks, nbytes);
    orc_dequantize_q8_0(x->q8, x->data, nel(x));
    return TSK_OK;
}

/* the stored type of one weight (F32 for vectors; Q8_0 for 2-D weights with
 * ne0 % 32 == 0 only) */
int orc_mmdit_set_type(orc_mmdit *m, const char *name, int type) {
    mw *x = lookup(m, name);
    if (!x) return TSK_ERR_INVALID_ARG;
    const int ok = type == TSK_TYPE_F32 || (x->kind != MK_VEC && type == TSK_TYPE_BF16) ||
                   (x->kind == MK_LIN && type == TSK_TYPE_Q8_0 && x->ne[0] % 32 == 0);
    if (!ok) return TSK_ERR_TYPE;
    set_type(x, type);
    return TSK_OK;
}

/* ---- node helpers: activations are ggml [C, S] (C fastest), contiguous */

static tsk_tensor act(float *p, int64_t C, int64_t S) {
    tsk_tensor t = { TSK_TYPE_F32, {C, S, 1, 1}, {4, (size_t) (4 * C), (size_t) (4 * C * S), (size_t) (4 * C * S)}, p };
    return t;
}

/* a weight as ggml holds it: its stored type when act_bf16, else F32 */
static tsk_tensor wten(orc_mmdit *m, const char *name, int act_bf16) {
    mw *x = find_w(m, name);
    if (act_bf16 && x->type == TSK_TYPE_Q8_0) {
        const size_t row = (size_t) (x->ne[0] / 32) * 34;
        tsk_tensor t = { TSK_TYPE_Q8_0, {x->ne[0], x->ne[1], x->ne[2], 1},
                         {34, row, row * (size_t) x->ne[1], row * (size_t) (x->ne[1] * x->ne[2])}, x->q8 };
        return t;
    }
    const int bf = act_bf16 && x->type == TSK_TYPE_BF16;
    const size_t es = bf ? 2 : 4;
    tsk_tensor t = { bf ? TSK_TYPE_BF16 : TSK_TYPE_F32, {x->ne[0], x->ne[1], x->ne[2], 1},
                     {es, es * (size_t) x->ne[0], es * (size_t) (x->ne[0] * x->ne[1]),
                      es * (size_t) (x->ne[0] * x->ne[1] * x->ne[2])},
                     bf ? (void *) x->bf : (void *) x->data };
    return t;
}

static float *fbuf(int64_t n) { return (float *) calloc((size_t) n, sizeof(float)); }

/* lin (mmdit.cpp:12-16): y [M, S] = W x + b */
static void lin(orc_mmdit *m, const char *p, int bias, const float *x, int64_t K, int64_t S, float *y, int act_bf16) {
    char nm[160];
    snprintf(nm, sizeof(nm), "%s.weight", p);
    tsk_tensor w = wten(m, nm, act_bf16);
    const int64_t M = w.ne[1];
    tsk_tensor tx = act((float *) x, K, S), ty = act(y, M, S), tb;
    if (bias) { snprintf(nm, sizeof(nm), "%s.bias", p); tb = act(find_w(m, nm)->data, M, 1); }
    orc_mul_mat(&w, &tx, bias ? &tb : NULL, &ty);
}

/* conv_cl (mmdit.cpp:28-34): [IC, S] -> [OC, S], stride 1, padding p */
static void conv_cl(orc_mmdit *m, const char *p, int bias, const float *x, int64_t IC, int64_t S, int pad, float *y,
                    int act_bf16) {
    char nm[160];
    snprintf(nm, sizeof(nm), "%s.weight", p);
    tsk_tensor w = wten(m, nm, act_bf16);
    const int64_t OC = w.ne[2];
    tsk_tensor tx = act((float *) x, IC, S), ty = act(y, OC, S), tb;
    if (bias) { snprintf(nm, sizeof(nm), "%s.bias", p); tb = act(find_w(m, nm)->data, OC, 1); }
    orc_conv1d(&w, bias ? &tb : NULL, &tx, 1, pad, 1, &ty);
}

/* convmlp / mlp (mmdit.cpp:39-52) on [H, S] */
static void swiglu_mlp(orc_mmdit *m, const char *p, int conv, const float *x, int64_t C, int64_t S, float *y,
                       int act_bf16) {
    char n1[160], n3[160], n2[160];
    snprintf(n1, sizeof(n1), "%s.w1.weight", p);
    snprintf(n3, sizeof(n3), "%s.w3.weight", p);
    snprintf(n2, sizeof(n2), "%s.w2.weight", p);
    tsk_tensor w1 = wten(m, n1, act_bf16), w3 = wten(m, n3, act_bf16), w2 = wten(m, n2, act_bf16);
    const int64_t OC = conv ? w2.ne[2] : w2.ne[1];
    tsk_tensor tx = act((float *) x, C, S), ty = act(y, OC, S);
    if (conv) orc_conv_mlp_swiglu(&w1, &w3, &w2, &tx, &ty);
    else orc_mlp_swiglu(&w1, &w3, &w2, &tx, &ty);
}

static void silu_n(float *x, int64_t n) { for (int64_t i = 0; i < n; ++i) x[i] = orc_silu(x[i]); }

/* modulate(layernorm(x), shift, scale) (mmdit.cpp:55-59, :218): x [H, S];
 * shift / scale columns of mod (row stride ld) per token, or column 0 for
 * every token when per_token == 0 */
static void ln_mod(const float *x, int64_t H, int64_t S, const float *mod, int64_t ld, int shift_i, int scale_i,
                   int per_token, float *y) {
    tsk_tensor tx = act((float *) x, H, S), ty = act(y, H, S);
    orc_norm(&tx, 1e-5f, &ty);
    for (int64_t s = 0; s < S; ++s) {
        const float *mm = mod + (per_token ? s : 0) * ld;
        const float *sh = mm + shift_i * H, *sc = mm + scale_i * H;
        for (int64_t i = 0; i < H; ++i) y[s * H + i] = y[s * H + i] * (sc[i] + 1.0f) + sh[i];
    }
}

/* x += f * gate (ggml_add(x, ggml_mul(f, gate)), mmdit.cpp:230, :234) */
static void gate_add(float *x, const float *f, int64_t H, int64_t S, const float *mod, int64_t ld, int gate_i,
                     int per_token) {
    for (int64_t s = 0; s < S; ++s) {
        const float *g = mod + (per_token ? s : 0) * ld + gate_i * H;
        for (int64_t i = 0; i < H; ++i) x[s * H + i] += f[s * H + i] * g[i];
    }
}

typedef struct {
    float *mod;            /* [nmod H, S or 1] */
    int64_t nmod;
    float *q, *k, *v;      /* [hd, nh, S] after norm / rope */
} pre_out;

/* pre_attn (mmdit.cpp:203-225) */
static void pre_attn(orc_mmdit *m, const char *bp, const float *x, int64_t S, const float *silu_cond, int per_token,
                     float fscale, int is_text, int pre_only, pre_out *o, int act_bf16) {
    const tsk_mmdit_config *c = &m->cfg;
    const int64_t H = c->hidden, nh = c->n_head, hd = c->head_dim;
    char nm[160];
    o->nmod = pre_only ? 2 : 6;
    o->mod = fbuf(o->nmod * H * (per_token ? S : 1));
    snprintf(nm, sizeof(nm), "%s.adaLN_modulation.1", bp);
    lin(m, nm, 1, silu_cond, H, per_token ? S : 1, o->mod, act_bf16);
    float *xn = fbuf(H * S);
    ln_mod(x, H, S, o->mod, o->nmod * H, 0, 1, per_token, xn);
    float *qkv = fbuf(3 * H * S);
    snprintf(nm, sizeof(nm), "%s.attn.qkv", bp);
    lin(m, nm, 1, xn, H, S, qkv, act_bf16);
    /* split_qkv: channel 3 * (h hd + d) + j (mmdit.cpp:67-76) */
    o->q = fbuf(H * S); o->k = fbuf(H * S); o->v = fbuf(H * S);
    for (int64_t s = 0; s < S; ++s)
        for (int64_t i = 0; i < H; ++i) {
            o->q[s * H + i] = qkv[s * 3 * H + 3 * i + 0];
            o->k[s * H + i] = qkv[s * 3 * H + 3 * i + 1];
            o->v[s * H + i] = qkv[s * 3 * H + 3 * i + 2];
        }
    free(qkv); free(xn);
    int32_t *pos = (int32_t *) malloc(sizeof(int32_t) * (size_t) S);
    for (int64_t i = 0; i < S; ++i) pos[i] = (int32_t) i;
    float *qk[2] = { o->q, o->k };
    const char *nn[2] = { "q_norm", "k_norm" };
    for (int j = 0; j < 2; ++j) {
        snprintf(nm, sizeof(nm), "%s.attn.%s.weight", bp, nn[j]);
        tsk_tensor t = { TSK_TYPE_F32, {hd, nh, S, 1}, {4, (size_t) (4 * hd), (size_t) (4 * H), (size_t) (4 * H * S)}, qk[j] };
        orc_rms_norm_mul(&t, find_w(m, nm)->data, 1e-6f, &t);
        if (!is_text) orc_rope_ext(&t, pos, (int) hd, c->rope_theta, fscale, &t);
    }
    free(pos);
}

static void free_pre(pre_out *o) { free(o->mod); free(o->q); free(o->k); free(o->v); }

/* attention() over the concatenation of ns streams (mmdit.cpp:85-95,
 * :251-260): K / V cast to F16 when kv_f16; out[s] = [H, S_s] */
static void joint_attention(orc_mmdit *m, int ns, const int64_t *S, pre_out **st, float **out, int kv_f16) {
    const tsk_mmdit_config *c = &m->cfg;
    const int64_t H = c->hidden, nh = c->n_head, hd = c->head_dim;
    int64_t N = 0;
    for (int s = 0; s < ns; ++s) N += S[s];
    float *Q = fbuf(N * H), *K = fbuf(N * H), *V = fbuf(N * H), *O = fbuf(N * H);
    uint16_t *K16 = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) (N * H));
    uint16_t *V16 = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) (N * H));
    int64_t off = 0;
    for (int s = 0; s < ns; ++s) {
        /* concat along tokens, permute to [hd, N, nh] (mmdit.cpp:88-90) */
        for (int64_t n = 0; n < S[s]; ++n)
            for (int64_t h = 0; h < nh; ++h)
                for (int64_t e = 0; e < hd; ++e) {
                    const int64_t src = n * H + h * hd + e, dst = (h * N + off + n) * hd + e;
                    Q[dst] = st[s]->q[src]; K[dst] = st[s]->k[src]; V[dst] = st[s]->v[src];
                }
        off += S[s];
    }
    tsk_tensor tq = { TSK_TYPE_F32, {hd, N, nh, 1}, {4, (size_t) (4 * hd), (size_t) (4 * hd * N), (size_t) (4 * hd * N * nh)}, Q };
    tsk_tensor tk = tq, tv = tq;
    tk.data = K; tv.data = V;
    if (kv_f16) {
        orc_fp32_to_fp16_row(K, K16, N * H);
        orc_fp32_to_fp16_row(V, V16, N * H);
        tk.type = TSK_TYPE_F16;
        tk.nb[0] = 2; tk.nb[1] = (size_t) (2 * hd); tk.nb[2] = (size_t) (2 * hd * N); tk.nb[3] = (size_t) (2 * hd * N * nh);
        tk.data = K16;
        tv = tk; tv.data = V16;
    }
    tsk_tensor to = { TSK_TYPE_F32, {hd, nh, N, 1}, {4, (size_t) (4 * hd), (size_t) (4 * H), (size_t) (4 * H * N)}, O };
    orc_flash_attn_ext(&tq, &tk, &tv, NULL, 1.0f / sqrtf((float) hd), 0.0f, 0.0f, 0, &to);
    off = 0;
    for (int s = 0; s < ns; ++s) {
        memcpy(out[s], O + off * H, sizeof(float) * (size_t) (S[s] * H));
        off += S[s];
    }
    free(Q); free(K); free(V); free(O); free(K16); free(V16);
}

/* post_attn (mmdit.cpp:226-235) */
static void post_attn(orc_mmdit *m, const char *bp, float *x, int64_t S, const float *ao, const pre_out *st,
                      int per_token, int is_text, int act_bf16) {
    const int64_t H = m->cfg.hidden, ld = 6 * H;
    char nm[160];
    float *l1 = fbuf(H * S), *f = fbuf(H * S);
    snprintf(nm, sizeof(nm), "%s.linear1", bp);
    if (is_text) lin(m, nm, 1, ao, H, S, l1, act_bf16);
    else conv_cl(m, nm, 1, ao, H, S, 1, l1, act_bf16);
    gate_add(x, l1, H, S, st->mod, ld, 2, per_token);
    ln_mod(x, H, S, st->mod, ld, 3, 4, per_token, l1);
    snprintf(nm, sizeof(nm), "%s.ffn", bp);
    swiglu_mlp(m, nm, !is_text, l1, H, S, f, act_bf16);
    gate_add(x, f, H, S, st->mod, ld, 5, per_token);
    free(l1); free(f);
}

/* ts_dit::forward for one batch row (mmdit.cpp:119-342). latent ne = [T, L];
 * clip_f [clip_dim, clip_S]; sync_f [sync_dim, sync_S]; text_f [clip_dim,
 * text_seq]; t5 [t5_dim, text_seq]; global_text [clip_dim]; flow [L, T]. */
static int forward1(orc_mmdit *m, int64_t T, const float *latent, float t, int64_t clip_S, const float *clip_f,
                    int64_t sync_S, const float *sync_f, const float *text_f, const float *t5, const float *gtext,
                    float *flow, int act_bf16, int kv_f16) {
    const tsk_mmdit_config *c = &m->cfg;
    const int64_t H = c->hidden, L = c->latent_dim, X = 2 * (int64_t) c->text_seq;
    const int nj = c->depth - c->fused_depth;
    /* audio_input_proj (:150-155) */
    int64_t smax = T;
    if (clip_S > smax) smax = clip_S;
    if (sync_S > smax) smax = sync_S;
    if (X > smax) smax = X;
    float *xl = fbuf(L * T), *tmp = fbuf(H * smax);
    for (int64_t ch = 0; ch < L; ++ch)
        for (int64_t i = 0; i < T; ++i) xl[i * L + ch] = latent[ch * T + i];
    float *lat = fbuf(H * T);
    conv_cl(m, "audio_input_proj.0", 1, xl, L, T, 1, tmp, act_bf16);
    silu_n(tmp, H * T);
    swiglu_mlp(m, "audio_input_proj.2", 1, tmp, H, T, lat, act_bf16);
    stage_add(m, "x_in", lat, H * T);
    /* t-embedding on the host (:305-314) and t_embed MLP (:157-161) */
    float *temb = fbuf(H), *te0 = fbuf(H), *te = fbuf(H);
    const float fscale_t = 10000.0f / c->t_max_period;
    for (int64_t kk = 0; kk < H / 2; ++kk) {
        const float fr = fscale_t * powf(10000.0f, -2.0f * (float) kk / (float) H);
        temb[kk] = cosf(t * fr);
        temb[H / 2 + kk] = sinf(t * fr);
    }
    lin(m, "t_embed.mlp.0", 1, temb, H, 1, te0, act_bf16);
    silu_n(te0, H);
    lin(m, "t_embed.mlp.2", 1, te0, H, 1, te, act_bf16);
    stage_add(m, "t_emb", te, H);
    /* clip (:163-167) */
    float *clip = fbuf(H * clip_S);
    lin(m, "clip_input_proj.0", 1, clip_f, c->clip_dim, clip_S, tmp, act_bf16);
    silu_n(tmp, H * clip_S);
    swiglu_mlp(m, "clip_input_proj.2", 1, tmp, H, clip_S, clip, act_bf16);
    stage_add(m, "clip_pp", clip, H * clip_S);
    /* sync (:168-178): + pos_emb per 8-frame segment, conv k7, convmlp */
    float *sx = fbuf(c->sync_dim * sync_S), *sync = fbuf(H * sync_S);
    const float *pe = find_w(m, "sync_pos_emb")->data;
    for (int64_t s = 0; s < sync_S; ++s)
        for (int64_t ch = 0; ch < c->sync_dim; ++ch)
            sx[s * c->sync_dim + ch] = sync_f[s * c->sync_dim + ch] + pe[(s % 8) * c->sync_dim + ch];
    conv_cl(m, "sync_input_proj.0", 1, sx, c->sync_dim, sync_S, 3, tmp, act_bf16);
    silu_n(tmp, H * sync_S);
    swiglu_mlp(m, "sync_input_proj.2", 1, tmp, H, sync_S, sync, act_bf16);
    /* text (:179-183): pad text_f to t5_dim, concat t5 along the sequence */
    float *tc = fbuf(c->t5_dim * X), *text = fbuf(H * X);
    for (int64_t s = 0; s < c->text_seq; ++s) {
        memcpy(tc + s * c->t5_dim, text_f + s * c->clip_dim, sizeof(float) * (size_t) c->clip_dim);
        memcpy(tc + (c->text_seq + s) * c->t5_dim, t5 + s * c->t5_dim, sizeof(float) * (size_t) c->t5_dim);
    }
    lin(m, "text_input_proj.0", 1, tc, c->t5_dim, X, tmp, act_bf16);
    silu_n(tmp, H * X);
    swiglu_mlp(m, "text_input_proj.2", 0, tmp, H, X, text, act_bf16);
    stage_add(m, "text_pp", text, H * X);
    /* conditioning vectors (:184-196) */
    float *tfc = fbuf(H), *cmean = fbuf(H), *cfc = fbuf(H), *gsum = fbuf(H), *gc = fbuf(H);
    lin(m, "text_cond_proj", 1, gtext, c->clip_dim, 1, tfc, act_bf16);
    for (int64_t i = 0; i < H; ++i) {      /* ggml_mean: double sum, fp32 / n */
        double s = 0.0;
        for (int64_t r = 0; r < clip_S; ++r) s += (double) clip[r * H + i];
        cmean[i] = (float) s / (float) clip_S;
    }
    lin(m, "clip_cond_proj", 1, cmean, H, 1, cfc, act_bf16);
    for (int64_t i = 0; i < H; ++i) gsum[i] = cfc[i] + tfc[i];
    swiglu_mlp(m, "global_cond_mlp", 0, gsum, H, 1, gc, act_bf16);
    stage_add(m, "clip_fc", cfc, H);
    stage_add(m, "text_fc", tfc, H);
    stage_add(m, "gcmlp", gc, H);
    for (int64_t i = 0; i < H; ++i) gc[i] = gc[i] + te[i];
    stage_add(m, "global_c", gc, H);
    float *ext = fbuf(H * T);
    for (int64_t i = 0; i < T; ++i) {
        const int64_t idx = (int64_t) floorf(((float) i + 0.5f) * (float) sync_S / (float) T);   /* :319 */
        for (int64_t ch = 0; ch < H; ++ch) ext[i * H + ch] = sync[idx * H + ch] + gc[ch];
    }
    stage_add(m, "extended_c", ext, H * T);
    float *sext = fbuf(H * T), *sgc = fbuf(H);
    for (int64_t i = 0; i < H * T; ++i) sext[i] = orc_silu(ext[i]);
    for (int64_t i = 0; i < H; ++i) sgc[i] = orc_silu(gc[i]);

    /* joint blocks (:238-271) */
    const float clip_fscale = (float) T / (float) clip_S;
    char bp[96];
    for (int i = 0; i < nj; ++i) {
        const int pre_only = i == nj - 1;
        pre_out pl, pc, px;
        snprintf(bp, sizeof(bp), "joint_blocks.%d.latent_block", i);
        pre_attn(m, bp, lat, T, sext, 1, 1.0f, 0, 0, &pl, act_bf16);
        snprintf(bp, sizeof(bp), "joint_blocks.%d.clip_block", i);
        pre_attn(m, bp, clip, clip_S, sgc, 0, clip_fscale, 0, pre_only, &pc, act_bf16);
        snprintf(bp, sizeof(bp), "joint_blocks.%d.text_block", i);
        pre_attn(m, bp, text, X, sgc, 0, 1.0f, 1, pre_only, &px, act_bf16);
        float *ol = fbuf(H * T), *oc = fbuf(H * clip_S), *ox = fbuf(H * X);
        const int64_t S3[3] = { T, clip_S, X };
        pre_out *s3[3] = { &pl, &pc, &px };
        float *o3[3] = { ol, oc, ox };
        joint_attention(m, 3, S3, s3, o3, kv_f16);
        snprintf(bp, sizeof(bp), "joint_blocks.%d.latent_block", i);
        post_attn(m, bp, lat, T, ol, &pl, 1, 0, act_bf16);
        if (!pre_only) {
            snprintf(bp, sizeof(bp), "joint_blocks.%d.clip_block", i);
            post_attn(m, bp, clip, clip_S, oc, &pc, 0, 0, act_bf16);
            snprintf(bp, sizeof(bp), "joint_blocks.%d.text_block", i);
            post_attn(m, bp, text, X, ox, &px, 0, 1, act_bf16);
        }
        free(ol); free(oc); free(ox);
        free_pre(&pl); free_pre(&pc); free_pre(&px);
        if (i == 0) {
            stage_add(m, "jb0_lat", lat, H * T);
            stage_add(m, "jb0_clip", clip, H * clip_S);
            stage_add(m, "jb0_text", text, H * X);
        }
    }
    stage_add(m, "after_joint", lat, H * T);
    /* fused blocks (:274-281) */
    for (int i = 0; i < c->fused_depth; ++i) {
        pre_out p1;
        snprintf(bp, sizeof(bp), "fused_blocks.%d", i);
        pre_attn(m, bp, lat, T, sext, 1, 1.0f, 0, 0, &p1, act_bf16);
        float *o1 = fbuf(H * T);
        const int64_t S1[1] = { T };
        pre_out *s1[1] = { &p1 };
        float *os[1] = { o1 };
        joint_attention(m, 1, S1, s1, os, kv_f16);
        post_attn(m, bp, lat, T, o1, &p1, 1, 0, act_bf16);
        free(o1);
        free_pre(&p1);
    }
    stage_add(m, "after_fused", lat, H * T);
    /* final layer (:284-289) */
    float *fmod = fbuf(2 * H * T), *fx = fbuf(H * T);
    lin(m, "final_layer.adaLN_modulation.1", 1, sext, H, T, fmod, act_bf16);
    ln_mod(lat, H, T, fmod, 2 * H, 0, 1, 1, fx);
    conv_cl(m, "final_layer.conv", 1, fx, H, T, 3, flow, act_bf16);
    free(xl); free(tmp); free(lat); free(temb); free(te0); free(te); free(clip); free(sx); free(sync); free(tc);
    free(text); free(tfc); free(cmean); free(cfc); free(gsum); free(gc); free(ext); free(sext); free(sgc);
    free(fmod); free(fx);
    return TSK_OK;
}

int orc_mmdit_forward(orc_mmdit *m, int B, int T, const float *latent, const float *t, int clip_S,
                      const float *clip_f, int sync_S, const float *sync_f, const float *text_f, const float *t5,
                      const float *global_text, float *flow, int act_bf16, int kv_f16) {
    const tsk_mmdit_config *c = &m->cfg;
    if (B < 1 || T < 1 || clip_S < 1 || sync_S < 8 || sync_S % 8) return TSK_ERR_SHAPE;
    stage_reset(m);
    for (int b = 0; b < B; ++b) {
        int rc = forward1(m, T, latent + (size_t) b * c->latent_dim * T, t[b], clip_S,
                          clip_f + (size_t) b * clip_S * c->clip_dim, sync_S, sync_f + (size_t) b * sync_S * c->sync_dim,
                          text_f + (size_t) b * c->text_seq * c->clip_dim, t5 + (size_t) b * c->text_seq * c->t5_dim,
                          global_text + (size_t) b * c->clip_dim, flow + (size_t) b * T * c->latent_dim, act_bf16,
                          kv_f16);
        if (rc) return rc;
    }
    return TSK_OK;
}

/* ts_dit::sample (mmdit.cpp:344-376): two B = 1 forwards per step, the
 * unconditional one on the learned empties and a zero global text feature */
int orc_mmdit_sample(orc_mmdit *m, int T, const float *noise, int clip_S, const float *clip_f, int sync_S,
                     const float *sync_f, const float *text_f, const float *t5, const float *global_text, int steps,
                     float cfg_scale, float *out, float *flow0, int act_bf16, int kv_f16) {
    const tsk_mmdit_config *c = &m->cfg;
    const int64_t L = c->latent_dim;
    float *fc = fbuf(L * T), *fu = fbuf(L * T), *zeros = fbuf(c->clip_dim);
    const float *es = find_w(m, "empty_string_feat")->data, *et = find_w(m, "empty_t5_feat")->data;
    memcpy(out, noise, sizeof(float) * (size_t) (L * T));
    for (int s = 0; s < steps; ++s) {
        const float t_curr = 1.0f - (float) s / (float) steps;
        const float t_prev = 1.0f - (float) (s + 1) / (float) steps;
        const float dt = t_prev - t_curr;
        forward1(m, T, out, t_curr, clip_S, clip_f, sync_S, sync_f, text_f, t5, global_text, fc, act_bf16, kv_f16);
        forward1(m, T, out, t_curr, clip_S, clip_f, sync_S, sync_f, es, et, zeros, fu, act_bf16, kv_f16);
        /* fc, fu ne = [L, T]; x ne = [T, L] */
        for (int64_t ch = 0; ch < L; ++ch)
            for (int64_t i = 0; i < T; ++i) {
                const float fcv = fc[i * L + ch], fuv = fu[i * L + ch];
                const float v = fuv + (fcv - fuv) * cfg_scale;
                if (s == 0 && flow0) flow0[ch * T + i] = v;
                out[ch * T + i] += dt * v;
            }
    }
    free(fc); free(fu); free(zeros);
    return TSK_OK;
}
