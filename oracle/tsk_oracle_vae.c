/*
 * tsk_oracle_vae.c — CPU restatement of ts_vae::decode (src/vae_decoder.cpp:
 * 62-124), the Oobleck VAE decoder, node by node with the ggml-semantics
 * convolution of tsk_oracle_conv.c (im2col + F32 mul_mat). TEST
 * INFRASTRUCTURE ONLY: the checker of tsk_vae_decode.
 *
 *   x = conv1d(layers.0, latent, k7 p3)                                 :73
 *   5 blocks: x = snake(x); x = conv_t1d(layers.1, x, s)                :80-83
 *             3 residual units: x = x + conv1d_k1(snake(conv1d_k7_d(snake(x))))   :84-91
 *   audio = conv1d(layers.7, snake(x), k7 p3, no bias)                  :95-96
 *   snake(x) = x + sin(x exp(alpha))^2 exp(-beta)                       :14-24
 *   conv_t1d: zero-stuff the input by s (s - 1 zeros after every frame,
 *   the trailing ones dropped), then conv1d with padding K - 1 - s / 2    :36-58
 *
 * Activations are kept with channels fastest ([T][C]); every convolution is
 * orc_conv1d (F32 weights: fp32 products summed in double).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tsk_oracle.h"

typedef struct { char name[96]; int64_t ne[3]; float *data; } vw;

struct orc_vae {
    tsk_vae_config cfg;
    int nw, capw;
    vw *w;
};

static void addv(orc_vae *v, const char *name, int64_t a, int64_t b, int64_t c) {
    if (v->nw == v->capw) {
        v->capw = v->capw ? 2 * v->capw : 128;
        v->w = (vw *) realloc(v->w, sizeof(vw) * (size_t) v->capw);
    }
    vw *x = &v->w[v->nw++];
    snprintf(x->name, sizeof(x->name), "%s", name);
    x->ne[0] = a; x->ne[1] = b; x->ne[2] = c;
    x->data = (float *) calloc((size_t) (a * b * c), sizeof(float));
}

/* block n (decoder.layers.n+1): in / out channels and stride (vae_decoder.cpp:76) */
static void dims(const tsk_vae_config *c, int n, int *in, int *out, int *s) {
    const int mult[6] = {1, c->c_mults[0], c->c_mults[1], c->c_mults[2], c->c_mults[3], c->c_mults[4]};
    *in = mult[5 - n] * c->channels;
    *out = mult[4 - n] * c->channels;
    *s = c->strides[4 - n];
}

orc_vae *orc_vae_create(const tsk_vae_config *cfg) {
    orc_vae *v = (orc_vae *) calloc(1, sizeof(orc_vae));
    v->cfg = *cfg;
    char nm[96];
    int ci, co, st;
    dims(cfg, 0, &ci, &co, &st);
    addv(v, "decoder.layers.0.weight", 7, cfg->latent_dim, ci);
    addv(v, "decoder.layers.0.bias", ci, 1, 1);
    for (int n = 0; n < 5; ++n) {
        dims(cfg, n, &ci, &co, &st);
        snprintf(nm, sizeof(nm), "decoder.layers.%d.layers.0.alpha", n + 1); addv(v, nm, ci, 1, 1);
        snprintf(nm, sizeof(nm), "decoder.layers.%d.layers.0.beta", n + 1);  addv(v, nm, ci, 1, 1);
        snprintf(nm, sizeof(nm), "decoder.layers.%d.layers.1.weight", n + 1); addv(v, nm, 2 * st, ci, co);
        snprintf(nm, sizeof(nm), "decoder.layers.%d.layers.1.bias", n + 1);   addv(v, nm, co, 1, 1);
        for (int r = 0; r < 3; ++r) {
            const char *sfx[8] = {"layers.0.alpha", "layers.0.beta", "layers.1.weight", "layers.1.bias",
                                  "layers.2.alpha", "layers.2.beta", "layers.3.weight", "layers.3.bias"};
            for (int j = 0; j < 8; ++j) {
                snprintf(nm, sizeof(nm), "decoder.layers.%d.layers.%d.%s", n + 1, r + 2, sfx[j]);
                if (j == 2) addv(v, nm, 7, co, co);
                else if (j == 6) addv(v, nm, 1, co, co);
                else addv(v, nm, co, 1, 1);
            }
        }
    }
    dims(cfg, 4, &ci, &co, &st);
    addv(v, "decoder.layers.6.alpha", co, 1, 1);
    addv(v, "decoder.layers.6.beta", co, 1, 1);
    addv(v, "decoder.layers.7.weight", 7, co, cfg->out_channels);
    return v;
}

void orc_vae_destroy(orc_vae *v) {
    if (!v) return;
    for (int i = 0; i < v->nw; ++i) free(v->w[i].data);
    free(v->w);
    free(v);
}

int orc_vae_n_tensors(const orc_vae *v) { return v->nw; }

int orc_vae_tensor_info(const orc_vae *v, int i, const char **name, int64_t ne[3]) {
    if (i < 0 || i >= v->nw) return TSK_ERR_INVALID_ARG;
    *name = v->w[i].name;
    for (int j = 0; j < 3; ++j) ne[j] = v->w[i].ne[j];
    return TSK_OK;
}

static vw *find(orc_vae *v, const char *name) {
    for (int i = 0; i < v->nw; ++i) if (!strcmp(v->w[i].name, name)) return &v->w[i];
    fprintf(stderr, "orc_vae: missing tensor %s\n", name);
    abort();
}

int orc_vae_set_tensor(orc_vae *v, const char *name, const float *src, int64_t n) {
    for (int i = 0; i < v->nw; ++i) {
        vw *x = &v->w[i];
        if (strcmp(x->name, name)) continue;
        if (n != x->ne[0] * x->ne[1] * x->ne[2]) return TSK_ERR_SHAPE;
        memcpy(x->data, src, sizeof(float) * (size_t) n);
        return TSK_OK;
    }
    return TSK_ERR_INVALID_ARG;
}

/* snake (vae_decoder.cpp:14-24) in place on rows [T][C] */
static void snake(orc_vae *v, const char *p, float *x, int64_t T, int64_t C) {
    char nm[128];
    snprintf(nm, sizeof(nm), "%s.alpha", p);
    const float *a = find(v, nm)->data;
    snprintf(nm, sizeof(nm), "%s.beta", p);
    const float *b = find(v, nm)->data;
    for (int64_t c = 0; c < C; ++c) {
        const float ea = expf(a[c]), eb = expf(-b[c]);
        for (int64_t t = 0; t < T; ++t) {
            const float s = sinf(x[t * C + c] * ea);
            x[t * C + c] = x[t * C + c] + (s * s) * eb;
        }
    }
}

/* conv1d (vae_decoder.cpp:26-35): x rows [T_in][IC] -> y rows [T_out][OC] */
static int64_t conv(orc_vae *v, const char *p, int bias, const float *x, int64_t IC, int64_t T_in, int pad, int dil,
                    float *y) {
    char nm[128];
    snprintf(nm, sizeof(nm), "%s.weight", p);
    vw *w = find(v, nm);
    const int64_t K = w->ne[0], OC = w->ne[2];
    const int64_t T_out = T_in + 2 * pad - dil * (K - 1);
    tsk_tensor tw = {TSK_TYPE_F32, {K, IC, OC, 1}, {4, (size_t) (4 * K), (size_t) (4 * K * IC), (size_t) (4 * K * IC * OC)}, w->data};
    tsk_tensor tx = {TSK_TYPE_F32, {IC, T_in, 1, 1}, {4, (size_t) (4 * IC), (size_t) (4 * IC * T_in), (size_t) (4 * IC * T_in)}, (void *) x};
    tsk_tensor ty = {TSK_TYPE_F32, {OC, T_out, 1, 1}, {4, (size_t) (4 * OC), (size_t) (4 * OC * T_out), (size_t) (4 * OC * T_out)}, y};
    tsk_tensor tb;
    if (bias) {
        snprintf(nm, sizeof(nm), "%s.bias", p);
        tsk_tensor t = {TSK_TYPE_F32, {OC, 1, 1, 1}, {4, (size_t) (4 * OC), (size_t) (4 * OC), (size_t) (4 * OC)}, find(v, nm)->data};
        tb = t;
    }
    orc_conv1d(&tw, bias ? &tb : NULL, &tx, 1, pad, dil, &ty);
    return T_out;
}

/* conv_t1d (vae_decoder.cpp:36-58): zero-stuff by s, drop the trailing zeros,
 * conv1d with the converter's kernel (K = 2 s) and padding K - 1 - s / 2 */
static int64_t conv_t(orc_vae *v, const char *p, const float *x, int64_t IC, int64_t T_in, int s, float *y) {
    const int64_t L = (T_in - 1) * s + 1;
    float *u = (float *) calloc((size_t) (L * IC), sizeof(float));
    for (int64_t t = 0; t < T_in; ++t) memcpy(u + t * s * IC, x + t * IC, sizeof(float) * (size_t) IC);
    const int K = 2 * s;
    const int64_t T_out = conv(v, p, 1, u, IC, L, K - 1 - s / 2, 1, y);
    free(u);
    return T_out;
}

int orc_vae_decode(orc_vae *v, int T, const float *latent, float *audio) {
    const tsk_vae_config *c = &v->cfg;
    int64_t hop = 1;
    for (int i = 0; i < 5; ++i) hop *= c->strides[i];
    int ci, co, st;
    dims(c, 0, &ci, &co, &st);
    /* the largest activation: max over stages of frames x channels */
    int64_t cap = (int64_t) T * ci, frames = T;
    for (int n = 0; n < 5; ++n) {
        dims(c, n, &ci, &co, &st);
        frames *= st;
        if (frames * co > cap) cap = frames * co;
    }
    if (frames * c->out_channels > cap) cap = frames * c->out_channels;
    float *x = (float *) malloc(sizeof(float) * (size_t) cap);
    float *h = (float *) malloc(sizeof(float) * (size_t) cap);
    float *g = (float *) malloc(sizeof(float) * (size_t) cap);
    float *lat = (float *) malloc(sizeof(float) * (size_t) T * (size_t) c->latent_dim);
    for (int ch = 0; ch < c->latent_dim; ++ch)
        for (int t = 0; t < T; ++t) lat[(int64_t) t * c->latent_dim + ch] = latent[(int64_t) ch * T + t];
    frames = conv(v, "decoder.layers.0", 1, lat, c->latent_dim, T, 3, 1, x);
    int64_t C = 0;
    char bp[64], rp[96];
    const int dil[3] = {1, 3, 9};
    for (int n = 0; n < 5; ++n) {
        dims(c, n, &ci, &co, &st);
        snprintf(bp, sizeof(bp), "decoder.layers.%d", n + 1);
        memcpy(h, x, sizeof(float) * (size_t) (frames * ci));
        snprintf(rp, sizeof(rp), "%s.layers.0", bp);
        snake(v, rp, h, frames, ci);
        snprintf(rp, sizeof(rp), "%s.layers.1", bp);
        frames = conv_t(v, rp, h, ci, frames, st, x);
        C = co;
        for (int r = 0; r < 3; ++r) {
            memcpy(h, x, sizeof(float) * (size_t) (frames * C));
            snprintf(rp, sizeof(rp), "%s.layers.%d.layers.0", bp, r + 2);
            snake(v, rp, h, frames, C);
            snprintf(rp, sizeof(rp), "%s.layers.%d.layers.1", bp, r + 2);
            conv(v, rp, 1, h, C, frames, 3 * dil[r], dil[r], g);
            snprintf(rp, sizeof(rp), "%s.layers.%d.layers.2", bp, r + 2);
            snake(v, rp, g, frames, C);
            snprintf(rp, sizeof(rp), "%s.layers.%d.layers.3", bp, r + 2);
            conv(v, rp, 1, g, C, frames, 0, 1, h);
            for (int64_t i = 0; i < frames * C; ++i) x[i] = x[i] + h[i];
        }
    }
    snake(v, "decoder.layers.6", x, frames, C);
    conv(v, "decoder.layers.7", 0, x, C, frames, 3, 1, g);
    for (int ch = 0; ch < c->out_channels; ++ch)
        for (int64_t t = 0; t < frames; ++t) audio[(int64_t) ch * frames + t] = g[t * c->out_channels + ch];
    free(x); free(h); free(g); free(lat);
    return TSK_OK;
}
