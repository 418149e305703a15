/*
 * tsk_oracle_t5.c — CPU restatement of the T5 encoder stack of thinksound.cpp
 * (ts_t5::encode, src/t5_encoder.cpp:40-104), composed from the ggml-semantics
 * ops of tsk_oracle.c. TEST INFRASTRUCTURE ONLY (checker).
 *
 * Per layer (t5_encoder.cpp:56-84):
 *   h = rms_norm(x, eps) * attn_norm                      (:10-12, :59)
 *   q, k, v = mul_mat(W, h)   (Q8_0 weights: h quantized to Q8_0)   (:60-62)
 *   s = mul_mat(k, q) + bias + pad; p = soft_max(s); o = mul_mat(v^T, p)
 *       (no logit scale; bias = rel_bias[bucket(k - q)][head])      (:49-54, :68-75)
 *   x += mul_mat(W_o, o)                                             (:76-78)
 *   h = rms_norm(x) * ffn_norm; x += wo( gelu(wi_0 h) * wi_1 h )     (:80-84)
 * and out_norm after the last layer (:86). The two ggml_add nodes of the
 * scores (bias, then pad) are one addend here: pad is 0 or -inf, so
 * (s + b) + pad == s + (b + pad) for every value.
 */
#include "tsk_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* t5_encoder.cpp:14-26, bidirectional: half the buckets per sign; exact
 * buckets below max_exact, log-spaced up to max_dist, clamped */
int orc_t5_bucket(int rel, int num_buckets, int max_dist) {
    int ret = 0;
    num_buckets /= 2;
    if (rel > 0) ret += num_buckets;
    const int n = rel < 0 ? -rel : rel;
    const int max_exact = num_buckets / 2;
    if (n < max_exact) {
        ret += n;
    } else {
        int v = max_exact + (int) (log((double) n / max_exact) / log((double) max_dist / max_exact) *
                                   (num_buckets - max_exact));
        ret += v < num_buckets - 1 ? v : num_buckets - 1;
    }
    return ret;
}

typedef struct {
    const float *q, *k, *v, *mask;
    int64_t ld;
    int n, H, D;
    float *out;
} attn_ctx;

/* one (head, query) row per item: scores in f32 (f32 dot), ggml-cpu soft_max,
 * then the P.V row */
static void t5_attn_rows(void *p, int64_t lo, int64_t hi) {
    attn_ctx *c = (attn_ctx *) p;
    const int n = c->n, D = c->D;
    float *s = (float *) malloc(sizeof(float) * (size_t) n);
    for (int64_t it = lo; it < hi; ++it) {
        const int h = (int) (it / n), qi = (int) (it % n);
        const float *qr = c->q + (int64_t) qi * c->ld + (int64_t) h * D;
        const float *mr = c->mask + ((int64_t) h * n + qi) * n;
        float mx = -INFINITY;
        for (int kk = 0; kk < n; ++kk) {
            const float *kr = c->k + (int64_t) kk * c->ld + (int64_t) h * D;
            float d = 0.0f;
            for (int e = 0; e < D; ++e) d += kr[e] * qr[e];
            s[kk] = d + mr[kk];
            if (s[kk] > mx) mx = s[kk];
        }
        double sum = 0.0;
        for (int kk = 0; kk < n; ++kk) {
            const float e = mx == -INFINITY ? 0.0f : expf(s[kk] - mx);
            s[kk] = e;
            sum += (double) e;
        }
        const float inv = sum > 0.0 ? (float) (1.0 / sum) : 0.0f;
        for (int kk = 0; kk < n; ++kk) s[kk] *= inv;
        float *orow = c->out + ((int64_t) qi * c->H + h) * D;
        for (int e = 0; e < D; ++e) {
            float a = 0.0f;
            for (int kk = 0; kk < n; ++kk) a += c->v[(int64_t) kk * c->ld + (int64_t) h * D + e] * s[kk];
            orow[e] = a;
        }
    }
    free(s);
}

int orc_t5_attention(const float *q, const float *k, const float *v, int64_t ld, const float *mask, int n, int H,
                     int D, float *out) {
    if (!q || !k || !v || !mask || !out || n < 1 || H < 1 || D < 1) return TSK_ERR_INVALID_ARG;
    attn_ctx c = {q, k, v, mask, ld, n, H, D, out};
    orc_parallel((int64_t) H * n, t5_attn_rows, &c);
    return TSK_OK;
}

/* ------------------------------------------------------------------------ */

typedef struct {
    char name[64];
    int64_t ne[2];
    int type;          /* TSK_TYPE_Q8_0 or TSK_TYPE_F32 */
    void *data;
    size_t nbytes;
} t5w;

struct orc_t5 {
    tsk_t5_config cfg;
    int nw;
    t5w *w;
};

static size_t t5w_bytes(int type, int64_t ne0, int64_t ne1) {
    return type == TSK_TYPE_Q8_0 ? (size_t) (ne0 / 32) * 34 * (size_t) ne1 : (size_t) (ne0 * ne1) * 4;
}

orc_t5 *orc_t5_create(const tsk_t5_config *cfg) {
    orc_t5 *t = (orc_t5 *) calloc(1, sizeof(orc_t5));
    t->cfg = *cfg;
    const int L = cfg->n_layers, d = cfg->d_model, inner = cfg->n_heads * cfg->d_kv, ff = cfg->d_ff;
    t->w = (t5w *) calloc((size_t) (2 + 9 * L), sizeof(t5w));
    const int mt = cfg->weight_type == TSK_TYPE_Q8_0 ? TSK_TYPE_Q8_0 : TSK_TYPE_F32;
#define ADD(nm, a, b, ty)                                                     \
    do {                                                                      \
        t5w *w = &t->w[t->nw++];                                              \
        snprintf(w->name, sizeof(w->name), "%s", nm);                         \
        w->ne[0] = (a); w->ne[1] = (b); w->type = (ty);                       \
        w->nbytes = t5w_bytes(ty, a, b);                                      \
        w->data = calloc(1, w->nbytes);                                       \
    } while (0)
    ADD("rel_bias", cfg->n_heads, cfg->rel_buckets, TSK_TYPE_F32);
    char nm[64];
    for (int i = 0; i < L; ++i) {
        snprintf(nm, sizeof(nm), "blk.%d.attn_norm", i); ADD(nm, d, 1, TSK_TYPE_F32);
        snprintf(nm, sizeof(nm), "blk.%d.q", i); ADD(nm, d, inner, mt);
        snprintf(nm, sizeof(nm), "blk.%d.k", i); ADD(nm, d, inner, mt);
        snprintf(nm, sizeof(nm), "blk.%d.v", i); ADD(nm, d, inner, mt);
        snprintf(nm, sizeof(nm), "blk.%d.o", i); ADD(nm, inner, d, mt);
        snprintf(nm, sizeof(nm), "blk.%d.ffn_norm", i); ADD(nm, d, 1, TSK_TYPE_F32);
        snprintf(nm, sizeof(nm), "blk.%d.wi_0", i); ADD(nm, d, ff, mt);
        snprintf(nm, sizeof(nm), "blk.%d.wi_1", i); ADD(nm, d, ff, mt);
        snprintf(nm, sizeof(nm), "blk.%d.wo", i); ADD(nm, ff, d, mt);
    }
    ADD("out_norm", d, 1, TSK_TYPE_F32);
#undef ADD
    return t;
}

void orc_t5_destroy(orc_t5 *t) {
    if (!t) return;
    for (int i = 0; i < t->nw; ++i) free(t->w[i].data);
    free(t->w);
    free(t);
}

int orc_t5_n_tensors(const orc_t5 *t) { return t ? t->nw : 0; }

int orc_t5_tensor_info(const orc_t5 *t, int i, const char **name, int64_t *ne0, int64_t *ne1, int *type) {
    if (!t || i < 0 || i >= t->nw) return TSK_ERR_INVALID_ARG;
    *name = t->w[i].name; *ne0 = t->w[i].ne[0]; *ne1 = t->w[i].ne[1]; *type = t->w[i].type;
    return TSK_OK;
}

static t5w *find(orc_t5 *t, const char *name) {
    for (int i = 0; i < t->nw; ++i)
        if (!strcmp(t->w[i].name, name)) return &t->w[i];
    return NULL;
}

int orc_t5_set_tensor(orc_t5 *t, const char *name, const void *data, size_t nbytes) {
    t5w *w = find(t, name);
    if (!w || !data) return TSK_ERR_INVALID_ARG;
    if (nbytes != w->nbytes) return TSK_ERR_SHAPE;
    memcpy(w->data, data, nbytes);
    return TSK_OK;
}

/* dst [N][M] = mul_mat(W [K][M], x [N][K]) with ggml's conversion of x */
static int mm(const t5w *w, const float *x, int N, float *y) {
    tsk_tensor a, b, o;
    memset(&a, 0, sizeof(a)); memset(&b, 0, sizeof(b)); memset(&o, 0, sizeof(o));
    const int64_t K = w->ne[0], M = w->ne[1];
    a.type = w->type; a.ne[0] = K; a.ne[1] = M; a.ne[2] = a.ne[3] = 1;
    a.nb[0] = w->type == TSK_TYPE_Q8_0 ? 34 : 4;
    a.nb[1] = w->type == TSK_TYPE_Q8_0 ? (size_t) (K / 32) * 34 : (size_t) K * 4;
    a.nb[2] = a.nb[3] = a.nb[1] * M; a.data = w->data;
    b.type = TSK_TYPE_F32; b.ne[0] = K; b.ne[1] = N; b.ne[2] = b.ne[3] = 1;
    b.nb[0] = 4; b.nb[1] = (size_t) K * 4; b.nb[2] = b.nb[3] = b.nb[1] * N; b.data = (void *) x;
    o.type = TSK_TYPE_F32; o.ne[0] = M; o.ne[1] = N; o.ne[2] = o.ne[3] = 1;
    o.nb[0] = 4; o.nb[1] = (size_t) M * 4; o.nb[2] = o.nb[3] = o.nb[1] * N; o.data = y;
    return orc_mul_mat(&a, &b, NULL, &o);
}

static int rmsnorm(const float *x, const t5w *w, float eps, int N, int d, float *y) {
    tsk_tensor a, o;
    memset(&a, 0, sizeof(a)); memset(&o, 0, sizeof(o));
    a.type = TSK_TYPE_F32; a.ne[0] = d; a.ne[1] = N; a.ne[2] = a.ne[3] = 1;
    a.nb[0] = 4; a.nb[1] = (size_t) d * 4; a.nb[2] = a.nb[3] = a.nb[1] * N; a.data = (void *) x;
    o = a; o.data = y;
    return orc_rms_norm_mul(&a, (const float *) w->data, eps, &o);
}

int orc_t5_encode(orc_t5 *t, int n, const float *x_in, const int32_t *ids, float *out) {
    if (!t) return TSK_ERR_INVALID_ARG;
    return orc_t5_encode_range(t, n, x_in, ids, 0, t->cfg.n_layers, 1, out);
}

int orc_t5_encode_range(orc_t5 *t, int n, const float *x_in, const int32_t *ids, int layer_begin, int layer_end,
                        int final_norm, float *out) {
    if (!t || !x_in || !ids || !out || n < 1) return TSK_ERR_INVALID_ARG;
    if (layer_begin < 0 || layer_end > t->cfg.n_layers || layer_begin > layer_end) return TSK_ERR_INVALID_ARG;
    const tsk_t5_config *c = &t->cfg;
    const int d = c->d_model, H = c->n_heads, D = c->d_kv, inner = H * D, ff = c->d_ff;
    int rc = TSK_OK;
    float *x = (float *) malloc(sizeof(float) * (size_t) n * d);
    float *h = (float *) malloc(sizeof(float) * (size_t) n * (d > ff ? d : ff));
    float *qkv = (float *) malloc(sizeof(float) * (size_t) n * inner * 3);
    float *o = (float *) malloc(sizeof(float) * (size_t) n * inner);
    float *g0 = (float *) malloc(sizeof(float) * (size_t) n * ff);
    float *g1 = (float *) malloc(sizeof(float) * (size_t) n * ff);
    float *y = (float *) malloc(sizeof(float) * (size_t) n * d);
    float *mask = (float *) malloc(sizeof(float) * (size_t) H * n * n);
    memcpy(x, x_in, sizeof(float) * (size_t) n * d);
    /* bias[h][q][k] = rel_bias[bucket(k - q)][h] (+ -inf for padded keys) */
    const float *rb = (const float *) find(t, "rel_bias")->data;    /* ne [H, buckets] */
    for (int qi = 0; qi < n; ++qi)
        for (int kk = 0; kk < n; ++kk) {
            const int bk = orc_t5_bucket(kk - qi, c->rel_buckets, c->rel_max_dist);
            for (int hh = 0; hh < H; ++hh)
                mask[((int64_t) hh * n + qi) * n + kk] = rb[bk * H + hh] + (ids[kk] != 0 ? 0.0f : -INFINITY);
        }
    char nm[64];
#define W(fmt) (snprintf(nm, sizeof(nm), fmt, i), find(t, nm))
    for (int i = layer_begin; i < layer_end && !rc; ++i) {
        rc = rmsnorm(x, W("blk.%d.attn_norm"), c->eps, n, d, h);
        float *q = qkv, *k = qkv + (size_t) n * inner, *v = qkv + (size_t) 2 * n * inner;
        if (!rc) rc = mm(W("blk.%d.q"), h, n, q);
        if (!rc) rc = mm(W("blk.%d.k"), h, n, k);
        if (!rc) rc = mm(W("blk.%d.v"), h, n, v);
        if (!rc) rc = orc_t5_attention(q, k, v, inner, mask, n, H, D, o);
        if (!rc) rc = mm(W("blk.%d.o"), o, n, y);
        for (int64_t j = 0; j < (int64_t) n * d; ++j) x[j] += y[j];
        if (!rc) rc = rmsnorm(x, W("blk.%d.ffn_norm"), c->eps, n, d, h);
        if (!rc) rc = mm(W("blk.%d.wi_0"), h, n, g0);
        if (!rc) rc = mm(W("blk.%d.wi_1"), h, n, g1);
        for (int64_t j = 0; j < (int64_t) n * ff; ++j) g0[j] = orc_gelu_tanh(g0[j]) * g1[j];
        if (!rc) rc = mm(W("blk.%d.wo"), g0, n, y);
        for (int64_t j = 0; j < (int64_t) n * d; ++j) x[j] += y[j];
    }
#undef W
    if (!rc && final_norm) rc = rmsnorm(x, find(t, "out_norm"), c->eps, n, d, out);
    else if (!rc) memcpy(out, x, sizeof(float) * (size_t) n * d);
    free(x); free(h); free(qkv); free(o); free(g0); free(g1); free(y); free(mask);
    return rc;
}
