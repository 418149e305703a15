/*
 * tsk_oracle.c — CPU restatement of ggml-cpu semantics for the MM-DiT hot
 * path. TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline);
 * the product library never links it.
 *
 * Upstream algorithm: ggml (github.com/ggml-org/ggml, submodule of the
 * reference, .gitmodules:1-3; the ggml of llama.cpp 911b67a60 per
 * docs/PROGRESS.md:17). Not present in this container: every function below
 * restates ggml's published CPU algorithm and names the reference call site
 * that emits the node. Pinning: tests/test_oracle_*.py check each function
 * against closed forms, brute force and known-answer vectors.
 */
#include "tsk_oracle.h"

#include <math.h>
#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* threads                                                                  */
/* ------------------------------------------------------------------------ */

static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }
int  orc_get_threads(void) { return g_threads; }

typedef struct { orc_range_fn fn; void *ctx; int64_t lo, hi; } orc_job;

static void *orc_job_run(void *p) {
    orc_job *j = (orc_job *) p;
    if (j->lo < j->hi) j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

/* Run fn over [0, n) split in contiguous chunks over g_threads threads. */
void orc_parallel(int64_t n, orc_range_fn fn, void *ctx) {
    int nt = g_threads;
    if (nt > n) nt = (int) (n > 0 ? n : 1);
    if (nt <= 1) { if (n > 0) fn(ctx, 0, n); return; }
    pthread_t th[256];
    orc_job jobs[256];
    int64_t chunk = (n + nt - 1) / nt;
    for (int i = 0; i < nt; ++i) {
        jobs[i].fn = fn; jobs[i].ctx = ctx;
        jobs[i].lo = i * chunk; jobs[i].hi = (i + 1) * chunk < n ? (i + 1) * chunk : n;
    }
    for (int i = 1; i < nt; ++i) pthread_create(&th[i], NULL, orc_job_run, &jobs[i]);
    orc_job_run(&jobs[0]);
    for (int i = 1; i < nt; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* fp16 / bf16                                                              */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float    u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16, round to nearest even, overflow to inf (GGML_FP32_TO_FP16). */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;               /* NaN -> quiet NaN */
    if (ax >= 0x477ff000u) return sign | 0x7c00u;              /* >= 65520 -> inf  */
    if (ax < 0x38800000u) {                                     /* below 2^-14      */
        /* f16 subnormal step is 2^-24: scale exactly, round to integer (RNE). */
        float m = rintf(u2f(ax) * 16777216.0f);
        return sign | (uint16_t) m;                             /* 1024 -> min normal */
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t h = (e << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return sign | (uint16_t) h;
}

float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {                                   /* zero / subnormal: m * 2^-24 */
        float v = (float) m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

/* bfloat16 RNE with quiet-NaN forcing (GGML_FP32_TO_BF16). */
uint16_t orc_fp32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((x >> 16) | 64u);
    return (uint16_t) ((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}
float orc_bf16_to_fp32(uint16_t h) { return u2f((uint32_t) h << 16); }

void orc_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = orc_fp32_to_fp16(x[i]); }
void orc_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = orc_fp16_to_fp32(x[i]); }
void orc_fp32_to_bf16_row(const float *x, uint16_t *y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = orc_fp32_to_bf16(x[i]); }
void orc_bf16_to_fp32_row(const uint16_t *x, float *y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_to_fp32(x[i]); }

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                     */
/* ------------------------------------------------------------------------ */

#define QK8_0 32
typedef struct { uint16_t d; int8_t qs[QK8_0]; } __attribute__((packed)) orc_block_q8_0;
_Static_assert(sizeof(orc_block_q8_0) == 34, "block_q8_0 is 34 bytes");

/* round half away from zero (C roundf; gguf-py np_roundf has the same ties) */
static inline float round_half_away(float x) { return roundf(x); }

/* Q8_0 quantization of n floats (n % 32 == 0). Weights of the reference's
 * q8 GGUF come from gguf-py (convert/quantize_gguf.py:41, mode GGUF_PY);
 * mul_mat activations are quantized by ggml-cpu (mode CPU_SIMD on x86). */
void orc_quantize_q8_0(const float *x, void *blocks, int64_t n, int mode) {
    orc_block_q8_0 *y = (orc_block_q8_0 *) blocks;
    for (int64_t ib = 0; ib < n / QK8_0; ++ib) {
        const float *xb = x + ib * QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; ++j) { float a = fabsf(xb[j]); if (a > amax) amax = a; }
        const float d = amax / 127.0f;
        y[ib].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK8_0; ++j) {
            float q;
            if (mode == ORC_Q8_CPU_SIMD) {
                const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
                q = rintf(xb[j] * id);
            } else if (mode == ORC_Q8_CPU_REF) {
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                q = round_half_away(xb[j] * id);
            } else {
                q = d != 0.0f ? round_half_away(xb[j] / d) : 0.0f;
            }
            y[ib].qs[j] = (int8_t) q;
        }
    }
}

void orc_dequantize_q8_0(const void *blocks, float *y, int64_t n) {
    const orc_block_q8_0 *x = (const orc_block_q8_0 *) blocks;
    for (int64_t ib = 0; ib < n / QK8_0; ++ib) {
        const float d = orc_fp16_to_fp32(x[ib].d);
        for (int j = 0; j < QK8_0; ++j) y[ib * QK8_0 + j] = d * (float) x[ib].qs[j];
    }
}

/* ------------------------------------------------------------------------ */
/* mul_mat  (ggml_mul_mat, emitted by lin() src/mmdit.cpp:13 and            */
/*           conv1d_f32() src/mmdit.cpp:24)                                  */
/* ------------------------------------------------------------------------ */

static inline float tget(const tsk_tensor *t, const char *p) {
    switch (t->type) {
        case TSK_TYPE_F32:  return *(const float *) p;
        case TSK_TYPE_F16:  return orc_fp16_to_fp32(*(const uint16_t *) p);
        case TSK_TYPE_BF16: return orc_bf16_to_fp32(*(const uint16_t *) p);
        default: return 0.0f;
    }
}

typedef struct {
    const tsk_tensor *a, *b, *bias; tsk_tensor *dst;
    int64_t K, M, N;           /* N = all src1 rows (ne1*ne2*ne3) */
    double *bx;                /* src1 rows converted to a's vec_dot precision (exact in fp64) */
    orc_block_q8_0 *bq;        /* src1 rows quantized (Q8_0 weights) */
    float  *arow_buf;          /* per-thread not needed: rows converted on the fly */
} mm_ctx;

static inline const char *b_row(const tsk_tensor *b, int64_t n) {
    int64_t n1 = n % b->ne[1], r = n / b->ne[1];
    int64_t n2 = r % b->ne[2], n3 = r / b->ne[2];
    return (const char *) b->data + n1 * b->nb[1] + n2 * b->nb[2] + n3 * b->nb[3];
}
static inline char *d_row(tsk_tensor *d, int64_t n) {
    int64_t n1 = n % d->ne[1], r = n / d->ne[1];
    int64_t n2 = r % d->ne[2], n3 = r / d->ne[2];
    return (char *) d->data + n1 * d->nb[1] + n2 * d->nb[2] + n3 * d->nb[3];
}

/* Dot products in fp64 with 8 independent lanes: lane j sums the products
 * of k = j, j + 8, ... in k order (each product of two floats is exact in
 * fp64), then s = ((0 + lane0) + lane1) + ... + lane7, then the k % 8 tail
 * in k order. Four weight rows share one pass over an x row (32 independent
 * accumulator chains); every output keeps exactly this summation order. */
typedef double orc_v4d __attribute__((vector_size(32)));

static inline orc_v4d ld4d(const double *p) { orc_v4d v; memcpy(&v, p, sizeof(v)); return v; }

static double lanes_sum(orc_v4d lo, orc_v4d hi) {
    double s = 0.0;
    for (int j = 0; j < 4; ++j) s += lo[j];
    for (int j = 0; j < 4; ++j) s += hi[j];
    return s;
}

/* lane-wise acc + a * b with one rounding: a and b hold float values, so
 * a * b is exact in fp64 and this is the same double as round(a * b) + acc */
static inline orc_v4d mad4d(orc_v4d acc, orc_v4d a, orc_v4d b) {
    __m256d r = _mm256_fmadd_pd((__m256d) a, (__m256d) b, (__m256d) acc);
    return (orc_v4d) r;
}

/* w: 4 rows of K doubles (row stride K), y: K doubles */
static void dot4_f64(const double *w, const double *y, int64_t K, double out[4]) {
    orc_v4d l0 = {0, 0, 0, 0}, h0 = l0, l1 = l0, h1 = l0, l2 = l0, h2 = l0, l3 = l0, h3 = l0;
    int64_t k = 0;
    for (; k + 8 <= K; k += 8) {
        const orc_v4d ylo = ld4d(y + k), yhi = ld4d(y + k + 4);
        l0 = mad4d(l0, ld4d(w + k), ylo);          h0 = mad4d(h0, ld4d(w + k + 4), yhi);
        l1 = mad4d(l1, ld4d(w + K + k), ylo);      h1 = mad4d(h1, ld4d(w + K + k + 4), yhi);
        l2 = mad4d(l2, ld4d(w + 2 * K + k), ylo);  h2 = mad4d(h2, ld4d(w + 2 * K + k + 4), yhi);
        l3 = mad4d(l3, ld4d(w + 3 * K + k), ylo);  h3 = mad4d(h3, ld4d(w + 3 * K + k + 4), yhi);
    }
    out[0] = lanes_sum(l0, h0); out[1] = lanes_sum(l1, h1);
    out[2] = lanes_sum(l2, h2); out[3] = lanes_sum(l3, h3);
    for (; k < K; ++k)
        for (int r = 0; r < 4; ++r) out[r] += w[r * K + k] * y[k];
}

/* weight rows in chunks of 16 (converted to fp64 once), each x row read once
 * per chunk and multiplied with its four groups of four rows */
static void mm_rows_float(void *p, int64_t lo, int64_t hi) {
    mm_ctx *c = (mm_ctx *) p;
    const tsk_tensor *a = c->a;
    const int64_t K = c->K;
    enum { CH = 16 };
    double *wrow = (double *) malloc(sizeof(double) * (size_t) (CH * K));
    for (int64_t m0 = lo; m0 < hi; m0 += CH) {
        const int nm = hi - m0 < CH ? (int) (hi - m0) : CH;
        for (int r = 0; r < CH; ++r) {
            /* rows past hi repeat the last one (computed, never stored) */
            const int64_t m = m0 + (r < nm ? r : nm - 1);
            const char *ar = (const char *) a->data + m * a->nb[1];
            for (int64_t k = 0; k < K; ++k) wrow[r * K + k] = (double) tget(a, ar + k * a->nb[0]);
        }
        for (int64_t n = 0; n < c->N; ++n) {
            float *dr = (float *) d_row(c->dst, n);
            for (int g = 0; g * 4 < nm; ++g) {
                double s[4];
                dot4_f64(wrow + (size_t) g * 4 * K, c->bx + n * K, K, s);
                for (int r = 0; r < 4 && g * 4 + r < nm; ++r) {
                    const int64_t m = m0 + g * 4 + r;
                    float v = (float) s[r];
                    if (c->bias) v += ((const float *) c->bias->data)[m];
                    dr[m] = v;
                }
            }
        }
    }
    free(wrow);
}

/* ggml_vec_dot_q8_0_q8_0: sumf += (float)sumi * (fp32(d_x) * fp32(d_y)) per block */
static void mm_rows_q8(void *p, int64_t lo, int64_t hi) {
    mm_ctx *c = (mm_ctx *) p;
    const int64_t nb = c->K / QK8_0;
    for (int64_t m = lo; m < hi; ++m) {
        const orc_block_q8_0 *wr = (const orc_block_q8_0 *) ((const char *) c->a->data + m * c->a->nb[1]);
        const float bm = c->bias ? ((const float *) c->bias->data)[m] : 0.0f;
        for (int64_t n = 0; n < c->N; ++n) {
            const orc_block_q8_0 *xr = c->bq + n * nb;
            float sumf = 0.0f;
            for (int64_t ib = 0; ib < nb; ++ib) {
                int sumi = 0;
                for (int j = 0; j < QK8_0; ++j) sumi += (int) wr[ib].qs[j] * (int) xr[ib].qs[j];
                sumf += (float) sumi * (orc_fp16_to_fp32(wr[ib].d) * orc_fp16_to_fp32(xr[ib].d));
            }
            float v = sumf;
            if (c->bias) v += bm;
            *(float *) (d_row(c->dst, n) + m * sizeof(float)) = v;
        }
    }
}

int orc_mul_mat(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias, tsk_tensor *dst) {
    if (!a || !b || !dst) return TSK_ERR_INVALID_ARG;
    if (b->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    const int64_t K = a->ne[0], M = a->ne[1];
    if (b->ne[0] != K || dst->ne[0] != M || dst->ne[1] != b->ne[1] ||
        dst->ne[2] != b->ne[2] || dst->ne[3] != b->ne[3]) return TSK_ERR_SHAPE;
    mm_ctx c; memset(&c, 0, sizeof(c));
    c.a = a; c.b = b; c.bias = bias; c.dst = dst; c.K = K; c.M = M;
    c.N = b->ne[1] * b->ne[2] * b->ne[3];
    if (a->type == TSK_TYPE_Q8_0) {
        if (K % QK8_0) return TSK_ERR_SHAPE;
        c.bq = (orc_block_q8_0 *) malloc(sizeof(orc_block_q8_0) * (size_t) (c.N * (K / QK8_0)));
        for (int64_t n = 0; n < c.N; ++n)
            orc_quantize_q8_0((const float *) b_row(b, n), c.bq + n * (K / QK8_0), K, ORC_Q8_CPU_SIMD);
        orc_parallel(M, mm_rows_q8, &c);
        free(c.bq);
        return TSK_OK;
    }
    if (a->type != TSK_TYPE_F32 && a->type != TSK_TYPE_F16 && a->type != TSK_TYPE_BF16) return TSK_ERR_TYPE;
    /* src1 converted to the weight's vec_dot type (BF16: RNE to bf16; F16: to fp16) */
    c.bx = (double *) malloc(sizeof(double) * (size_t) (c.N * K));
    for (int64_t n = 0; n < c.N; ++n) {
        const float *xr = (const float *) b_row(b, n);
        double *o = c.bx + n * K;
        for (int64_t k = 0; k < K; ++k) {
            float x = xr[k];
            if (a->type == TSK_TYPE_BF16) x = orc_bf16_to_fp32(orc_fp32_to_bf16(x));
            else if (a->type == TSK_TYPE_F16) x = orc_fp16_to_fp32(orc_fp32_to_fp16(x));
            o[k] = (double) x;
        }
    }
    orc_parallel(M, mm_rows_float, &c);
    free(c.bx);
    return TSK_OK;
}

/* ------------------------------------------------------------------------ */
/* flash_attn_ext  (ggml_flash_attn_ext, src/mmdit.cpp:91-92; T5 config     */
/*                  drives it with a per-head additive mask)                 */
/* ------------------------------------------------------------------------ */

typedef struct {
    const tsk_tensor *q, *k, *v, *mask; tsk_tensor *dst;
    float scale, max_bias, softcap; int vacc_f16;
    int64_t D, Dv, Nq, Nkv, H, B, Hkv;
    float m0, m1; uint32_t n_head_log2;
} fa_ctx;

/* K and V of one (kv head, batch item) as floats, converted once per slice
 * (the rows of a thread's range mostly share one slice) */
typedef struct {
    int64_t ik2, iq3;
    float *K, *V;
} fa_slice;

static void fa_load_slice(const fa_ctx *c, fa_slice *sl, int64_t ik2, int64_t iq3) {
    if (sl->ik2 == ik2 && sl->iq3 == iq3) return;
    for (int64_t ic = 0; ic < c->Nkv; ++ic) {
        const char *kp = (const char *) c->k->data + ic * c->k->nb[1] + ik2 * c->k->nb[2] + iq3 * c->k->nb[3];
        const char *vp = (const char *) c->v->data + ic * c->v->nb[1] + ik2 * c->v->nb[2] + iq3 * c->v->nb[3];
        for (int64_t d = 0; d < c->D; ++d) sl->K[ic * c->D + d] = tget(c->k, kp + d * c->k->nb[0]);
        for (int64_t d = 0; d < c->Dv; ++d) sl->V[ic * c->Dv + d] = tget(c->v, vp + d * c->v->nb[0]);
    }
    sl->ik2 = ik2;
    sl->iq3 = iq3;
}

static void fa_rows(void *p, int64_t lo, int64_t hi) {
    fa_ctx *c = (fa_ctx *) p;
    const int64_t D = c->D, Dv = c->Dv;
    float *Qc = (float *) malloc(sizeof(float) * D);
    double *acc = (double *) malloc(sizeof(double) * Dv);
    uint16_t *acc16 = (uint16_t *) malloc(sizeof(uint16_t) * Dv);
    fa_slice sl = { -1, -1, (float *) malloc(sizeof(float) * (size_t) (c->Nkv * D)),
                    (float *) malloc(sizeof(float) * (size_t) (c->Nkv * Dv)) };
    double *sdots = (double *) malloc(sizeof(double) * (size_t) c->Nkv);
    float scale = c->scale;
    if (c->softcap != 0.0f) scale /= c->softcap;
    for (int64_t r = lo; r < hi; ++r) {
        const int64_t iq1 = r % c->Nq, iq2 = (r / c->Nq) % c->H, iq3 = r / (c->Nq * c->H);
        const int64_t ik2 = iq2 / (c->H / c->Hkv);
        fa_load_slice(c, &sl, ik2, iq3);
        /* ALiBi slope (ggml): 1 when max_bias == 0 */
        float slope = 1.0f;
        if (c->max_bias > 0.0f) {
            const uint32_t h = (uint32_t) iq2;
            slope = h < c->n_head_log2 ? powf(c->m0, (float) (h + 1))
                                       : powf(c->m1, (float) (2 * (h - c->n_head_log2) + 1));
        }
        /* Q row converted to K's vec_dot type (F16 / BF16), as ggml-cpu does */
        const char *qp = (const char *) c->q->data + iq1 * c->q->nb[1] + iq2 * c->q->nb[2] + iq3 * c->q->nb[3];
        for (int64_t d = 0; d < D; ++d) {
            float x = tget(c->q, qp + d * c->q->nb[0]);
            if (c->k->type == TSK_TYPE_F16) x = orc_fp16_to_fp32(orc_fp32_to_fp16(x));
            else if (c->k->type == TSK_TYPE_BF16) x = orc_bf16_to_fp32(orc_fp32_to_bf16(x));
            Qc[d] = x;
        }
        /* q.k of every key, each one summed over d in order in fp64 (exact
         * products); four keys side by side as independent chains */
        int64_t ic = 0;
        for (; ic + 4 <= c->Nkv; ic += 4) {
            const float *k0 = sl.K + ic * D;
            double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
            for (int64_t d = 0; d < D; ++d) {
                const double qd = (double) Qc[d];
                s0 += qd * (double) k0[d];
                s1 += qd * (double) k0[D + d];
                s2 += qd * (double) k0[2 * D + d];
                s3 += qd * (double) k0[3 * D + d];
            }
            sdots[ic] = s0; sdots[ic + 1] = s1; sdots[ic + 2] = s2; sdots[ic + 3] = s3;
        }
        for (; ic < c->Nkv; ++ic) {
            double sd = 0.0;
            for (int64_t d = 0; d < D; ++d) sd += (double) Qc[d] * (double) sl.K[ic * D + d];
            sdots[ic] = sd;
        }
        const char *mp = NULL;
        if (c->mask) {
            const tsk_tensor *mk = c->mask;
            mp = (const char *) mk->data + iq1 * mk->nb[1] + (iq2 % mk->ne[2]) * mk->nb[2] + (iq3 % mk->ne[3]) * mk->nb[3];
        }
        double S = 0.0; float M = -INFINITY;
        for (int64_t d = 0; d < Dv; ++d) { acc[d] = 0.0; acc16[d] = 0; }
        const int f16acc = c->vacc_f16 && c->v->type == TSK_TYPE_F16;
        for (ic = 0; ic < c->Nkv; ++ic) {
            float mv = 0.0f;
            if (mp) {
                float mval = c->mask->type == TSK_TYPE_F16 ? orc_fp16_to_fp32(((const uint16_t *) mp)[ic])
                                                           : ((const float *) mp)[ic];
                mv = slope * mval;
                if (mv == -INFINITY) continue;
            }
            float s = (float) sdots[ic] * scale;
            if (c->softcap != 0.0f) s = c->softcap * tanhf(s);
            s += mv;
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            const float *Vr = sl.V + ic * Dv;
            if (s > M) { M = s; ms = expf(Mold - M); } else { vs = expf(s - M); }
            if (f16acc) {
                /* ggml_vec_scale_f16 / ggml_vec_mad_f16: every update rounds to fp16 */
                if (ms != 1.0f)
                    for (int64_t d = 0; d < Dv; ++d) acc16[d] = orc_fp32_to_fp16(orc_fp16_to_fp32(acc16[d]) * ms);
                for (int64_t d = 0; d < Dv; ++d) acc16[d] = orc_fp32_to_fp16(orc_fp16_to_fp32(acc16[d]) + Vr[d] * vs);
            } else {
                if (ms != 1.0f) for (int64_t d = 0; d < Dv; ++d) acc[d] *= (double) ms;
                for (int64_t d = 0; d < Dv; ++d) acc[d] += (double) Vr[d] * (double) vs;
            }
            S = S * (double) ms + (double) vs;
        }
        const double S_inv = S == 0.0 ? 0.0 : 1.0 / S;
        /* permuted result: dst[(iq3*ne2*ne1 + iq2 + iq1*ne1)] with ne1 = H */
        float *o = (float *) ((char *) c->dst->data + iq2 * c->dst->nb[1] + iq1 * c->dst->nb[2] + iq3 * c->dst->nb[3]);
        for (int64_t d = 0; d < Dv; ++d) {
            double a = f16acc ? (double) orc_fp16_to_fp32(acc16[d]) : acc[d];
            o[d] = (float) (a * S_inv);
        }
    }
    free(Qc); free(acc); free(acc16); free(sl.K); free(sl.V); free(sdots);
}

int orc_flash_attn_ext(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v,
                       const tsk_tensor *mask, float scale, float max_bias,
                       float logit_softcap, int vacc_f16, tsk_tensor *dst) {
    if (!q || !k || !v || !dst) return TSK_ERR_INVALID_ARG;
    if (dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    fa_ctx c; memset(&c, 0, sizeof(c));
    c.q = q; c.k = k; c.v = v; c.mask = mask; c.dst = dst;
    c.scale = scale; c.max_bias = max_bias; c.softcap = logit_softcap; c.vacc_f16 = vacc_f16;
    c.D = q->ne[0]; c.Nq = q->ne[1]; c.H = q->ne[2]; c.B = q->ne[3];
    c.Nkv = k->ne[1]; c.Hkv = k->ne[2]; c.Dv = v->ne[0];
    if (k->ne[0] != c.D || v->ne[1] != c.Nkv || v->ne[2] != c.Hkv || c.H % c.Hkv) return TSK_ERR_SHAPE;
    if (dst->ne[0] != c.Dv || dst->ne[1] != c.H || dst->ne[2] != c.Nq || dst->ne[3] != c.B) return TSK_ERR_SHAPE;
    c.n_head_log2 = 1u << (uint32_t) floor(log2((double) c.H));
    c.m0 = powf(2.0f, -(max_bias) / (float) c.n_head_log2);
    c.m1 = powf(2.0f, -(max_bias / 2.0f) / (float) c.n_head_log2);
    orc_parallel(c.Nq * c.H * c.B, fa_rows, &c);
    return TSK_OK;
}

/* ------------------------------------------------------------------------ */
/* rms_norm (+mul), norm, rope_ext                                          */
/* ------------------------------------------------------------------------ */

/* ggml_rms_norm: sum of squares in fp64, y = x * 1/sqrtf(mean + eps);
 * then ggml_mul(., w) (src/mmdit.cpp:78-80). */
int orc_rms_norm_mul(const tsk_tensor *x, const float *w, float eps, tsk_tensor *dst) {
    if (!x || !dst) return TSK_ERR_INVALID_ARG;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    const int64_t ne0 = x->ne[0];
    for (int64_t i3 = 0; i3 < x->ne[3]; ++i3)
    for (int64_t i2 = 0; i2 < x->ne[2]; ++i2)
    for (int64_t i1 = 0; i1 < x->ne[1]; ++i1) {
        const float *xr = (const float *) ((const char *) x->data + i1 * x->nb[1] + i2 * x->nb[2] + i3 * x->nb[3]);
        float *yr = (float *) ((char *) dst->data + i1 * dst->nb[1] + i2 * dst->nb[2] + i3 * dst->nb[3]);
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; ++i) sum += (double) (xr[i] * xr[i]);
        const float mean = (float) (sum / (double) ne0);
        const float sc = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < ne0; ++i) {
            float y = xr[i] * sc;
            yr[i] = w ? y * w[i] : y;
        }
    }
    return TSK_OK;
}

/* ggml_norm (src/mmdit.cpp:59, eps 1e-5): mean and variance in fp64. */
int orc_norm(const tsk_tensor *x, float eps, tsk_tensor *dst) {
    if (!x || !dst) return TSK_ERR_INVALID_ARG;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    const int64_t ne0 = x->ne[0];
    for (int64_t i3 = 0; i3 < x->ne[3]; ++i3)
    for (int64_t i2 = 0; i2 < x->ne[2]; ++i2)
    for (int64_t i1 = 0; i1 < x->ne[1]; ++i1) {
        const float *xr = (const float *) ((const char *) x->data + i1 * x->nb[1] + i2 * x->nb[2] + i3 * x->nb[3]);
        float *yr = (float *) ((char *) dst->data + i1 * dst->nb[1] + i2 * dst->nb[2] + i3 * dst->nb[3]);
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; ++i) sum += (double) xr[i];
        const float mean = (float) (sum / (double) ne0);
        double sum2 = 0.0;
        for (int64_t i = 0; i < ne0; ++i) { float v = xr[i] - mean; yr[i] = v; sum2 += (double) (v * v); }
        const float variance = (float) (sum2 / (double) ne0);
        const float sc = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < ne0; ++i) yr[i] *= sc;
    }
    return TSK_OK;
}

/* ggml_rope_ext NORMAL (src/mmdit.cpp:96-99): the angle of pair i is built by
 * ggml-cpu's rope cache as a running product theta = p; theta *= theta_scale,
 * theta_scale = powf(base, -2/n_dims), then scaled by freq_scale; cos/sin in
 * fp32. Dimensions past n_dims are copied. */
int orc_rope_ext(const tsk_tensor *x, const int32_t *pos, int n_dims, float freq_base,
                 float freq_scale, tsk_tensor *dst) {
    if (!x || !dst || !pos) return TSK_ERR_INVALID_ARG;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    const int64_t ne0 = x->ne[0];
    if (n_dims > ne0 || (n_dims & 1)) return TSK_ERR_SHAPE;
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    float *cache = (float *) malloc(sizeof(float) * (size_t) ne0);
    for (int64_t i3 = 0; i3 < x->ne[3]; ++i3)
    for (int64_t i2 = 0; i2 < x->ne[2]; ++i2) {
        const float p = (float) pos[i2];
        float theta = p;
        for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
            const float th = freq_scale * theta;
            cache[i0 + 0] = cosf(th);
            cache[i0 + 1] = sinf(th);
            theta *= theta_scale;
        }
        for (int64_t i1 = 0; i1 < x->ne[1]; ++i1) {
            const float *xr = (const float *) ((const char *) x->data + i1 * x->nb[1] + i2 * x->nb[2] + i3 * x->nb[3]);
            float *yr = (float *) ((char *) dst->data + i1 * dst->nb[1] + i2 * dst->nb[2] + i3 * dst->nb[3]);
            for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
                const float c0 = cache[i0], s0 = cache[i0 + 1];
                const float x0 = xr[i0], x1 = xr[i0 + 1];
                yr[i0]     = x0 * c0 - x1 * s0;
                yr[i0 + 1] = x0 * s0 + x1 * c0;
            }
            for (int64_t i0 = n_dims; i0 < ne0; ++i0) yr[i0] = xr[i0];
        }
    }
    free(cache);
    return TSK_OK;
}

float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* GELU, tanh approximation: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) */
float orc_gelu_tanh(float x) {
    const double c = 0.7978845608028654; /* sqrt(2/pi) */
    double xd = x;
    return (float) (0.5 * xd * (1.0 + tanh(c * (xd + 0.044715 * xd * xd * xd))));
}
