/*
 * tsk_oracle_conv.c — CPU restatement of the convolution and SwiGLU nodes of
 * the reference graph (src/mmdit.cpp:20-52). TEST INFRASTRUCTURE ONLY: the
 * checker of tsk_im2col_1d / tsk_conv1d / tsk_swiglu / tsk_conv_mlp_swiglu /
 * tsk_mlp_swiglu.
 *
 * Each function builds the same node chain the reference builds, in the
 * reference's own order: ggml_cont(ggml_transpose(x)) -> ggml_im2col (F32) ->
 * ggml_mul_mat(reshape_2d(w, KW*IC, OC), cols) -> ggml_add(bias), then
 * silu / mul for the MLPs. ggml_mul_mat is orc_mul_mat (src1 converted to the
 * kernel's vec_dot type, sums in double).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "tsk_oracle.h"

static int64_t conv_len(int64_t IW, int64_t KW, int s0, int p0, int d0) {
    return (IW + 2 * (int64_t) p0 - (int64_t) d0 * (KW - 1) - 1) / s0 + 1;
}

/* ggml_im2col, 1-D, F32 destination (conv1d_f32, src/mmdit.cpp:21): for
 * batch n, output position ow, channel ic and tap kw,
 * dst[n][ow][ic*KW + kw] = x[n][ic][ow*s0 + kw*d0 - p0], 0 outside [0, IW). */
int orc_im2col_1d(int KW, const tsk_tensor *x, int s0, int p0, int d0, tsk_tensor *dst) {
    if (!x || !dst || KW < 1 || s0 < 1 || d0 < 1 || p0 < 0) return TSK_ERR_INVALID_ARG;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    const int64_t IW = x->ne[0], IC = x->ne[1], N = x->ne[2];
    const int64_t OW = conv_len(IW, KW, s0, p0, d0);
    if (OW < 1 || dst->ne[0] != IC * KW || dst->ne[1] != OW || dst->ne[2] != N) return TSK_ERR_SHAPE;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t ow = 0; ow < OW; ++ow) {
            float *row = (float *) ((char *) dst->data + n * dst->nb[2] + ow * dst->nb[1]);
            for (int64_t ic = 0; ic < IC; ++ic)
                for (int64_t kw = 0; kw < KW; ++kw) {
                    const int64_t iw = ow * s0 + kw * d0 - p0;
                    float v = 0.0f;
                    if (iw >= 0 && iw < IW)
                        v = *(const float *) ((const char *) x->data + n * x->nb[2] + ic * x->nb[1] + iw * x->nb[0]);
                    row[ic * KW + kw] = v;
                }
        }
    return TSK_OK;
}

/* conv_cl (src/mmdit.cpp:28-34) on contiguous host tensors:
 *   w   ne = [KW, IC, OC] F32 / BF16 / F16 (ggml layout, contiguous)
 *   x   F32 ne = [IC, IW, B]   (channels fastest)
 *   dst F32 ne = [OC, OW, B]
 * Per batch item: xt = cont(transpose(x)) ne = [IW, IC]; cols = im2col;
 * dst = mul_mat(w as [KW*IC, OC], cols) + bias. */
int orc_conv1d(const tsk_tensor *w, const tsk_tensor *bias, const tsk_tensor *x, int s0, int p0, int d0,
               tsk_tensor *dst) {
    if (!w || !x || !dst) return TSK_ERR_INVALID_ARG;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32) return TSK_ERR_TYPE;
    const int64_t KW = w->ne[0], IC = w->ne[1], OC = w->ne[2];
    const int64_t IW = x->ne[1], B = x->ne[2];
    if (x->ne[0] != IC) return TSK_ERR_SHAPE;
    const int64_t OW = conv_len(IW, KW, s0, p0, d0);
    if (OW < 1 || dst->ne[0] != OC || dst->ne[1] != OW || dst->ne[2] != B) return TSK_ERR_SHAPE;
    float *xt = (float *) malloc(sizeof(float) * (size_t) (IW * IC));
    float *cols = (float *) malloc(sizeof(float) * (size_t) (OW * IC * KW));
    int rc = TSK_OK;
    for (int64_t b = 0; b < B && rc == TSK_OK; ++b) {
        /* ggml_cont(ggml_transpose(x)): [IC, IW] -> [IW, IC] */
        for (int64_t ic = 0; ic < IC; ++ic)
            for (int64_t iw = 0; iw < IW; ++iw)
                xt[ic * IW + iw] =
                    *(const float *) ((const char *) x->data + b * x->nb[2] + iw * x->nb[1] + ic * x->nb[0]);
        tsk_tensor tx = {TSK_TYPE_F32, {IW, IC, 1, 1},
                         {4, (size_t) IW * 4, (size_t) (IW * IC) * 4, (size_t) (IW * IC) * 4}, xt};
        tsk_tensor tc = {TSK_TYPE_F32, {IC * KW, OW, 1, 1},
                         {4, (size_t) (IC * KW) * 4, (size_t) (IC * KW * OW) * 4, (size_t) (IC * KW * OW) * 4}, cols};
        if ((rc = orc_im2col_1d((int) KW, &tx, s0, p0, d0, &tc))) break;
        /* ggml_reshape_2d(w, KW*IC, OC): the kernel's rows of K = KW*IC */
        tsk_tensor wr = *w;
        wr.ne[0] = KW * IC; wr.ne[1] = OC; wr.ne[2] = 1; wr.ne[3] = 1;
        wr.nb[1] = w->nb[2]; wr.nb[2] = wr.nb[3] = w->nb[2] * (size_t) OC;
        tsk_tensor td = *dst;
        td.data = (char *) dst->data + b * dst->nb[2];
        td.ne[2] = 1; td.ne[3] = 1;
        rc = orc_mul_mat(&wr, &tc, bias, &td);
    }
    free(xt);
    free(cols);
    return rc;
}

/* ggml_mul(ggml_silu(a), b) over n floats; silu(x) = x / (1 + exp(-x)) */
void orc_swiglu(const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_silu(a[i]) * b[i];
}

/* convmlp (src/mmdit.cpp:39-44): conv_cl(w2, silu(conv_cl(w1, x)) * conv_cl(w3, x)),
 * every conv stride 1, padding 1, dilation 1, no bias. x F32 [IC, IW, B];
 * dst F32 [OC, OW2, B]. */
int orc_conv_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, const tsk_tensor *x,
                        tsk_tensor *dst) {
    if (!w1 || !w3 || !w2 || !x || !dst) return TSK_ERR_INVALID_ARG;
    const int64_t HID = w1->ne[2], B = x->ne[2];
    const int64_t OW1 = conv_len(x->ne[1], w1->ne[0], 1, 1, 1);
    if (OW1 < 1 || w3->ne[2] != HID || w2->ne[1] != HID) return TSK_ERR_SHAPE;
    const size_t nh = (size_t) (HID * OW1 * B);
    float *h1 = (float *) malloc(sizeof(float) * nh);
    float *h3 = (float *) malloc(sizeof(float) * nh);
    tsk_tensor t1 = {TSK_TYPE_F32, {HID, OW1, B, 1}, {4, (size_t) HID * 4, (size_t) (HID * OW1) * 4, nh * 4}, h1};
    tsk_tensor t3 = t1;
    t3.data = h3;
    int rc = orc_conv1d(w1, NULL, x, 1, 1, 1, &t1);
    if (!rc) rc = orc_conv1d(w3, NULL, x, 1, 1, 1, &t3);
    if (!rc) {
        orc_swiglu(h1, h3, h1, (int64_t) nh);
        rc = orc_conv1d(w2, NULL, &t1, 1, 1, 1, dst);
    }
    free(h1);
    free(h3);
    return rc;
}

/* mlp (src/mmdit.cpp:47-52): w2 x (silu(w1 x) * (w3 x)), linear, no bias.
 * w1, w3 ne = [IC, HID]; w2 ne = [HID, OC]; x F32 [IC, N]; dst F32 [OC, N]. */
int orc_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, const tsk_tensor *x,
                   tsk_tensor *dst) {
    if (!w1 || !w3 || !w2 || !x || !dst) return TSK_ERR_INVALID_ARG;
    const int64_t HID = w1->ne[1], N = x->ne[1] * x->ne[2] * x->ne[3];
    if (w3->ne[1] != HID || w2->ne[0] != HID) return TSK_ERR_SHAPE;
    const size_t nh = (size_t) (HID * N);
    float *h1 = (float *) malloc(sizeof(float) * nh);
    float *h3 = (float *) malloc(sizeof(float) * nh);
    tsk_tensor t1 = {TSK_TYPE_F32, {HID, N, 1, 1}, {4, (size_t) HID * 4, nh * 4, nh * 4}, h1};
    tsk_tensor t3 = t1;
    t3.data = h3;
    int rc = orc_mul_mat(w1, x, NULL, &t1);
    if (!rc) rc = orc_mul_mat(w3, x, NULL, &t3);
    if (!rc) {
        orc_swiglu(h1, h3, h1, (int64_t) nh);
        rc = orc_mul_mat(w2, &t1, NULL, dst);
    }
    free(h1);
    free(h3);
    return rc;
}
