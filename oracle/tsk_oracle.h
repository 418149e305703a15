/*
 * tsk_oracle.h — CPU restatement of the ggml-cpu arithmetic behind the
 * thinksound.cpp MM-DiT hot path.  TEST INFRASTRUCTURE ONLY: this is the
 * checker the HIP path is compared against (and the timed CPU baseline). The
 * product library never links or calls it.
 *
 * The arithmetic being restated lives in ggml (github.com/ggml-org/ggml), an
 * un-vendored submodule of the reference (.gitmodules:1-3); the published
 * numbers were made with the ggml of llama.cpp commit 911b67a60
 * (docs/PROGRESS.md:17). ggml is absent from this container, so each function
 * restates ggml's published algorithm and cites the reference call site that
 * emits the node. Tensors use ggml's ne/nb conventions (tsk_tensor) with HOST
 * data pointers.
 */
#ifndef TSK_ORACLE_H
#define TSK_ORACLE_H

#include <stddef.h>
#include <stdint.h>
#include "../include/tsk/tsk.h"

#ifdef __cplusplus
extern "C" {
#endif

/* threads used by the parallel loops below (default 1) */
void     orc_set_threads(int n);
int      orc_get_threads(void);
/* run fn over [0, n) in contiguous chunks on those threads */
typedef void (*orc_range_fn)(void *ctx, int64_t lo, int64_t hi);
void     orc_parallel(int64_t n, orc_range_fn fn, void *ctx);

/* scalar conversions, round-to-nearest-even (ggml GGML_FP32_TO_FP16 / _BF16) */
uint16_t orc_fp32_to_fp16(float f);
float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_bf16(float f);
float    orc_bf16_to_fp32(uint16_t h);
void     orc_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n);
void     orc_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n);
void     orc_fp32_to_bf16_row(const float *x, uint16_t *y, int64_t n);
void     orc_bf16_to_fp32_row(const uint16_t *x, float *y, int64_t n);

/* Q8_0 (34-byte blocks {fp16 d; int8 qs[32]}) */
enum orc_q8_mode {
    ORC_Q8_CPU_SIMD = 0,  /* ggml-cpu x86 quantize_row_q8_0: d=amax/127, q=rne(x*127/amax) */
    ORC_Q8_CPU_REF  = 1,  /* quantize_row_q8_0_ref: q=roundf(x*(1/d)) (half away)        */
    ORC_Q8_GGUF_PY  = 2   /* gguf-py quants.Q8_0: q=roundf(x/d) (half away)               */
};
void     orc_quantize_q8_0(const float *x, void *blocks, int64_t n, int mode);
void     orc_dequantize_q8_0(const void *blocks, float *y, int64_t n);

/* ggml_mul_mat: dst[M,N,..] = a[K,M] x b[K,N,..] (+bias[M]); dst F32. */
int      orc_mul_mat(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias,
                     tsk_tensor *dst);

/* ggml_flash_attn_ext (ggml-cpu one-row-at-a-time online softmax).
 * vacc_f16 = 1 reproduces ggml-cpu's fp16 V accumulator for F16 V; 0 keeps
 * the accumulator in fp64 (exact reference for the same rounded inputs). */
int      orc_flash_attn_ext(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v,
                            const tsk_tensor *mask, float scale, float max_bias,
                            float logit_softcap, int vacc_f16, tsk_tensor *dst);

/* ggml_rms_norm followed by ggml_mul with w (w may be NULL). F32 only. */
int      orc_rms_norm_mul(const tsk_tensor *x, const float *w, float eps, tsk_tensor *dst);
/* ggml_norm (no affine). F32 only. */
int      orc_norm(const tsk_tensor *x, float eps, tsk_tensor *dst);
/* ggml_rope_ext NORMAL mode, ext_factor 0, attn_factor 1. F32 only. */
int      orc_rope_ext(const tsk_tensor *x, const int32_t *pos, int n_dims, float freq_base,
                      float freq_scale, tsk_tensor *dst);

/* elementwise helpers used by the DiT restatement */
float    orc_silu(float x);

/* convolution / SwiGLU nodes (tsk_oracle_conv.c, src/mmdit.cpp:20-52) */
int      orc_im2col_1d(int KW, const tsk_tensor *x, int s0, int p0, int d0, tsk_tensor *dst);
int      orc_conv1d(const tsk_tensor *w, const tsk_tensor *bias, const tsk_tensor *x, int s0, int p0,
                    int d0, tsk_tensor *dst);
void     orc_swiglu(const float *a, const float *b, float *y, int64_t n);
int      orc_conv_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2,
                             const tsk_tensor *x, tsk_tensor *dst);
int      orc_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2,
                        const tsk_tensor *x, tsk_tensor *dst);
float    orc_gelu_tanh(float x);

/* ---- MM-DiT flow step (BASELINE textbook configuration) ------------------
 * Structure of ts_dit::forward (src/mmdit.cpp:119-342) with the benchmarked
 * block shape: linear layers, GELU(tanh) MLP, two streams (latent, text),
 * adaLN from the timestep embedding. Weights are given by name as host F32
 * arrays (already rounded the way the device holds them). */
typedef struct orc_dit orc_dit;
orc_dit *orc_dit_create(const tsk_dit_config *cfg);
void     orc_dit_destroy(orc_dit *d);
int      orc_dit_set_tensor(orc_dit *d, const char *name, const float *src, int64_t n);
/* weight_type Q8_0: the block projections' ggml Q8_0 blocks, as stored */
int      orc_dit_set_tensor_q8_0(orc_dit *d, const char *name, const void *blocks, size_t nbytes);
int      orc_dit_n_tensors(const orc_dit *d);
/* name and ggml ne[0], ne[1] of the i-th weight */
int      orc_dit_tensor_info(const orc_dit *d, int i, const char **name, int64_t *ne0, int64_t *ne1);
/* act_bf16 = 1 rounds the activations of the per-block projections (qkv,
 * linear1, fc1, fc2) to bf16 (ggml's BF16-weight mul_mat) and keeps F32
 * activations for the conditioning, input and output projections (the device
 * path's precision policy); 0 keeps all activations F32 (the "GGML F32
 * path"). kv_f16 = 1 casts K/V to F16 before attention as mmdit.cpp:89-90. */
int      orc_dit_forward(orc_dit *d, int B, int T, const float *latent, const float *t,
                         const float *text, float *flow, int act_bf16, int kv_f16);
int      orc_dit_sample(orc_dit *d, int T, const float *noise, const float *text_cond,
                        const float *text_uncond, int steps, float cfg_scale, float *out,
                        float *flow0, int act_bf16, int kv_f16);

/* ---- The reference's MM-DiT graph (ts_dit::forward / ::sample,
 * src/mmdit.cpp:119-376), tsk_oracle_mmdit.c --------------------------------
 * Weights by the converter's names from host f32 in ggml order (or Q8_0
 * blocks), each stored in the type cfg->weight_type's converter rule gives it
 * (orc_mmdit_set_type overrides one); with act_bf16 the products run in the
 * stored types (BF16: src1 rounded; Q8_0: src1 quantized), else all in F32 on
 * the same values. kv_f16 casts K / V to F16 (mmdit.cpp:89-90). Layouts as
 * tsk_mmdit_forward / tsk_mmdit_sample. */
typedef struct orc_mmdit orc_mmdit;
orc_mmdit *orc_mmdit_create(const tsk_mmdit_config *cfg);
void     orc_mmdit_destroy(orc_mmdit *m);
int      orc_mmdit_n_tensors(const orc_mmdit *m);
int      orc_mmdit_tensor_info(const orc_mmdit *m, int i, const char **name, int64_t ne[3], int *type);
int      orc_mmdit_set_tensor(orc_mmdit *m, const char *name, const float *src, int64_t n);
int      orc_mmdit_set_tensor_q8_0(orc_mmdit *m, const char *name, const void *blocks, size_t nbytes);
int      orc_mmdit_set_type(orc_mmdit *m, const char *name, int type);
int      orc_mmdit_forward(orc_mmdit *m, int B, int T, const float *latent, const float *t, int clip_S,
                           const float *clip_f, int sync_S, const float *sync_f, const float *text_f,
                           const float *t5, const float *global_text, float *flow, int act_bf16, int kv_f16);
/* stage outputs of the last orc_mmdit_forward by the reference's debug names
 * (x_in, t_emb, clip_pp, text_pp, clip_fc, text_fc, gcmlp, global_c,
 * extended_c, jb0_lat, jb0_clip, jb0_text, after_joint, after_fused; ggml
 * [H, S] per batch row, rows concatenated); size -1 if absent */
int64_t  orc_mmdit_stage_size(const orc_mmdit *m, const char *name);
int      orc_mmdit_stage(const orc_mmdit *m, const char *name, float *out, int64_t n);
int      orc_mmdit_sample(orc_mmdit *m, int T, const float *noise, int clip_S, const float *clip_f, int sync_S,
                          const float *sync_f, const float *text_f, const float *t5, const float *global_text,
                          int steps, float cfg_scale, float *out, float *flow0, int act_bf16, int kv_f16);

/* ---- Oobleck VAE decoder (ts_vae::decode, src/vae_decoder.cpp:62-124),
 * tsk_oracle_vae.c: weights by the converter's names from host f32 in ggml
 * order; latent [latent_dim][T] -> audio [out_channels][T * hop]. */
typedef struct orc_vae orc_vae;
orc_vae *orc_vae_create(const tsk_vae_config *cfg);
void     orc_vae_destroy(orc_vae *v);
int      orc_vae_n_tensors(const orc_vae *v);
int      orc_vae_tensor_info(const orc_vae *v, int i, const char **name, int64_t ne[3]);
int      orc_vae_set_tensor(orc_vae *v, const char *name, const float *src, int64_t n);
int      orc_vae_decode(orc_vae *v, int T, const float *latent, float *audio);

/* ---- T5 encoder stack (ts_t5::encode, src/t5_encoder.cpp:40-104) ---------
 * Relative-position bucket of t5_encoder.cpp:14-26 (bidirectional). */
int      orc_t5_bucket(int rel, int num_buckets, int max_dist);
/* The attention of one T5 layer as the reference graph computes it
 * (t5_encoder.cpp:68-75): per head h, s[q][k] = sum_d k[k][d] q[q][d] (no
 * scale) + mask[h][q][k]; soft_max over k (ggml-cpu: max subtracted, expf,
 * sum in double, scaled by 1/sum); o[q][d] = sum_k v[k][d] p[q][k].
 * q, k, v: rows of n tokens with H heads of D values at row stride ld
 * (floats); mask [H][n][n]; out [n][H][D]. */
int      orc_t5_attention(const float *q, const float *k, const float *v, int64_t ld, const float *mask,
                          int n, int H, int D, float *out);
/* Whole encoder stack on embedded tokens x [n][d_model] with key padding from
 * ids (id 0 = padded key, t5_encoder.cpp:97): weights by the converter's
 * names, matrices as ggml Q8_0 blocks (or F32), vectors F32. */
typedef struct orc_t5 orc_t5;
orc_t5  *orc_t5_create(const tsk_t5_config *cfg);
void     orc_t5_destroy(orc_t5 *t);
int      orc_t5_n_tensors(const orc_t5 *t);
int      orc_t5_tensor_info(const orc_t5 *t, int i, const char **name, int64_t *ne0, int64_t *ne1, int *type);
/* data: Q8_0 blocks (type Q8_0) or floats (type F32), nbytes checked */
int      orc_t5_set_tensor(orc_t5 *t, const char *name, const void *data, size_t nbytes);
int      orc_t5_encode(orc_t5 *t, int n, const float *x, const int32_t *ids, float *out);
/* layers [layer_begin, layer_end), then out_norm if final_norm */
int      orc_t5_encode_range(orc_t5 *t, int n, const float *x, const int32_t *ids, int layer_begin,
                             int layer_end, int final_norm, float *out);

#ifdef __cplusplus
}
#endif
#endif
