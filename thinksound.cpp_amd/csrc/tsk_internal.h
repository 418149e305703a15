// tsk_internal.h — kernel parameter blocks and launchers shared by the C ABI
// (tsk_api.cpp) and the MM-DiT driver (dit.cpp). Host-side validation has
// already happened when a launcher is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tsk/tsk.h"

namespace tsk {

// ---------------------------------------------------------------- attention
struct AttnParams {
    const void *q, *k, *v, *mask;
    void *o;
    int q_type, kv_type;          // tsk_type
    int out_bf16;                 // 0: f32 dst, 1: bf16 dst
    int mask_f16;                 // mask element type (1: F16, 0: F32)
    int Nq, Nkv, H, Hkv, B;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int m_ne2, m_ne3;
    int64_t o_nb1, o_nb2, o_nb3;  // dst ne = [D, H, Nq, B]
    float scale;                  // divided by softcap when softcap != 0 (ggml)
    float softcap;
    float max_bias, m0, m1;
    uint32_t n_head_log2;
};
hipError_t launch_attention(const AttnParams &p, hipStream_t s);

// ---------------------------------------------------------------- GEMM
// Y[n, m] = epi( sum_k X[n, k] * W[m, k] + bias[m] ), n < N tokens, m < M.
enum GemmEpi : int {
    EPI_STORE = 0,      // Y = acc (+bias)
    EPI_GELU = 1,       // Y = gelu_tanh(acc + bias)
    EPI_GATE_RES = 2    // R[n, m] += gate[n / rows_per_gate, m] * (acc + bias); Y unused
};

struct GemmParams {
    const void *x;           // activations: bf16 or f32 rows of K
    const void *w;           // weights: bf16 rows of K, or Q8_0_SPLIT planes
    const float *bias;       // nullable, [M]
    void *y;                 // output rows of M: f32 or bf16
    float *res;              // EPI_GATE_RES: f32 residual rows of M (in/out)
    const float *gate;       // EPI_GATE_RES: gate rows of M (row stride ld_gate)
    int64_t ld_x, ld_w, ld_y, ld_res, ld_gate;  // row strides in elements
    // optional grouping of activation rows: row n of X starts at
    // x + (n / x_group_rows) * x_group_stride + (n % x_group_rows) * ld_x
    // (x_group_rows == 0: plain row stride)
    int x_group_rows;
    int64_t x_group_stride;
    int M, N, K;
    int rows_per_gate;
    int x_f32, y_bf16, epi;
    int x_split;             // f32 activations as bf16 hi + lo (two MFMAs): f32-grade products
    // Q8_0: activations pre-quantized into planes qx [N][K] int8 and
    // dx [N][K/32] f32 (fp16-representable scales)
    const int8_t *qx;
    const float *dx;
    const int8_t *qw;        // [M][K]
    const uint16_t *dw;      // [M][K/32] fp16 bits
};
hipError_t launch_gemm_bf16(const GemmParams &p, hipStream_t s);
hipError_t launch_gemm_q8(const GemmParams &p, hipStream_t s);
// Activation quantization to planes for launch_gemm_q8 (ggml-cpu x86 rounding).
// x rows of K (f32 or bf16, row stride ld_x elements).
hipError_t launch_quantize_rows_q8(const void *x, int x_f32, int64_t ld_x, int N, int K,
                                   int8_t *qx, float *dx, hipStream_t s);

// ---------------------------------------------------------------- small ops
// generic 4-D strided views used by the C-ABI element-wise entry points
struct View4 {
    void *data;
    int type;
    int64_t ne[4];
    int64_t nb[4];
};
hipError_t launch_rms_norm_mul(const View4 &x, const float *w, float eps, const View4 &y,
                               hipStream_t s);
hipError_t launch_norm(const View4 &x, float eps, const View4 &y, hipStream_t s);
hipError_t launch_rope(const View4 &x, const int32_t *pos, int n_dims, float theta_scale,
                       float freq_scale, const View4 &y, hipStream_t s);
hipError_t launch_qk_norm_rope(const View4 &x, const float *w, const int32_t *pos, float eps,
                               int n_dims, float theta_scale, float freq_scale, const View4 &y,
                               hipStream_t s);
hipError_t launch_q8_quantize_blocks(const float *x, int64_t ld_x, int64_t rows, int64_t K,
                                     void *blocks, int64_t ld_blocks, hipStream_t s);
hipError_t launch_q8_dequantize(const void *src, int split, int64_t rows, int64_t K,
                                int64_t ld_src, float *y, int64_t ld_y, hipStream_t s);
hipError_t launch_q8_repack(const void *src, int64_t ld_src, int64_t rows, int64_t K,
                            void *dst, hipStream_t s);
hipError_t launch_f32_to_bf16(const float *x, uint16_t *y, int64_t n, hipStream_t s);

// ---------------------------------------------------------------- DiT glue
// y[r, :] = LN(x[r, :], eps) * (1 + scale[b, :]) + shift[b, :], b = r / rows_per_b;
// x f32 (row stride ld_x), y bf16 (row stride ld_y).
hipError_t launch_ln_modulate(const float *x, int64_t ld_x, int rows, int H, int rows_per_b,
                              const float *shift, const float *scale, int64_t ld_mod, float eps,
                              uint16_t *y, int64_t ld_y, hipStream_t s);
hipError_t launch_ln_modulate_f32(const float *x, int64_t ld_x, int rows, int H, int rows_per_b,
                                  const float *shift, const float *scale, int64_t ld_mod, float eps,
                                  float *y, int64_t ld_y, hipStream_t s);
// Split the QKV GEMM output (f32 rows of [q | k | v], head-major) into the
// fp16 attention layout [B, nh, Ntot, 64] at token offset tok_off, applying
// RMSNorm*w to q and k and (if rope) RoPE with position = row % S.
hipError_t launch_qkv_prologue(const float *qkv, int rows, int S, int nh,
                               const float *qn_w, const float *kn_w, float eps, int rope,
                               float theta_scale, float freq_scale, uint16_t *q, uint16_t *k,
                               uint16_t *v, int Ntot, int tok_off, hipStream_t s);
// A list of small-batch GEMVs with f32 activations (products exact in fp32):
// out[b, j] = act( sum_k W[j, k] * x[b, k] + bias[j] ), act = silu if silu_out
struct GemvJob {
    const uint16_t *w;     // bf16 [M][K]
    const float *bias;     // [M], nullable
    const float *x;        // [B][K] f32
    float *out;            // [B][ld_out]
    int M;
    int silu_out;
    int64_t ld_out;
};
hipError_t launch_gemv_jobs(const GemvJob *jobs_dev, int njobs, int max_m, int B, int K,
                            hipStream_t s);
hipError_t launch_silu_inplace(float *x, int64_t n, hipStream_t s);
// t-embedding: temb[b, k] = cos(t_b * freq[k]), temb[b, H/2 + k] = sin(t_b * freq[k])
struct TimeVals { float t[32]; };
hipError_t launch_timestep_embed(const float *freq, const TimeVals &tv, int B, int H, float *temb,
                                 hipStream_t s);
// CFG combine + Euler step: x[i] += dt * (fu + (fc - fu) * cfg); flow0 optional
hipError_t launch_cfg_euler(const float *flow2, int64_t n, float cfg, float dt, float *x,
                            float *x2, float *flow0, hipStream_t s);

}  // namespace tsk
