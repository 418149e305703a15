// tsk_internal.h — kernel parameter blocks and launchers shared by the C ABI
// (tsk_api.cpp) and the MM-DiT driver (dit.cpp). Host-side validation has
// already happened when a launcher is called.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tsk/tsk.h"

namespace tsk {

// Kernel timing of the step driver: while `stop` is set on the calling
// thread, launch_kernel() launches with hipExtLaunchKernelGGL so that the
// dispatch packets themselves stamp `start` (first launch) and `stop` (every
// launch; the last one stands): the events then bracket kernel execution only.
struct LaunchEvents {
    hipEvent_t start, stop;
};
LaunchEvents &launch_events();
template <typename F, typename... Args>
inline void launch_kernel(F kern, const dim3 &grid, const dim3 &block, size_t shm, hipStream_t s, Args... args) {
    LaunchEvents &ev = launch_events();
    if (ev.stop) {
        hipExtLaunchKernelGGL(kern, grid, block, (uint32_t) shm, s, ev.start, ev.stop, 0u, args...);
        ev.start = nullptr;
    } else {
        hipLaunchKernelGGL(kern, grid, block, shm, s, args...);
    }
}

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
    // relative-position bias in place of a mask (T5): key k of query q adds
    // rel_lut[h * rel_nh + rel_off + k - q] + (key_valid[k] ? 0 : -inf) -- the
    // value the materialised mask would hold; null: unused
    const float *rel_lut;
    int64_t rel_nh;
    int rel_off;
    const uint8_t *key_valid;
};
hipError_t launch_attention(const AttnParams &p, hipStream_t s);

// Fast path of ggml_flash_attn_ext for head_dim 64, H == Hkv, no mask /
// softcap / ALiBi, 16-bit K (attn_dit.hip): q rows (F32/F16/BF16) and k rows
// (F16/BF16) with ggml byte strides (rows 16-byte aligned), V given
// transposed as fp16 vt [B*H][64][ldv] (slice stride vt_bh elements) with the
// key positions of every 16-key group permuted by vt_pos() (ldv >= Nkv rounded
// up to 64; the positions past Nkv hold finite values), output F32/BF16 in
// ggml's permuted [D, H, Nq, B] byte strides. c = scale * log2(e).
struct AttnFastParams {
    const void *q, *k;
    const uint16_t *vt;  // V^T (below), or with v_rows the F16 V rows themselves:
    const void *v;       // v_rows: F16 rows of 64 (ggml strides v_nb1..3, 16-byte aligned)
    int64_t v_nb1, v_nb2, v_nb3;
    int v_rows;          // fp16 K only: V read as rows, transposed by the LDS reads
    void *o;
    int q_type, k_bf16, out_bf16;
    int Nq, Nkv, H, B;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t vt_bh;
    int ldv;
    int64_t o_nb1, o_nb2, o_nb3;
    float c;
    int q_prescaled;     // q is fp16 (K's type) already multiplied by c: loaded as is
    int bounded;         // fp16 K only: every |q.k| * c <= ATTN_LOGIT_BOUND (no running max)
    int qtiles;          // set by the launcher
    int force_cfg;       // 0: launcher picks; else 10 * key ranges + query blocks
    int rule_b;          // > 0: the batch the launcher's shape rule counts with (a model's capacity,
                         // so that a batch row's key ranges, and so its bits, do not depend on the call's B)
    // > 0: workgroups of head h run on XCD (h / xcd_hdiv) % 8, where a QKV
    // GEMM with xcd_hdiv heads per weight tile wrote that head's q / k / V^T
    // (the launcher drops it unless H is a multiple of 8 * xcd_hdiv); 0: the
    // units of one (batch, head) are consecutive within an XCD in (batch,
    // head) order
    int xcd_hdiv;
    // Q8_0 output (q8x non-null; o is not written): each query row of up to
    // two streams (tokens [q8_tok[i], q8_tok[i] + q8_S[i]) of every batch
    // item) quantized per 32 as quantize_rows_q8 does, into the planes
    // q8x [row][H * 64] int8 and q8d [row][H * 2] f32 (fp16-valued d) at
    // row q8_row[i] + b * q8_S[i] + (token - q8_tok[i]); other tokens are dropped
    int8_t *q8x;
    float *q8d;
    int q8_ns;
    int q8_tok[2], q8_S[2], q8_row[2];
};
// Logit bound (log2 units) under which softmax runs without a running max:
// exp2 of it (~6e3) and sums of it over 2^14 keys stay far inside fp16 / fp32.
constexpr float ATTN_LOGIT_BOUND = 14.0f;
hipError_t launch_attn_fast(const AttnFastParams &p, hipStream_t s);
int attn_fast_default_cfg(int Nq, int H, int B, int k_bf16, int rule_b = 0);
// V (F16/BF16 rows of 64, ggml strides) -> the transposed fp16 layout above
hipError_t launch_vt_transpose(const void *v, int v_bf16, int64_t nb1, int64_t nb2, int64_t nb3, int Nkv, int H,
                               int B, uint16_t *vt, int ldv, hipStream_t s);
// position of key k in a V^T row: bits 2 and 3 swapped
__host__ __device__ inline int vt_pos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

// ---------------------------------------------------------------- GEMM
// Y[n, m] = epi( sum_k X[n, k] * W[m, k] + bias[m] ), n < N tokens, m < M.
enum GemmEpi : int {
    EPI_STORE = 0,      // Y = acc (+bias)
    EPI_GELU = 1,       // Y = gelu_tanh(acc + bias)
    EPI_GATE_RES = 2,   // R[n, m] += gate[n / rows_per_gate, m] * (acc + bias); Y unused
    EPI_GEGLU = 3,      // rows interleaved (a_j, b_j): Y[n, j] = gelu_tanh(a_j) * b_j, M even (Q8_0 only)
    // gelu_tanh(acc + bias) converted to Q8_0 planes for the next Q8_0 GEMM:
    // Y int8 [N][ld_y], yd f32 block scales [N][M / 32] (Q8_0 cooperative
    // tiles only, M % 64 == 0)
    EPI_GELU_Q8 = 4,
    // acc + bias -> the attention operands, the arithmetic of
    // launch_qkv_scatter on each token's 64 features of one head (qs: the
    // scatter's parameters; qkv, ld and rows unused). Q8_0 cooperative 64 x 64
    // tiles only: a tile is one head's q, k or v for 64 tokens
    EPI_QKV_ATTN = 5
};

// The QKV epilogue of the BF16 block GEMMs as a kernel over f32 rows (the
// Q8_0 driver's QKV GEMM stores them): row n = b * seq + s of qkv [rows][3 H]
// ([q | k | v] head-major, bias included) -> RMSNorm(eps) * w on q and k,
// RoPE on q and k from rope_cs (when rope), q * q_scale, fp16 into q / k
// [B][nh][Ntot][64] at token tok_off + s and into V^T [B][nh][64][ldv] at
// vt_pos(tok_off + s), or with v_rows into vt as rows like k.
struct QkvScatter {
    const float *qkv;
    int64_t ld;
    const float *qn_w, *kn_w, *rope_cs;
    uint16_t *q, *k, *vt;
    int ldv, seq, Ntot, tok_off, rope, nh, rows;
    float eps, q_scale;
    int v_rows;          // V into vt as rows like k: fp16 [B][nh][Ntot][64]
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
    // Q8_0: activations pre-quantized into planes qx [N][K] int8 and
    // dx [N][K/32] f32 (fp16-representable scales)
    const int8_t *qx;
    const float *dx;
    const int8_t *qw;        // [M][K]
    const uint16_t *dw;      // [M][K/32] fp16 bits
    // Q8_0 cooperative tiles, split-K (splits > 1, EPI_STORE into f32 y, no
    // bias): slice s sums k in [s K / splits, (s + 1) K / splits) into
    // y + s * part_stride
    int splits;
    int64_t part_stride;
    float *yd;               // EPI_GELU_Q8: block scales of the output planes
    QkvScatter qs;           // EPI_QKV_ATTN
};
hipError_t launch_gemm_bf16(const GemmParams &p, hipStream_t s);

// ---------------------------------------------------------------- grouped GEMM
// One launch runs up to two independent problems (the latent and text streams
// of a joint block), Y[n, m] = sum_k X[n, k] W[m, k], with one of:
enum GroupEpi : int {
    EPI_STORE_F32 = 10,   // y f32 = acc + bias
    EPI_STORE_BF16 = 11,  // y bf16 = acc + bias
    EPI_GELU_BF16 = 12,   // y bf16 = gelu_tanh(acc + bias)
    EPI_QKV = 13,         // acc + bias -> RMSNorm*w (q, k), RoPE, fp16 -> attention layout
    EPI_PARTIAL = 14,     // split-K: y f32 slice [split][N][M] = partial acc (no bias)
    // SwiGLU over two weights sharing X: y[n, m] = silu(X W[m]) * (X W3[m]),
    // no bias (convmlp / mlp, src/mmdit.cpp:39-52)
    EPI_SWIGLU_F32 = 15,
    EPI_SWIGLU_BF16 = 16,
    EPI_F32X = 17         // y f32 = acc + bias (+ y), SnakeBeta into y / y2 / split planes (see GemmProblem)
};
enum GemmFlags : int { GEMM_X_F32 = 1 };

struct GemmProblem {
    const void *x;                 // activations (bf16, or f32 with GEMM_X_F32)
    const uint16_t *w;             // bf16 weights [M][K] row-major (ld_w), or tiled (w_tiled)
    int w_tiled;                   // 1: MFMA-tiled layout of tile_bf16_weights() (M % 16 == 0, K % 32 == 0)
    const float *bias;             // [M] nullable (ignored by EPI_PARTIAL)
    void *y;                       // output (see GroupEpi)
    int64_t ld_x, ld_w, ld_y;      // row strides in elements
    int x_group_rows;              // see GemmParams
    int64_t x_group_stride;
    int M, N, K;
    int splits;                    // K slices (EPI_PARTIAL), else 1
    const uint16_t *w3;            // EPI_SWIGLU_*: the second weight (same layout as w)
    const float *wf;               // launch_gemm_f32: f32 weights [M][K] row-major (ld_w)
    int accumulate;                // launch_gemm_f32: y += acc + bias (f32 y)
    // implicit im2col (conv_ic > 0): row n of X is output position ow = n % conv_ow
    // of batch item b = n / conv_ow, and column k = kw * conv_ic + ic reads
    // x[b * x_group_stride + (ow * conv_s + kw * conv_d - conv_p) * ld_x + ic],
    // zero outside [0, conv_iw) (x_group_rows must be 0, conv_ic % 8 == 0)
    int conv_ic, conv_iw, conv_ow, conv_s, conv_p, conv_d;
    // EPI_QKV: M = 3 * n_head * 64 with [q | k | v] head-major
    const float *qn_w, *kn_w;      // RMSNorm weights [64]
    uint16_t *q, *k;               // fp16 [B][n_head][Ntot][64]
    uint16_t *vt;                  // fp16 [B][n_head][64][ldv], key positions vt_pos()
    int ldv;
    int v_rows;                    // V into vt as rows like k instead: fp16 [B][n_head][Ntot][64]
    int seq;                       // rows per batch item (row n -> b = n / seq, s = n % seq)
    int Ntot, tok_off, rope;
    float theta_scale, freq_scale, eps;
    float q_scale;                 // q is multiplied by this before its fp16 cast
    const float *rope_cs;          // launch_gemm_ks: (cos, sin) of pair i at position s: [s * 64 + 2 i]
    // EPI_F32X (split products of F32 weights): y f32 = acc + bias, plus the
    // old y with accumulate (y nullable: not written), then optionally a
    // SnakeBeta (snk_ea non-null; channel m % snk_period, ea = exp(alpha),
    // eb = exp(-beta)) into y2 (f32, row stride ld_y) or yp (bf16 split
    // planes, rows of 3 ld_y: period group g of a row at 3 g snk_period holds
    // hi | hi | lo of its channels), else in place of y
    const float *snk_ea, *snk_eb;
    int snk_period;
    float *y2;
    uint16_t *yp;
    // filled by the launchers
    int tiles_m, tiles_n, block_begin;
    int kt_split;                  // 32-wide k tiles per split (launch_gemm_ks)
};
struct GemmGroup {
    GemmProblem p[2];
    int nprob;
};
hipError_t launch_gemm_group(GemmGroup &g, int flags, int epi, hipStream_t s);
// The DiT block projections (gemm_ks.hip): bf16 activations, MFMA-tiled
// weights (w_tiled) or row-major ones (ld_w % 8 == 0, 16-byte aligned),
// M % 16 == 0, K % 32 == 0. cfg picks the tile shape: 0 / 30 64 x 64, 22
// 64 x 64 of 32-wide stages, 28 / 29 128 x 64 (3 / 2 stages).
hipError_t launch_gemm_ks(GemmGroup &g, int epi, int cfg, hipStream_t s);
int gemm_ks_tiles(const GemmGroup &g, int bm, int bn);
// output rows per tile (BM) of a launch_gemm_ks configuration
int gemm_ks_bm(int cfg);
// Cooperative-tile GEMM of gemm_ks.hip over row-major (or tiled) bf16 weights
// and bf16 activation rows, optionally an implicit im2col (conv_ic % 32 == 0)
// and the SwiGLU epilogue: EPI_STORE_F32 / _BF16, EPI_SWIGLU_F32 / _BF16.
// M % 16 == 0, K % 32 == 0, 16-byte aligned rows.
hipError_t launch_gemm_coop(GemmGroup &g, int epi, hipStream_t s);
// RoPE (cos, sin) table for positions 0 .. npos-1 and n_dims / 2 pairs, the
// angle freq_scale * p * theta_scale^i evaluated as rope_theta() does:
// cs[p * n_dims + 2 i] = cos, [.. + 1] = sin
hipError_t launch_rope_table(float *cs, int npos, int n_dims, float theta_scale, float freq_scale, hipStream_t s);

// MFMA-tiled weight layout: W[m][k] (M % 16 == 0, K % 32 == 0) is stored as
// 16 x 32 tiles, tile (m / 16, k / 32) at element (m / 16 * (K / 32) + k / 32) * 512,
// inside it lane l = m % 16 + 16 * (k % 32 / 8) holds k % 8 = 0..7 at l * 8 + k % 8.
// One wave's A operand of a 16x16x32 MFMA is then 1 KiB of consecutive bytes.
inline int64_t tiled_index(int64_t m, int64_t k, int64_t K) {
    return ((m / 16) * (K / 32) + k / 32) * 512 + ((m % 16) + 16 * ((k % 32) / 8)) * 8 + (k % 8);
}
hipError_t launch_gemm_q8(const GemmParams &p, hipStream_t s);
// the same for two problems (a joint block's streams), in one launch when they
// share the cooperative tile configuration (same epilogue, output type, splits)
hipError_t launch_gemm_q8_pair(const GemmParams &p0, const GemmParams &p1, hipStream_t s);
// Activation quantization to planes for launch_gemm_q8 (ggml-cpu x86 rounding).
// x rows of K (f32 or bf16, row stride ld_x elements); grp > 0 gathers output
// row n from source row (n / grp) * gstride + n % grp (gstride in ROWS of
// ld_x, unlike the element strides of GemmProblem::x_group_stride).
hipError_t launch_quantize_rows_q8(const void *x, int x_f32, int64_t ld_x, int N, int K,
                                   int8_t *qx, float *dx, hipStream_t s, int grp = 0, int64_t gstride = 0);
// f32 rows of two streams quantized in one launch (each as launch_quantize_rows_q8)
struct QuantRows {
    const float *x;
    int64_t ld_x;
    int N, K;
    int8_t *qx;
    float *dx;
    int grp;
    int64_t gstride;
};
hipError_t launch_quantize_rows_q8_pair(const QuantRows &r0, const QuantRows &r1, hipStream_t s);
// the QKV epilogue over f32 rows (QkvScatter, above)
hipError_t launch_qkv_scatter(const QkvScatter &p, hipStream_t s);
// two streams' scatters in one launch
hipError_t launch_qkv_scatter2(const QkvScatter &p0, const QkvScatter &p1, hipStream_t s);

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
// Q8_0 planes (qx int8 [rows][K], dx f32 [rows][K/32] of fp16 values) ->
// ggml blocks with row stride ld_blocks bytes (bit-preserving)
hipError_t launch_q8_planes_to_blocks(const int8_t *qx, const float *dx, int64_t rows, int64_t K, void *blocks,
                                     int64_t ld_blocks, hipStream_t s);
hipError_t launch_q8_repack(const void *src, int64_t ld_src, int64_t rows, int64_t K,
                            void *dst, hipStream_t s);
hipError_t launch_f32_to_bf16(const float *x, uint16_t *y, int64_t n, hipStream_t s);

// ---------------------------------------------------------------- DiT glue
// Residual update + LayerNorm + modulate for up to two streams in one launch.
// Row r of a stream (b = r / rows_per_b):
//   if part: x[r] += gate[b * ld_gate] * (sum_{s < nsplit} part[s * part_stride + r * H] + bias)
//   y[r] = LN(x[r], eps) * (1 + scale[b]) + shift[b]   (bf16, f32, or Q8_0 planes: y_mode)
enum LnOut : int { LN_Y_BF16 = 0, LN_Y_F32 = 1, LN_Y_Q8 = 2 };
struct LnStream {
    float *x;                     // f32 rows of H (in/out), row stride ld_x
    int64_t ld_x;
    const float *part;            // split-K partial sums [nsplit][rows][H], or null
    int nsplit;
    int64_t part_stride;          // elements between split slices
    const float *bias;            // [H] added to the partial sum, nullable
    const float *gate;            // [B][ld_gate]
    int64_t ld_gate;
    const float *shift, *scale;   // [B][ld_mod]
    int64_t ld_mod;
    void *y;                      // output rows, row stride ld_y (LN_Y_Q8: int8 planes)
    int64_t ld_y;
    float *yd;                    // LN_Y_Q8: f32 block scales [rows][H / 32]
    int rows, rows_per_b;
};
// Weights of a block GEMM that follows, fetched early into the L2 of the XCD
// that the GEMM will run each weight tile on: with (tiles_m * splits) % 8 ==
// 0, launch_gemm_ks deals the (m tile, split) pairs c = tm * splits + split to
// XCD c % 8 (workgroup L runs on XCD L % 8). One dword per 128-byte line.
struct L2Prefetch {
    const uint16_t *w;            // MFMA-tiled bf16 weights: row block rb, k tile kt at (rb * kt_n + kt) * 512
    int kt_n;                     // K / 32
    int rb_tile;                  // 16-row blocks per m tile of the GEMM
    int rb_n;                     // M / 16
    int tiles_m, splits;
};
constexpr int L2PF_MAX = 4;
struct L2PrefetchList {
    L2Prefetch pf[L2PF_MAX];
    int npf;
};
struct LnGroup {
    LnStream s[2];
    int nstream, H, y_mode;       // LnOut
    float eps;
};
// pf (nullable, npf > 0): weights the LN workgroups touch into L2 while they run
hipError_t launch_ln_group(const LnGroup &g, hipStream_t s, const L2PrefetchList *pf = nullptr);
// y = x / sqrt(mean(x^2) + eps) * w on F32 rows of n in {1024, 2048, 4096}
// (16-byte aligned), quantized to Q8_0 planes qx [rows][n] / dx [rows][n/32]
// as launch_quantize_rows_q8 does: the two launches' bits in one
hipError_t launch_rms_norm_q8(const float *x, int64_t ldx, const float *w, float eps, int8_t *qx, float *dx,
                              int64_t rows, int n, hipStream_t s);
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
// ggml_im2col 1-D: dst row (n * OW + ow), column ic * KW + kw; dst_type an
// Elt value (F32 / F16 / BF16); x element strides sp (position), sc
// (channel), sn (batch)
hipError_t launch_im2col_1d(const float *x, int64_t sp, int64_t sc, int64_t sn, int IW, int IC, int KW, int OW, int N,
                           int s0, int p0, int d0, void *dst, int dst_type, int64_t ld, hipStream_t s);
// f32 rows -> contiguous bf16 rows (RNE): row b * rows_per_b + i read at
// x + b * ld_b + i * ld_x (element strides, multiples of 4; cols % 4 == 0)
hipError_t launch_cast_rows_bf16(const float *x, int64_t ld_x, int64_t ld_b, int rows_per_b, int64_t rows, int cols,
                                 uint16_t *y, hipStream_t s);
// f32 rows as [hi | hi | lo] bf16 planes, 3 cols per row (split products of F32 weights)
hipError_t launch_cast_rows_split3(const float *x, int64_t ld_x, int64_t ld_b, int rows_per_b, int64_t rows, int cols,
                                   uint16_t *y, hipStream_t s);
// conv kernel [KW, IC, OC] of es-byte elements (element strides s0..s2) ->
// kw-major rows dst[oc][kw * IC + ic]
hipError_t launch_conv_pack(const void *w, int es, int64_t s0, int64_t s1, int64_t s2, int KW, int IC, int OC, void *dst,
                            hipStream_t s);
// SnakeBeta v + sin^2(v ea[c]) eb[c] (src/vae_decoder.cpp:14-24, in the
// reference's node order mul, sin, sqr, mul, add) applied to an f32 GEMM's
// output: c = m % period (period a multiple of 4 dividing M), ea = exp(alpha),
// eb = exp(-beta); written in place of the output (y2 null), or next to it
// into y2 (same row stride; the output itself then stays plain)
struct F32Snake {
    const float *ea, *eb;
    float *y2;
    int period;
};
// F32-weight GEMM (gemm_f32.hip): p.wf [M][K] (ld_w), f32 activations p.x
// (plain rows or implicit im2col), y f32 or bf16 (+bias), optionally followed
// by a SnakeBeta (f32 y only)
hipError_t launch_gemm_f32(const GemmProblem &p, int y_bf16, hipStream_t s, const F32Snake *snake = nullptr);
// y = silu(a) * b, f32, n elements
hipError_t launch_silu_mul(const float *a, const float *b, float *y, int64_t n, hipStream_t s);
// y[n][m] = sum of S K-split slices p[z][n][m] (rows of M, slices `stride` apart, summed in order)
// + bias[m] (nullable), into rows of ld_y; M, ld_y, stride multiples of 4, 16-byte aligned
hipError_t launch_sum_slices(const float *p, int S, int64_t stride, const float *bias, int64_t N, int M, float *y,
                             int64_t ld_y, hipStream_t s);
// the same with a and b each the sum of S K-split slices (stride elements apart, summed in order)
hipError_t launch_silu_mul_slices(const float *a, const float *b, int S, int64_t stride, float *y, int64_t n,
                                  hipStream_t s);
// y[n, m] = sum_k W[m, k] x[n, k] + bias[m]: bf16 row-major W, f32 x and y,
// fp32 fma accumulation (the DiT's input and output projections)
hipError_t launch_proj_f32(const uint16_t *w, const float *bias, const float *x, int64_t ld_x, int N, int K, int M,
                           float *y, int64_t ld_y, hipStream_t s);
// the same with x channel-major per batch item, [N / T][K][T] (ne0 = T): the
// latent layout of ts_dit::forward; tmp holds N * K floats (used when K != 64)
hipError_t launch_proj_f32_cm(const uint16_t *w, const float *bias, const float *x, int T, int N, int K, int M,
                              float *y, int64_t ld_y, float *tmp, hipStream_t s);
// t-embedding: temb[b, k] = cos(t_b * freq[k]), temb[b, H/2 + k] = sin(t_b * freq[k])
struct TimeVals { float t[32]; };
hipError_t launch_timestep_embed(const float *freq, const TimeVals &tv, int B, int H, float *temb,
                                 hipStream_t s);
// glue of the reference graph: y = bf16(silu(x)); y = a + b; the mean over
// the S rows of [B][S][H]; extended_c = sync rows at floor((t + 0.5) S / T)
// plus g[b] (nearest-exact interpolation of src/mmdit.cpp:319, :196)
hipError_t launch_silu_bf16(const float *x, uint16_t *y, int64_t n, hipStream_t s);
// [B][C][T] -> [B][T][C] (f32); y[r][c] = x[r][c] + pe[r % period][c]
hipError_t launch_transpose_ct(const float *x, int B, int C, int T, float *y, hipStream_t s);
// stride-1, dilation-1 convolution of channels-fastest rows x [T][IC] into
// planar y[oc][t] (row stride ld_y) with OC <= 2 output channels: weights
// [OC][KW][IC], zero padding `pad`, optional bias. IC = 128, KW = 7, OC = 2
// (the VAE's final convolution); other shapes: hipErrorInvalidValue
hipError_t launch_conv_small_oc(const float *x, int T, int IC, int KW, int OC, const float *w, const float *bias,
                                 int pad, float *y, int64_t ld_y, hipStream_t s);
hipError_t launch_add_period_rows(const float *x, int64_t rows, int cols, const float *pe, int period, float *y,
                                  hipStream_t s);
hipError_t launch_add_f32(const float *a, const float *b, float *y, int64_t n, hipStream_t s);
hipError_t launch_row_mean(const float *x, int B, int S, int H, float *y, hipStream_t s);
hipError_t launch_sync_extend(const float *sync, int B, int S, int T, int H, const float *g, float *y, hipStream_t s);
// CFG combine + Euler step: x[i] += dt * (fu + (fc - fu) * cfg); flow0 optional
hipError_t launch_cfg_euler(const float *flow2, int64_t n, float cfg, float dt, float *x,
                            float *x2, float *flow0, hipStream_t s);

}  // namespace tsk
