// ops.hip — memory-bound kernels of the MM-DiT path for gfx950:
//   rms_norm*w (src/mmdit.cpp:78-80), layer norm (:59), rope NORMAL (:96-99),
//   the fused QK-RMSNorm+RoPE prologue (:221-223), Q8_0 (de)quantisation and
//   repacking, and the DiT driver's glue (LN+modulate, QKV split, adaLN GEMV,
//   CFG/Euler update).
// One wave (64 lanes) or one 256-thread block per row; rows are streamed once.
#include <cstdlib>

#include "qkv_row.h"
#include "tsk_common.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

namespace tsk {

namespace {

__device__ __forceinline__ float vload(const View4 &v, const char *row, int64_t i) {
    return v.type == TSK_TYPE_F32 ? ((const float *) row)[i] : bf16_bits_to_f32(((const uint16_t *) row)[i]);
}
__device__ __forceinline__ void vstore(const View4 &v, char *row, int64_t i, float x) {
    if (v.type == TSK_TYPE_F32) ((float *) row)[i] = x;
    else ((uint16_t *) row)[i] = f32_to_bf16_bits(x);
}
__device__ __forceinline__ const char *vrow(const View4 &v, int64_t r) {
    const int64_t i1 = r % v.ne[1], i2 = (r / v.ne[1]) % v.ne[2], i3 = r / (v.ne[1] * v.ne[2]);
    return (const char *) v.data + i1 * v.nb[1] + i2 * v.nb[2] + i3 * v.nb[3];
}

// ---------------------------------------------------------------- rms_norm * w
__global__ void rms_norm_mul_kernel(const View4 x, const float *w, float eps, const View4 y, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const char *xr = vrow(x, r);
    char *yr = (char *) vrow(y, r);
    const int64_t n = x.ne[0];
    float ss = 0.0f;
    for (int64_t i = lane; i < n; i += 64) { const float v = vload(x, xr, i); ss += v * v; }
    ss = wave_sum(ss);
    const float mean = ss / (float) n;
    const float sc = 1.0f / sqrtf(mean + eps);
    for (int64_t i = lane; i < n; i += 64) {
        float v = vload(x, xr, i) * sc;
        if (w) v = v * w[i];
        vstore(y, yr, i, v);
    }
}

// ---------------------------------------------------------------- layer norm (no affine)
__global__ void norm_kernel(const View4 x, float eps, const View4 y, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const char *xr = vrow(x, r);
    char *yr = (char *) vrow(y, r);
    const int64_t n = x.ne[0];
    float s = 0.0f;
    for (int64_t i = lane; i < n; i += 64) s += vload(x, xr, i);
    const float mean = wave_sum(s) / (float) n;
    float s2 = 0.0f;
    for (int64_t i = lane; i < n; i += 64) { const float v = vload(x, xr, i) - mean; s2 += v * v; }
    const float var = wave_sum(s2) / (float) n;
    const float sc = 1.0f / sqrtf(var + eps);
    for (int64_t i = lane; i < n; i += 64) vstore(y, yr, i, (vload(x, xr, i) - mean) * sc);
}

// ---------------------------------------------------------------- rows held in registers
// F32 rows of n = 256 NV contiguous floats, 16-byte aligned: one wave per row
// loads the whole row (and w) before its reductions and stores after them, so
// no load waits behind a store of the same wave. RMS: y = x / sqrt(mean(x^2) +
// eps) * w; NORM: y = (x - mean) / sqrt(mean((x - mean)^2) + eps).
template <bool RMS, int NV>
__global__ __launch_bounds__(256) void norm_rows_kernel(const float *x, int64_t ldx, const float *w, float eps,
                                                        float *y, int64_t ldy, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    constexpr int n = 256 * NV;
    const float *xr = x + r * ldx;
    f32x4 v[NV], wv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        v[j] = *(const f32x4 *) (xr + (lane + 64 * j) * 4);
        wv[j] = RMS && w ? *(const f32x4 *) (w + (lane + 64 * j) * 4) : f32x4{1, 1, 1, 1};
    }
    float mean = 0.0f;
    if constexpr (!RMS) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) s += v[j][0] + v[j][1] + v[j][2] + v[j][3];
        mean = wave_sum(s) / (float) n;
    }
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        for (int e = 0; e < 4; ++e) { const float d = v[j][e] - mean; s2 += d * d; }
    const float sc = 1.0f / sqrtf(wave_sum(s2) / (float) n + eps);
    float *yr = y + r * ldy;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        f32x4 o;
        for (int e = 0; e < 4; ++e) o[e] = RMS && w ? v[j][e] * sc * wv[j][e] : (v[j][e] - mean) * sc;
        *(f32x4 *) (yr + (lane + 64 * j) * 4) = o;
    }
}

// rows of x and y uniformly strided F32 with n = 256 NV, NV in {1, 2, 4, 8, 16}
bool rows_fit(const View4 &x, const View4 &y, int64_t *ldx, int64_t *ldy) {
    const int64_t n = x.ne[0];
    if (x.type != TSK_TYPE_F32 || y.type != TSK_TYPE_F32 || n % 256 || n > 4096 || (n / 256) & (n / 256 - 1))
        return false;
    for (const View4 *v : {&x, &y}) {
        if (v->nb[0] != 4 || v->nb[1] % 16 || ((uintptr_t) v->data & 15) || v->nb[2] != v->ne[1] * v->nb[1] ||
            v->nb[3] != v->ne[2] * v->nb[2])
            return false;
    }
    for (int d = 0; d < 4; ++d)
        if (x.ne[d] != y.ne[d]) return false;
    *ldx = x.nb[1] / 4;
    *ldy = y.nb[1] / 4;
    return true;
}

template <bool RMS>
void launch_norm_rows(const float *x, int64_t ldx, const float *w, float eps, float *y, int64_t ldy, int64_t rows,
                      int n, hipStream_t s) {
    const dim3 grid((unsigned) ((rows + 3) / 4)), blk(256);
    switch (n / 256) {
        case 1: launch_kernel(norm_rows_kernel<RMS, 1>, grid, blk, 0, s, x, ldx, w, eps, y, ldy, rows); break;
        case 2: launch_kernel(norm_rows_kernel<RMS, 2>, grid, blk, 0, s, x, ldx, w, eps, y, ldy, rows); break;
        case 4: launch_kernel(norm_rows_kernel<RMS, 4>, grid, blk, 0, s, x, ldx, w, eps, y, ldy, rows); break;
        case 8: launch_kernel(norm_rows_kernel<RMS, 8>, grid, blk, 0, s, x, ldx, w, eps, y, ldy, rows); break;
        default: launch_kernel(norm_rows_kernel<RMS, 16>, grid, blk, 0, s, x, ldx, w, eps, y, ldy, rows); break;
    }
}

// ---------------------------------------------------------------- rope NORMAL
// x ne = [ne0, n_head, S, B]; pos[i2]. One wave per (i1, i2, i3) row.
__global__ void rope_kernel(const View4 x, const int32_t *pos, int n_dims, float theta_scale,
                            float freq_scale, const View4 y, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int64_t i2 = (r / x.ne[1]) % x.ne[2];
    const char *xr = vrow(x, r);
    char *yr = (char *) vrow(y, r);
    const float p = (float) pos[i2];
    for (int i = lane; 2 * i < n_dims; i += 64) {
        const float th = freq_scale * rope_theta(p, theta_scale, i);
        const float c = cosf(th), sn = sinf(th);
        const float x0 = vload(x, xr, 2 * i), x1 = vload(x, xr, 2 * i + 1);
        vstore(y, yr, 2 * i, x0 * c - x1 * sn);
        vstore(y, yr, 2 * i + 1, x0 * sn + x1 * c);
    }
    for (int64_t i = n_dims + lane; i < x.ne[0]; i += 64) vstore(y, yr, i, vload(x, xr, i));
}

__global__ void rope_table_kernel(float *cs, int npos, int n_dims, float theta_scale, float freq_scale) {
    const int half = n_dims / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npos * half) return;
    const int p = i / half, pr = i % half;
    const float th = freq_scale * rope_theta((float) p, theta_scale, pr);
    cs[(int64_t) p * n_dims + 2 * pr] = cosf(th);
    cs[(int64_t) p * n_dims + 2 * pr + 1] = sinf(th);
}

// ---------------------------------------------------------------- fused qk norm + rope
// x ne = [64, n_head, S, B]; 32 lanes per head vector (one pair each).
__global__ void qk_norm_rope_kernel(const View4 x, const float *w, const int32_t *pos, float eps,
                                    int n_dims, float theta_scale, float freq_scale, const View4 y,
                                    int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * (blockDim.x / 32) + threadIdx.x / 32;
    const int i = threadIdx.x & 31;
    if (r >= rows) return;
    const char *xr = vrow(x, r);
    char *yr = (char *) vrow(y, r);
    float x0 = vload(x, xr, 2 * i), x1 = vload(x, xr, 2 * i + 1);
    const float ss = row_pair_sum(row16_sum(x0 * x0 + x1 * x1));   // 32 lanes of one 32-lane half
    const float sc = 1.0f / sqrtf(ss / 64.0f + eps);
    x0 = x0 * sc * w[2 * i];
    x1 = x1 * sc * w[2 * i + 1];
    if (pos && 2 * i < n_dims) {
        const int64_t i2 = (r / x.ne[1]) % x.ne[2];
        const float th = freq_scale * rope_theta((float) pos[i2], theta_scale, i);
        const float c = cosf(th), sn = sinf(th);
        const float y0 = x0 * c - x1 * sn, y1 = x0 * sn + x1 * c;
        x0 = y0; x1 = y1;
    }
    vstore(y, yr, 2 * i, x0);
    vstore(y, yr, 2 * i + 1, x1);
}

// ---------------------------------------------------------------- Q8_0 blocks
struct __attribute__((packed)) BlockQ8 { uint16_t d; int8_t qs[32]; };

__global__ void q8_quantize_blocks_kernel(const float *x, int64_t ld_x, int64_t rows, int64_t K,
                                          char *blocks, int64_t ld_blocks) {
    const int64_t KB = K / 32;
    const int64_t blk = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= rows * KB) return;
    const int64_t row = blk / KB, kb = blk % KB;
    const float *xr = x + row * ld_x + kb * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xr[j]));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    BlockQ8 *o = (BlockQ8 *) (blocks + row * ld_blocks) + kb;
    o->d = f32_to_f16_bits(d);
    for (int j = 0; j < 32; ++j) o->qs[j] = (int8_t) __builtin_rintf(xr[j] * id);
}

// Q8_0 planes (int8 [rows][K], f32 scales [rows][K/32] holding fp16 values)
// -> ggml blocks {fp16 d; int8 qs[32]}: one thread per block, bit-preserving
__global__ void q8_planes_to_blocks_kernel(const int8_t *qx, const float *dx, int64_t rows, int64_t K,
                                           char *blocks, int64_t ld_blocks) {
    const int64_t KB = K / 32;
    const int64_t blk = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= rows * KB) return;
    const int64_t row = blk / KB, kb = blk % KB;
    BlockQ8 *o = (BlockQ8 *) (blocks + row * ld_blocks) + kb;
    o->d = f32_to_f16_bits(dx[blk]);
    const int8_t *q = qx + row * K + kb * 32;
    for (int j = 0; j < 32; ++j) o->qs[j] = q[j];
}

__global__ void q8_dequantize_kernel(const char *src, int split, int64_t rows, int64_t K, int64_t ld_src,
                                     float *y, int64_t ld_y) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * K) return;
    const int64_t row = i / K, k = i % K;
    float d;
    int q;
    if (split) {
        const int8_t *qs = (const int8_t *) src;
        const uint16_t *ds = (const uint16_t *) (src + rows * K);
        q = qs[row * K + k];
        d = f16_bits_to_f32(ds[row * (K / 32) + k / 32]);
    } else {
        const BlockQ8 *b = (const BlockQ8 *) (src + row * ld_src) + k / 32;
        q = b->qs[k % 32];
        d = f16_bits_to_f32(b->d);
    }
    y[row * ld_y + k] = d * (float) q;
}

__global__ void q8_repack_kernel(const char *src, int64_t ld_src, int64_t rows, int64_t K, char *dst) {
    const int64_t KB = K / 32;
    const int64_t blk = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= rows * KB) return;
    const int64_t row = blk / KB, kb = blk % KB;
    const BlockQ8 *b = (const BlockQ8 *) (src + row * ld_src) + kb;
    int8_t *qs = (int8_t *) dst + row * K + kb * 32;
    for (int j = 0; j < 32; ++j) qs[j] = b->qs[j];
    uint16_t *ds = (uint16_t *) (dst + rows * K);
    ds[row * KB + kb] = b->d;
}

__global__ void f32_to_bf16_kernel(const float *x, uint16_t *y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = f32_to_bf16_bits(x[i]);
}

// ---------------------------------------------------------------- DiT glue
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < (int) (blockDim.x >> 6); ++i) t += red[i];
    return t;
}

// acc[j] += slices p[0], p[stride], ..., p[(C - 1) stride] at the lane's
// offsets (lane + 64 j) * 4, in slice order; every load is issued before the
// first add, so a run of C slices costs one memory round trip
template <int NV, int C>
__device__ __forceinline__ void add_slice_run(f32x4 (&acc)[NV], const float *p, int64_t stride, int lane) {
    f32x4 t[C][NV];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int j = 0; j < NV; ++j) t[c][j] = *(const f32x4 *) (p + c * stride + (lane + 64 * j) * 4);
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[j][e] += t[c][j][e];
}

// acc[j] += slices 1 .. nsplit - 1 of p (slice stride `stride`), in order, in
// runs of up to three slices
template <int NV>
__device__ __forceinline__ void add_slices(f32x4 (&acc)[NV], const float *p, int64_t stride, int nsplit, int lane) {
    for (int sp = 1; sp < nsplit; sp += 3) {
        const int n = nsplit - sp;
        if (n >= 3) add_slice_run<NV, 3>(acc, p + sp * stride, stride, lane);
        else if (n == 2) add_slice_run<NV, 2>(acc, p + sp * stride, stride, lane);
        else add_slice_run<NV, 1>(acc, p + sp * stride, stride, lane);
    }
}

// Residual update + LayerNorm + adaLN modulate, one 256-thread block per row
// of up to two streams (mmdit.cpp:196-231: x = x + gate * y, then
// modulate(LN(x), shift, scale) for the next projection):
//   pending: x += gate[b] * (sum_s part[s][r] + bias)   (splits summed in order)
//   y = LN(x, eps) * (1 + scale[b]) + shift[b]           (bf16, or f32)
// A row of H <= 4096 floats stays in registers (4 per thread per 1024).
// One row of stream `st` (the kernel argument g.s[0] or g.s[1] by name, so
// every field is read at a fixed kernel-argument offset).
template <bool YF32>
__device__ __forceinline__ void ln_group_row(const LnStream &st, int r, int H, float eps) {
    __shared__ float red[4];
    const int b = r / st.rows_per_b;
    float *xr = st.x + (int64_t) r * st.ld_x;
    constexpr int VMAX = 4;
    f32x4 v[VMAX];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VMAX; ++j) {
        const int i = (threadIdx.x + 256 * j) * 4;
        if (i >= H) break;
        v[j] = *(const f32x4 *) (xr + i);
        if (st.part) {
            const float *pp = st.part + (int64_t) r * H + i;
            f32x4 acc[1] = {*(const f32x4 *) pp};
            add_slices<1>(acc, pp, st.part_stride, st.nsplit, 0);
            const f32x4 bv = st.bias ? *(const f32x4 *) (st.bias + i) : f32x4{0, 0, 0, 0};
            const f32x4 gv = *(const f32x4 *) (st.gate + (int64_t) b * st.ld_gate + i);
            for (int e = 0; e < 4; ++e) v[j][e] += gv[e] * (acc[0][e] + bv[e]);
            *(f32x4 *) (xr + i) = v[j];
        }
        s += v[j][0] + v[j][1] + v[j][2] + v[j][3];
    }
    const float mean = block_sum_256(s, red) / (float) H;
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < VMAX; ++j) {
        const int i = (threadIdx.x + 256 * j) * 4;
        if (i >= H) break;
        for (int e = 0; e < 4; ++e) { const float d = v[j][e] - mean; s2 += d * d; }
    }
    const float var = block_sum_256(s2, red) / (float) H;
    const float rs = 1.0f / sqrtf(var + eps);
    const float *sh = st.shift + (int64_t) b * st.ld_mod, *sc = st.scale + (int64_t) b * st.ld_mod;
#pragma unroll
    for (int j = 0; j < VMAX; ++j) {
        const int i = (threadIdx.x + 256 * j) * 4;
        if (i >= H) break;
        const f32x4 shv = *(const f32x4 *) (sh + i), scv = *(const f32x4 *) (sc + i);
        float o[4];
        for (int e = 0; e < 4; ++e) o[e] = (v[j][e] - mean) * rs * (scv[e] + 1.0f) + shv[e];
        if constexpr (YF32) {
            *(f32x4 *) ((float *) st.y + (int64_t) r * st.ld_y + i) = f32x4{o[0], o[1], o[2], o[3]};
        } else {
            uint16_t ob[4];
            for (int e = 0; e < 4; ++e) ob[e] = f32_to_bf16_bits(o[e]);
            u32x2 w;
            __builtin_memcpy(&w, ob, 8);
            *(u32x2 *) ((uint16_t *) st.y + (int64_t) r * st.ld_y + i) = w;
        }
    }
}

template <bool YF32>
__global__ __launch_bounds__(256) void ln_group_kernel(const LnGroup g) {
    const int r = blockIdx.x;
    if (g.nstream > 1 && r >= g.s[0].rows) ln_group_row<YF32>(g.s[1], r - g.s[0].rows, g.H, g.eps);
    else ln_group_row<YF32>(g.s[0], r, g.H, g.eps);
}

// The same row update with one wave per row and H = 256 NV: every load of the
// row (residual, split slices, bias, gate, shift, scale) is issued before the
// first reduction, and both reductions stay inside the wave (no LDS, no
// barrier).
// YM: LN_Y_BF16 / LN_Y_F32 rows, or LN_Y_Q8 -- the row quantized to Q8_0
// planes (int8 st.y [rows][H], f32 scales st.yd [rows][H / 32]) as
// quantize_rows_q8_kernel quantizes an f32 row: the 32-element block of
// element (lane + 64 j) * 4 + e is held by lanes 8 (b % 8) .. + 7 at register
// j, so its amax is three DPP steps (the conversion ggml_mul_mat applies to
// src1 for a Q8_0 weight).
template <int YM, int NV>
__device__ __forceinline__ void ln_wave_row(const LnStream &st, int r, float eps) {
    constexpr int H = 256 * NV;
    const int lane = threadIdx.x, b = r / st.rows_per_b;
    float *xr = st.x + (int64_t) r * st.ld_x;
    const float *sh = st.shift + (int64_t) b * st.ld_mod, *sc = st.scale + (int64_t) b * st.ld_mod;
    f32x4 v[NV], shv[NV], scv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = (lane + 64 * j) * 4;
        v[j] = *(const f32x4 *) (xr + i);
        shv[j] = *(const f32x4 *) (sh + i);
        scv[j] = *(const f32x4 *) (sc + i);
    }
    if (st.part) {
        f32x4 acc[NV], gv[NV], bv[NV];
        const float *gr = st.gate + (int64_t) b * st.ld_gate;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int i = (lane + 64 * j) * 4;
            acc[j] = *(const f32x4 *) (st.part + (int64_t) r * H + i);
            gv[j] = *(const f32x4 *) (gr + i);
            bv[j] = st.bias ? *(const f32x4 *) (st.bias + i) : f32x4{0, 0, 0, 0};
        }
        add_slices<NV>(acc, st.part + (int64_t) r * H, st.part_stride, st.nsplit, lane);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            for (int e = 0; e < 4; ++e) v[j][e] += gv[j][e] * (acc[j][e] + bv[j][e]);
            *(f32x4 *) (xr + (lane + 64 * j) * 4) = v[j];
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) s += v[j][0] + v[j][1] + v[j][2] + v[j][3];
    const float mean = wave_sum(s) / (float) H;
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        for (int e = 0; e < 4; ++e) { const float d = v[j][e] - mean; s2 += d * d; }
    const float rs = 1.0f / sqrtf(wave_sum(s2) / (float) H + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = (lane + 64 * j) * 4;
        float o[4];
        for (int e = 0; e < 4; ++e) o[e] = (v[j][e] - mean) * rs * (scv[j][e] + 1.0f) + shv[j][e];
        if constexpr (YM == LN_Y_Q8) {
            float amax = 0.0f;
            for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(o[e]));
#pragma unroll
            for (int k = 0; k < 3; ++k) amax = fmaxf(amax, dpp_f(amax, k));   // the 8 lanes of the block
            const float d = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            if ((lane & 7) == 0) st.yd[(int64_t) r * (H / 32) + 8 * j + (lane >> 3)] = f16_bits_to_f32(f32_to_f16_bits(d));
            int8_t q[4];
            for (int e = 0; e < 4; ++e) q[e] = (int8_t) __builtin_rintf(o[e] * id);
            uint32_t w4;
            __builtin_memcpy(&w4, q, 4);
            *(uint32_t *) ((int8_t *) st.y + (int64_t) r * st.ld_y + i) = w4;
        } else if constexpr (YM == LN_Y_F32) {
            *(f32x4 *) ((float *) st.y + (int64_t) r * st.ld_y + i) = f32x4{o[0], o[1], o[2], o[3]};
        } else {
            uint16_t ob[4];
            for (int e = 0; e < 4; ++e) ob[e] = f32_to_bf16_bits(o[e]);
            u32x2 w;
            __builtin_memcpy(&w, ob, 8);
            *(u32x2 *) ((uint16_t *) st.y + (int64_t) r * st.ld_y + i) = w;
        }
    }
}

// The workgroups on XCD x (blockIdx.x % 8 == x) touch one dword of every
// 128-byte line of the weight tiles the following GEMM runs on XCD x, so its
// first stages find them in that XCD's L2 instead of waiting on memory. The
// touches are loads into a 256-byte LDS slot that is never read; the caller
// waits for them (vmcnt) before the workgroup ends.
__device__ __forceinline__ void l2_prefetch(const L2Prefetch *pf, int npf, void *sink) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int xcd = (int) (blockIdx.x & 7), wg = (int) (blockIdx.x >> 3);
    const int nwg = (int) ((gridDim.x + 7 - xcd) >> 3);      // workgroups on this XCD
    const int lane = threadIdx.x & 63;
    for (int i = 0; i < npf; ++i) {
        const L2Prefetch &f = pf[i];
        const int kts = f.kt_n / f.splits;                     // k tiles (1 KiB each) per slice
        const int per_rb = kts * 8, per_pair = f.rb_tile * per_rb;
        const int total = (f.tiles_m * f.splits >> 3) * per_pair;
        for (int l = wg * 64 + lane; l < total; l += nwg * 64) {
            const int pi = l / per_pair, rem = l - pi * per_pair;
            const int c = xcd + 8 * pi, tm = c / f.splits, sp = c - tm * f.splits;
            const int rbl = rem / per_rb, ln = rem - rbl * per_rb;
            const int rb = tm * f.rb_tile + rbl;
            if (rb < f.rb_n)
                __builtin_amdgcn_global_load_lds(f.w + ((int64_t) rb * f.kt_n + sp * kts) * 512 + ln * 64,
                                                 (lds_void *) sink, 4, 0, 0);
        }
    }
}

template <int YM, int NV>
__global__ __launch_bounds__(64) void ln_wave_kernel(const LnGroup g) {
    const int r = blockIdx.x;
    if (g.nstream > 1 && r >= g.s[0].rows) ln_wave_row<YM, NV>(g.s[1], r - g.s[0].rows, g.eps);
    else ln_wave_row<YM, NV>(g.s[0], r, g.eps);
}

// the same rows, the workgroups also touching the next GEMMs' weights into L2
template <int YM, int NV>
__global__ __launch_bounds__(64) void ln_wave_pf_kernel(const LnGroup g, const L2PrefetchList pf) {
    __shared__ __attribute__((aligned(16))) uint32_t sink[64];
    const int r = blockIdx.x;
    l2_prefetch(pf.pf, pf.npf, sink);
    if (g.nstream > 1 && r >= g.s[0].rows) ln_wave_row<YM, NV>(g.s[1], r - g.s[0].rows, g.eps);
    else ln_wave_row<YM, NV>(g.s[0], r, g.eps);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// GEMV list: one wave per output row; lane k-slices of 8, f32 activations
template <int MAXB, int RW>
__global__ __launch_bounds__(256) void gemv_jobs_kernel(const GemvJob *jobs, int B, int K) {
    // RW rows per wave: their weight loads are issued together and each
    // activation slice is loaded once for all of them; every row is summed
    // in the same order whatever RW (lane partials over k, then the wave sum)
    const GemvJob jb = jobs[blockIdx.y];
    const int j0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RW;
    const int lane = threadIdx.x & 63;
    if (j0 >= jb.M) return;
    float acc[RW][MAXB];
    for (int r = 0; r < RW; ++r)
        for (int b = 0; b < MAXB; ++b) acc[r][b] = 0.0f;
    for (int k = lane * 8; k < K; k += 512) {
        u32x4 raw[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r)
            raw[r] = j0 + r < jb.M ? *(const u32x4 *) (jb.w + (int64_t) (j0 + r) * K + k) : u32x4{0, 0, 0, 0};
        for (int b = 0; b < MAXB; ++b) {
            if (b >= B) break;
            const float *cr = jb.x + (int64_t) b * K + k;
            const f32x4 c0 = *(const f32x4 *) cr, c1 = *(const f32x4 *) (cr + 4);
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const uint16_t *h = (const uint16_t *) &raw[r];
                float wv[8];
                for (int e = 0; e < 8; ++e) wv[e] = bf16_bits_to_f32(h[e]);
                acc[r][b] += wv[0] * c0[0] + wv[1] * c0[1] + wv[2] * c0[2] + wv[3] * c0[3] +
                             wv[4] * c1[0] + wv[5] * c1[1] + wv[6] * c1[2] + wv[7] * c1[3];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int j = j0 + r;
        for (int b = 0; b < MAXB; ++b) {
            if (b >= B) break;
            const float s = wave_sum(acc[r][b]);
            if (lane == 0 && j < jb.M) {
                float v = s + (jb.bias ? jb.bias[j] : 0.0f);
                if (jb.silu_out) v = v / (1.0f + __expf(-v));
                jb.out[(int64_t) b * jb.ld_out + j] = v;
            }
        }
    }
}

// Thin f32-accurate projection y[n, m] = sum_k W[m, k] x[n, k] + b[m] with bf16
// W (row-major) and f32 x: one wave per (token, 64 outputs), lane = output.
// Four fp32 accumulators over k mod 4 (fixed order, fma per element: the
// bf16 x f32 products are exact inside the fma), summed in order at the end.
__global__ __launch_bounds__(256) void proj_f32_kernel(const uint16_t *w, const float *bias, const float *x,
                                                       int64_t ld_x, int N, int K, int M, float *y, int64_t ld_y) {
    const int lane = threadIdx.x & 63;
    const int chunks = (M + 63) / 64;
    const int64_t wv = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wv >= (int64_t) N * chunks) return;
    const int n = (int) (wv / chunks), m = (int) (wv % chunks) * 64 + lane;
    const float *xr = x + (int64_t) n * ld_x;
    const uint16_t *wr = w + (int64_t) (m < M ? m : M - 1) * K;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < K; k += 8) {
        const u32x4 w8 = *(const u32x4 *) (wr + k);
        const f32x4 x0 = *(const f32x4 *) (xr + k), x1 = *(const f32x4 *) (xr + k + 4);
        const uint16_t *h = (const uint16_t *) &w8;
        for (int j = 0; j < 4; ++j) a[j] = fmaf(bf16_bits_to_f32(h[j]), x0[j], a[j]);
        for (int j = 0; j < 4; ++j) a[j] = fmaf(bf16_bits_to_f32(h[4 + j]), x1[j], a[j]);
    }
    if (m < M) y[(int64_t) n * ld_y + m] = ((a[0] + a[1]) + (a[2] + a[3])) + (bias ? bias[m] : 0.0f);
}

// Same projection for long K and few outputs (the DiT's final layer, K = 1024,
// M = 64): one 256-thread workgroup per (token, 64 outputs), the token's row
// staged in LDS; wave w owns outputs 16 w .. 16 w + 15 and its lanes split K
// (lane l: k = (K / 64) l .. +K / 64), so all 16 weight-row slices of a lane
// are in flight at once; each output is one fixed-order wave sum.
template <int KPL, int TOK>
__global__ __launch_bounds__(256) void proj_f32_kt_kernel(const uint16_t *w, const float *bias, const float *x,
                                                          int64_t ld_x, int N, int M, float *y, int64_t ld_y) {
    // a workgroup: 64 outputs (16 per wave) of TOK consecutive tokens; lane l
    // holds k slice [l * KPL * 8, +KPL * 8) of its wave's 16 weight rows in
    // registers for all TOK tokens; each output is its lane partials summed in
    // k order, then the wave sum -- the same order for any TOK
    constexpr int K = KPL * 8 * 64;
    __shared__ __attribute__((aligned(16))) float xs[TOK][K];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.x * 64 + wave * 16, n0 = blockIdx.y * TOK;
    for (int i = threadIdx.x * 4; i < TOK * K; i += 256 * 4) {
        const int t = i / K, c = i - t * K;
        const int n = min(n0 + t, N - 1);
        *(f32x4 *) &xs[t][c] = *(const f32x4 *) (x + (int64_t) n * ld_x + c);
    }
    u32x4 wv[16][KPL];
#pragma unroll
    for (int o = 0; o < 16; ++o) {
        const int m = m0 + o < M ? m0 + o : M - 1;
#pragma unroll
        for (int j = 0; j < KPL; ++j) wv[o][j] = *(const u32x4 *) (w + (int64_t) m * K + lane * KPL * 8 + 8 * j);
    }
    __syncthreads();
    for (int t = 0; t < TOK; ++t) {
        const int n = n0 + t;
        if (n >= N) break;
        float xv[KPL * 8];
#pragma unroll
        for (int j = 0; j < KPL * 8; j += 4) {
            const f32x4 v = *(const f32x4 *) &xs[t][lane * KPL * 8 + j];
            xv[j] = v[0]; xv[j + 1] = v[1]; xv[j + 2] = v[2]; xv[j + 3] = v[3];
        }
#pragma unroll
        for (int o = 0; o < 16; ++o) {
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                const uint16_t *h = (const uint16_t *) &wv[o][j];
                for (int e = 0; e < 8; ++e) a = fmaf(bf16_bits_to_f32(h[e]), xv[8 * j + e], a);
            }
            a = wave_sum(a);
            const int m = m0 + o;
            if (lane == 0 && m < M) y[(int64_t) n * ld_y + m] = a + (bias ? bias[m] : 0.0f);
        }
    }
}

// Short-K projection (the 64-channel latent input): lane l holds output
// m0 + l's K weights in registers, a workgroup runs TT tokens whose rows are
// staged in LDS (float4 broadcasts); k is summed as in proj_f32_kernel
// (a[k % 4] in k order, then ((a0 + a1) + (a2 + a3)) + bias).
// cm_T > 0: x is channel-major per batch item, [N / cm_T][K][cm_T] (the
// ne0 = T latent of ts_dit::forward), token n = b * cm_T + t.
template <int K, int TT>
__global__ __launch_bounds__(256) void proj_f32_rows_kernel(const uint16_t *w, const float *bias, const float *x,
                                                            int64_t ld_x, int N, int M, float *y, int64_t ld_y,
                                                            int cm_T) {
    __shared__ __attribute__((aligned(16))) float xs[TT][K];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.x * 64, n0 = blockIdx.y * TT;
    if (cm_T > 0) {
        // consecutive threads read consecutive tokens of one channel
        for (int i = threadIdx.x; i < TT * K; i += 256) {
            const int t = i % TT, c = i / TT;
            const int n = min(n0 + t, N - 1);
            const int b = n / cm_T, tt = n - b * cm_T;
            xs[t][c] = x[((int64_t) b * K + c) * cm_T + tt];
        }
    } else {
        for (int i = threadIdx.x; i < TT * (K / 4); i += 256) {
            const int t = i / (K / 4), c = (i - t * (K / 4)) * 4;
            const int n = min(n0 + t, N - 1);
            *(f32x4 *) &xs[t][c] = *(const f32x4 *) (x + (int64_t) n * ld_x + c);
        }
    }
    const int m = m0 + lane;
    const uint16_t *wr = w + (int64_t) (m < M ? m : M - 1) * K;
    float wv[K];
#pragma unroll
    for (int k = 0; k < K; k += 8) {
        const u32x4 w8 = *(const u32x4 *) (wr + k);
        const uint16_t *h = (const uint16_t *) &w8;
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[k + e] = bf16_bits_to_f32(h[e]);
    }
    const float bv = bias && m < M ? bias[m] : 0.0f;
    __syncthreads();
    for (int t = wave; t < TT; t += 4) {
        const int n = n0 + t;
        if (n >= N) break;
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < K; k += 4) {
            const f32x4 xv = *(const f32x4 *) &xs[t][k];
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] = fmaf(wv[k + e], xv[e], a[e]);
        }
        if (m < M) y[(int64_t) n * ld_y + m] = ((a[0] + a[1]) + (a[2] + a[3])) + bv;
    }
}

// ggml_im2col, 1-D (conv1d_f32, src/mmdit.cpp:20-25): dst[n][ow][ic * KW + kw]
// = x(iw = ow * s0 + kw * d0 - p0, ic, n), 0 outside [0, IW). x addressed by
// element strides of position, channel and batch (so a channels-fastest
// [IC, S] input needs no transpose first).
template <Elt E>
__global__ void im2col_1d_kernel(const float *x, int64_t sp, int64_t sc, int64_t sn, int IW, int IC, int KW, int OW,
                                 int N, int s0, int p0, int d0, void *dst, int64_t ld) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t K = (int64_t) IC * KW;
    if (i >= K * OW * N) return;
    const int64_t kk = i % K, row = i / K;
    const int ow = (int) (row % OW), n = (int) (row / OW);
    const int ic = (int) (kk / KW), kw = (int) (kk % KW);
    const int iw = ow * s0 + kw * d0 - p0;
    const float v = iw >= 0 && iw < IW ? x[(int64_t) iw * sp + (int64_t) ic * sc + (int64_t) n * sn] : 0.0f;
    store_from_f32<E>(dst, row * ld + kk, v);
}

// f32 rows -> bf16 (RNE), 4 elements per thread: row r = b * rows_per_b + i of
// x at b * ld_b + i * ld_x, y contiguous rows of `cols`
__global__ void cast_rows_bf16_kernel(const float *x, int64_t ld_x, int64_t ld_b, int rows_per_b, int64_t rows,
                                      int cols, uint16_t *y) {
    const int64_t q = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int cq = cols / 4;
    if (q >= rows * cq) return;
    const int64_t r = q / cq;
    const int c = (int) (q - r * cq) * 4;
    const int64_t b = r / rows_per_b, i = r - b * rows_per_b;
    const f32x4 v = *(const f32x4 *) (x + b * ld_b + i * ld_x + c);
    uint16_t t4[4] = {f32_to_bf16_bits(v[0]), f32_to_bf16_bits(v[1]), f32_to_bf16_bits(v[2]), f32_to_bf16_bits(v[3])};
    u32x2 w;
    __builtin_memcpy(&w, t4, 8);
    *(u32x2 *) (y + r * cols + c) = w;
}

// f32 rows -> the bf16 operand of a split product: row r of y (3 cols wide)
// is [hi | hi | lo] with hi = bf16(x), lo = bf16(x - hi), both RNE (x - hi is
// exact in f32). Against a weight held as [hi | lo | hi] one bf16 GEMM over
// 3 K sums x_hi w_hi + x_hi w_lo + x_lo w_hi, which is x w up to x_lo w_lo
// and the rounding of the two lo parts: about 2^-17 of |x w| per term. An
// infinite or NaN x keeps hi and gets lo = 0.
__global__ void cast_rows_split3_kernel(const float *x, int64_t ld_x, int64_t ld_b, int rows_per_b, int64_t rows,
                                        int cols, uint16_t *y) {
    const int64_t q = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int cq = cols / 4;
    if (q >= rows * cq) return;
    const int64_t r = q / cq;
    const int c = (int) (q - r * cq) * 4;
    const int64_t b = r / rows_per_b, i = r - b * rows_per_b;
    const f32x4 v = *(const f32x4 *) (x + b * ld_b + i * ld_x + c);
    uint16_t h4[4], l4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h4[e] = f32_to_bf16_bits(v[e]);
        const float hf = bf16_bits_to_f32(h4[e]);
        l4[e] = __builtin_isfinite(hf) ? f32_to_bf16_bits(v[e] - hf) : (uint16_t) 0;
    }
    u32x2 wh, wl;
    __builtin_memcpy(&wh, h4, 8);
    __builtin_memcpy(&wl, l4, 8);
    uint16_t *yr = y + r * 3 * cols + c;
    *(u32x2 *) yr = wh;
    *(u32x2 *) (yr + cols) = wh;
    *(u32x2 *) (yr + 2 * cols) = wl;
}

// conv kernel [KW, IC, OC] (element strides s0, s1, s2) -> kw-major rows
// dst[oc][kw * IC + ic], a bit copy
template <typename T>
__global__ void conv_pack_kernel(const T *w, int64_t s0, int64_t s1, int64_t s2, int KW, int IC, int OC, T *dst) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t) KW * IC * OC) return;
    const int ic = (int) (i % IC);
    const int64_t r = i / IC;
    const int kw = (int) (r % KW), oc = (int) (r / KW);
    dst[i] = w[kw * s0 + ic * s1 + oc * s2];
}

// ggml_mul(ggml_silu(a), b) (convmlp / mlp, src/mmdit.cpp:39-52): y = a / (1 + e^-a) * b
__global__ void silu_mul_kernel(const float *a, const float *b, float *y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { const float v = a[i]; y[i] = v / (1.0f + expf(-v)) * b[i]; }
}

// the same over K-split slices: a = sum of S slices of stride `stride`, b likewise, summed in slice order
__global__ void silu_mul_slices_kernel(const float *a, const float *b, int S, int64_t stride, float *y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = a[i], g = b[i];
    for (int z = 1; z < S; ++z) {
        v += a[z * stride + i];
        g += b[z * stride + i];
    }
    y[i] = v / (1.0f + expf(-v)) * g;
}

// y[n][m] = (sum of S K-split slices p[z][n][m], slice stride `stride`,
// rows of M, summed in slice order) + bias[m] (nullable), rows of ld_y
__global__ void sum_slices_kernel(const float *p, int S, int64_t stride, const float *bias, int64_t N, int M, float *y,
                                  int64_t ld_y) {
    const int64_t q = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int mq = M / 4;
    if (q >= N * mq) return;
    const int64_t n = q / mq;
    const int m = (int) (q - n * mq) * 4;
    const float *src = p + n * M + m;
    f32x4 v = *(const f32x4 *) src;
    for (int z = 1; z < S; ++z) {
        const f32x4 a = *(const f32x4 *) (src + z * stride);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += a[e];
    }
    if (bias) {
        const f32x4 b = *(const f32x4 *) (bias + m);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += b[e];
    }
    *(f32x4 *) (y + n * ld_y + m) = v;
}

// Convolution with few output channels (the VAE's final k7, 128 -> 2
// channels): stride 1, dilation 1, channels-fastest rows x [T][64 NI] in,
// planar y[oc][t] (row stride ld_y) out. One wave streams PW consecutive
// output positions: lane l holds channels l + 64 j of the KW input rows of
// the window in registers (zero outside [0, T)), one new row per position,
// prefetched CONV_SO_D rows ahead; each output is a wave sum of per-lane
// fp32 sums (kw, then j); lane (t - t0) % 64 keeps position t and stores 64
// positions per channel at once. A 128-row GEMM tile would carry 126 zero
// rows for these 2 outputs.
constexpr int CONV_SO_D = 8;
template <int NI, int KW, int OC>
__global__ __launch_bounds__(256) void conv_small_oc_kernel(const float *x, int T, const float *w, const float *bias,
                                                            int pad, float *y, int64_t ld_y, int PW) {
    constexpr int IC = 64 * NI, D = CONV_SO_D;
    const int lane = threadIdx.x & 63;
    const int t0 = (int) (blockIdx.x * 4 + (threadIdx.x >> 6)) * PW;
    if (t0 >= T) return;
    const int tend = min(T, t0 + PW);
    float wr[OC][KW][NI];
#pragma unroll
    for (int oc = 0; oc < OC; ++oc)
#pragma unroll
        for (int kw = 0; kw < KW; ++kw)
#pragma unroll
            for (int j = 0; j < NI; ++j) wr[oc][kw][j] = w[(int64_t) (oc * KW + kw) * IC + 64 * j + lane];
    auto row = [&](int r, float (&dst)[NI]) {
#pragma unroll
        for (int j = 0; j < NI; ++j) dst[j] = (r >= 0 && r < T) ? x[(int64_t) r * IC + 64 * j + lane] : 0.0f;
    };
    // window slot kw holds input row t - pad + kw at position t; before t0,
    // slots 1 .. KW - 1 hold rows t0 - pad .. t0 - pad + KW - 2
    float win[KW][NI];
#pragma unroll
    for (int kw = 1; kw < KW; ++kw) row(t0 - pad + kw - 1, win[kw]);
    float pf[D][NI], nx[D][NI];
#pragma unroll
    for (int i = 0; i < D; ++i) row(t0 - pad + KW - 1 + i, pf[i]);
    float keep[OC];
#pragma unroll
    for (int oc = 0; oc < OC; ++oc) keep[oc] = 0.0f;
    for (int tc = t0; tc < tend; tc += D) {
        if (tc + D < tend) {
#pragma unroll
            for (int i = 0; i < D; ++i) row(tc + D - pad + KW - 1 + i, nx[i]);
        }
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const int t = tc + i;
            if (t >= tend) break;
#pragma unroll
            for (int kw = 0; kw + 1 < KW; ++kw)
#pragma unroll
                for (int j = 0; j < NI; ++j) win[kw][j] = win[kw + 1][j];
#pragma unroll
            for (int j = 0; j < NI; ++j) win[KW - 1][j] = pf[i][j];
            const int slot = (t - t0) & 63;
#pragma unroll
            for (int oc = 0; oc < OC; ++oc) {
                float acc = 0.0f;
#pragma unroll
                for (int kw = 0; kw < KW; ++kw)
#pragma unroll
                    for (int j = 0; j < NI; ++j) acc = fmaf(wr[oc][kw][j], win[kw][j], acc);
                acc = wave_sum(acc);
                if (lane == slot) keep[oc] = acc;
            }
            if (slot == 63 || t == tend - 1) {
                const int tb = t - slot;
                if (lane <= slot)
#pragma unroll
                    for (int oc = 0; oc < OC; ++oc) y[oc * ld_y + tb + lane] = keep[oc] + (bias ? bias[oc] : 0.0f);
            }
        }
#pragma unroll
        for (int i = 0; i < D; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) pf[i][j] = nx[i][j];
    }
}

__global__ void silu_kernel(float *x, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { const float v = x[i]; x[i] = v / (1.0f + __expf(-v)); }
}

__global__ void timestep_embed_kernel(const float *freq, const TimeVals tv, int B, int H, float *temb) {
    const int half = H / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * half) return;
    const int b = i / half, k = i % half;
    const float a = tv.t[b] * freq[k];
    temb[(int64_t) b * H + k] = cosf(a);
    temb[(int64_t) b * H + half + k] = sinf(a);
}

// v = u + (c - u) cfg, x += dt v with every product and sum rounded as the
// reference's host loop writes them (src/mmdit.cpp:366-372): no FMA contraction
__global__ void cfg_euler_kernel(const float *flow2, int64_t n, float cfg, float dt, float *x, float *x2,
                                 float *flow0) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float fc = flow2[i], fu = flow2[n + i];
    const float v = fu + (fc - fu) * cfg;
    if (flow0) flow0[i] = v;
    const float nx = x[i] + dt * v;
    x[i] = nx;
    if (x2) { x2[i] = nx; x2[n + i] = nx; }
}

// RMS norm * w of norm_rows_kernel (RMS, one wave per row of 256 NV floats)
// followed by the Q8_0 quantization of quantize_rows_q8_kernel, in one pass:
// the 32-element block b of element (lane + 64 j) * 4 + e is held by lanes
// 8 (b % 8) .. + 7 at register j = b / 8, so its amax is three DPP steps.
// Same arithmetic as the two kernels in a row, so the same bits.
template <int NV>
__global__ __launch_bounds__(256) void rms_norm_q8_kernel(const float *x, int64_t ldx, const float *w, float eps,
                                                         int8_t *qx, float *dx, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    constexpr int n = 256 * NV;
    const float *xr = x + r * ldx;
    f32x4 v[NV], wv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        v[j] = *(const f32x4 *) (xr + (lane + 64 * j) * 4);
        wv[j] = *(const f32x4 *) (w + (lane + 64 * j) * 4);
    }
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        for (int e = 0; e < 4; ++e) s2 += v[j][e] * v[j][e];
    const float sc = 1.0f / sqrtf(wave_sum(s2) / (float) n + eps);
    int8_t *qr = qx + r * n;
    float *dr = dx + r * (n / 32);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        float o[4], amax = 0.0f;
        for (int e = 0; e < 4; ++e) {
            o[e] = v[j][e] * sc * wv[j][e];
            amax = fmaxf(amax, fabsf(o[e]));
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) amax = fmaxf(amax, dpp_f(amax, i));   // the 8 lanes of the block
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        if ((lane & 7) == 0) dr[8 * j + (lane >> 3)] = f16_bits_to_f32(f32_to_f16_bits(d));
        int8_t q[4];
        for (int e = 0; e < 4; ++e) q[e] = (int8_t) __builtin_rintf(o[e] * id);
        uint32_t w4;
        __builtin_memcpy(&w4, q, 4);
        *(uint32_t *) (qr + (lane + 64 * j) * 4) = w4;
    }
}

inline unsigned blocks_for(int64_t n, int per) { return (unsigned) ((n + per - 1) / per); }

}  // namespace

hipError_t launch_rms_norm_mul(const View4 &x, const float *w, float eps, const View4 &y, hipStream_t s) {
    const int64_t rows = x.ne[1] * x.ne[2] * x.ne[3];
    int64_t ldx, ldy;
    if (rows_fit(x, y, &ldx, &ldy) && !((uintptr_t) w & 15)) {
        launch_norm_rows<true>((const float *) x.data, ldx, w, eps, (float *) y.data, ldy, rows, (int) x.ne[0], s);
        return hipGetLastError();
    }
    launch_kernel(rms_norm_mul_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, w, eps, y, rows);
    return hipGetLastError();
}

hipError_t launch_norm(const View4 &x, float eps, const View4 &y, hipStream_t s) {
    const int64_t rows = x.ne[1] * x.ne[2] * x.ne[3];
    int64_t ldx, ldy;
    if (rows_fit(x, y, &ldx, &ldy)) {
        launch_norm_rows<false>((const float *) x.data, ldx, nullptr, eps, (float *) y.data, ldy, rows, (int) x.ne[0], s);
        return hipGetLastError();
    }
    launch_kernel(norm_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, eps, y, rows);
    return hipGetLastError();
}

hipError_t launch_rope(const View4 &x, const int32_t *pos, int n_dims, float theta_scale, float freq_scale,
                       const View4 &y, hipStream_t s) {
    const int64_t rows = x.ne[1] * x.ne[2] * x.ne[3];
    launch_kernel(rope_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, pos, n_dims, theta_scale,
                       freq_scale, y, rows);
    return hipGetLastError();
}

hipError_t launch_rope_table(float *cs, int npos, int n_dims, float theta_scale, float freq_scale, hipStream_t s) {
    if (npos < 1 || n_dims < 2 || n_dims % 2) return hipErrorInvalidValue;
    launch_kernel(rope_table_kernel, dim3(blocks_for((int64_t) npos * (n_dims / 2), 256)), dim3(256), 0, s, cs, npos,
                  n_dims, theta_scale, freq_scale);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope(const View4 &x, const float *w, const int32_t *pos, float eps, int n_dims,
                               float theta_scale, float freq_scale, const View4 &y, hipStream_t s) {
    const int64_t rows = x.ne[1] * x.ne[2] * x.ne[3];
    launch_kernel(qk_norm_rope_kernel, dim3(blocks_for(rows, 8)), dim3(256), 0, s, x, w, pos, eps, n_dims,
                       theta_scale, freq_scale, y, rows);
    return hipGetLastError();
}

hipError_t launch_q8_quantize_blocks(const float *x, int64_t ld_x, int64_t rows, int64_t K, void *blocks,
                                     int64_t ld_blocks, hipStream_t s) {
    launch_kernel(q8_quantize_blocks_kernel, dim3(blocks_for(rows * (K / 32), 256)), dim3(256), 0, s, x, ld_x,
                       rows, K, (char *) blocks, ld_blocks);
    return hipGetLastError();
}

hipError_t launch_q8_planes_to_blocks(const int8_t *qx, const float *dx, int64_t rows, int64_t K, void *blocks,
                                     int64_t ld_blocks, hipStream_t s) {
    launch_kernel(q8_planes_to_blocks_kernel, dim3(blocks_for(rows * (K / 32), 256)), dim3(256), 0, s, qx, dx, rows,
                  K, (char *) blocks, ld_blocks);
    return hipGetLastError();
}

hipError_t launch_q8_dequantize(const void *src, int split, int64_t rows, int64_t K, int64_t ld_src, float *y,
                                int64_t ld_y, hipStream_t s) {
    launch_kernel(q8_dequantize_kernel, dim3(blocks_for(rows * K, 256)), dim3(256), 0, s, (const char *) src,
                       split, rows, K, ld_src, y, ld_y);
    return hipGetLastError();
}

hipError_t launch_q8_repack(const void *src, int64_t ld_src, int64_t rows, int64_t K, void *dst, hipStream_t s) {
    launch_kernel(q8_repack_kernel, dim3(blocks_for(rows * (K / 32), 256)), dim3(256), 0, s, (const char *) src,
                       ld_src, rows, K, (char *) dst);
    return hipGetLastError();
}

hipError_t launch_f32_to_bf16(const float *x, uint16_t *y, int64_t n, hipStream_t s) {
    launch_kernel(f32_to_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_ln_group(const LnGroup &g, hipStream_t s, const L2PrefetchList *pf) {
    if (g.nstream < 1 || g.nstream > 2 || g.H < 4 || g.H % 4 || g.H > 4096) return hipErrorInvalidValue;
    if (pf && (pf->npf < 0 || pf->npf > L2PF_MAX)) return hipErrorInvalidValue;
    for (int i = 0; pf && i < pf->npf; ++i) {
        const L2Prefetch &f = pf->pf[i];
        if (!f.w || f.kt_n < 1 || f.splits < 1 || f.kt_n % f.splits || f.rb_tile < 1 || f.rb_n < 1 ||
            (f.tiles_m * f.splits) % 8 || (int64_t) f.tiles_m * f.rb_tile < f.rb_n)
            return hipErrorInvalidValue;
    }
    if (pf && pf->npf > 0) {
        // the BF16 DiT's LN (H = 1024, bf16 rows) only
        const int rows = g.s[0].rows + (g.nstream > 1 ? g.s[1].rows : 0);
        if (g.H != 1024 || g.y_mode != LN_Y_BF16) return hipErrorInvalidValue;
        launch_kernel(ln_wave_pf_kernel<LN_Y_BF16, 4>, dim3(rows), dim3(64), 0, s, g, *pf);
        return hipGetLastError();
    }
    const int rows = g.s[0].rows + (g.nstream > 1 ? g.s[1].rows : 0);
    if (g.y_mode == LN_Y_Q8) {
        // Q8_0 output: the wave kernel only (H = 1024 or 2048)
        if (g.H == 1024) launch_kernel(ln_wave_kernel<LN_Y_Q8, 4>, dim3(rows), dim3(64), 0, s, g);
        else if (g.H == 2048) launch_kernel(ln_wave_kernel<LN_Y_Q8, 8>, dim3(rows), dim3(64), 0, s, g);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (g.H == 1024 && !tuning().ln_block) {
        if (g.y_mode == LN_Y_F32) launch_kernel(ln_wave_kernel<LN_Y_F32, 4>, dim3(rows), dim3(64), 0, s, g);
        else launch_kernel(ln_wave_kernel<LN_Y_BF16, 4>, dim3(rows), dim3(64), 0, s, g);
        return hipGetLastError();
    }
    if (g.y_mode == LN_Y_F32) launch_kernel(ln_group_kernel<true>, dim3(rows), dim3(256), 0, s, g);
    else launch_kernel(ln_group_kernel<false>, dim3(rows), dim3(256), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_gemv_jobs(const GemvJob *jobs_dev, int njobs, int max_m, int B, int K, hipStream_t s) {
    // rows per wave at B <= 2 (2 measured best on the adaLN lists; 1 and 4 for sweeps)
    const int rw_env = tuning().gemv_rw;
    if (B <= 2 && rw_env == 4)
        launch_kernel(gemv_jobs_kernel<2, 4>, dim3(blocks_for(max_m, 16), njobs), dim3(256), 0, s, jobs_dev, B, K);
    else if (B <= 2 && rw_env == 2)
        launch_kernel(gemv_jobs_kernel<2, 2>, dim3(blocks_for(max_m, 8), njobs), dim3(256), 0, s, jobs_dev, B, K);
    else if (B <= 2)
        launch_kernel(gemv_jobs_kernel<2, 1>, dim3(blocks_for(max_m, 4), njobs), dim3(256), 0, s, jobs_dev, B, K);
    else if (B <= 8)
        launch_kernel(gemv_jobs_kernel<8, 2>, dim3(blocks_for(max_m, 8), njobs), dim3(256), 0, s, jobs_dev, B, K);
    else
        launch_kernel(gemv_jobs_kernel<32, 1>, dim3(blocks_for(max_m, 4), njobs), dim3(256), 0, s, jobs_dev, B, K);
    return hipGetLastError();
}

hipError_t launch_proj_f32(const uint16_t *w, const float *bias, const float *x, int64_t ld_x, int N, int K, int M,
                           float *y, int64_t ld_y, hipStream_t s) {
    if (N < 1 || M < 1 || K < 8 || K % 8 || ld_x % 4) return hipErrorInvalidValue;
    if (K == 1024) {   // long rows: lanes split K (final layer), one token per workgroup
        // (4 tokens per workgroup measured slower: 10.4 -> 16.6 us at 388 tokens)
        launch_kernel(proj_f32_kt_kernel<2, 1>, dim3((unsigned) ((M + 63) / 64), (unsigned) N), dim3(256), 0, s, w,
                      bias, x, ld_x, N, M, y, ld_y);
        return hipGetLastError();
    }
    if (K == 64) {     // the latent input: weights in registers, 16 tokens per workgroup
        launch_kernel(proj_f32_rows_kernel<64, 16>, dim3((unsigned) ((M + 63) / 64), (unsigned) ((N + 15) / 16)),
                      dim3(256), 0, s, w, bias, x, ld_x, N, M, y, ld_y, 0);
        return hipGetLastError();
    }
    const int64_t waves = (int64_t) N * ((M + 63) / 64);
    launch_kernel(proj_f32_kernel, dim3(blocks_for(waves, 4)), dim3(256), 0, s, w, bias, x, ld_x, N, K, M, y, ld_y);
    return hipGetLastError();
}

// [B][C][T] -> [B][T][C] (f32)
__global__ void transpose_ct_kernel(const float *x, int B, int C, int T, float *y) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t) B * C * T) return;
    const int t = (int) (i % T), c = (int) ((i / T) % C), b = (int) (i / ((int64_t) T * C));
    y[((int64_t) b * T + t) * C + c] = x[i];
}

// one 16-lane row per (token, head): lane sl of the row holds dimensions
// 4 sl .. 4 sl + 3 of q, k and v; row g of stream p: token g / nh, head g % nh
// (p.rows * p.nh is a multiple of 4, or the last wave's extra rows repeat
// the last pair, whose stores are the same)
__device__ __forceinline__ void qkv_scatter_wave(const QkvScatter &p, const int64_t w) {
    const int lane = threadIdx.x & 63, sl = lane & 15;
    const int64_t g = min(4 * w + (lane >> 4), (int64_t) p.rows * p.nh - 1);
    const int n = (int) (g / p.nh), h = (int) (g % p.nh);
    const int H = p.nh * 64;
    const float *row = p.qkv + (int64_t) n * p.ld + h * 64 + 4 * sl;
    f32x4 v[3];
#pragma unroll
    for (int sec = 0; sec < 3; ++sec) v[sec] = *(const f32x4 *) (row + sec * H);
#pragma unroll
    for (int sec = 0; sec < 3; ++sec) {
        const float x[4] = {v[sec][0], v[sec][1], v[sec][2], v[sec][3]};
        qkv_row_store(p, sec, h, n, x, sl);
    }
}

__global__ __launch_bounds__(256) void qkv_scatter_kernel(const QkvScatter p) {
    const int64_t w = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w < ((int64_t) p.rows * p.nh + 3) / 4) qkv_scatter_wave(p, w);
}

// two streams in one launch: waves from p0's (rows * nh + 3) / 4 on run p1
__global__ __launch_bounds__(256) void qkv_scatter2_kernel(const QkvScatter p0, const QkvScatter p1) {
    const int64_t w = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6), w0 = ((int64_t) p0.rows * p0.nh + 3) / 4;
    if (w < w0) qkv_scatter_wave(p0, w);
    else if (w - w0 < ((int64_t) p1.rows * p1.nh + 3) / 4) qkv_scatter_wave(p1, w - w0);
}

hipError_t launch_qkv_scatter(const QkvScatter &p, hipStream_t s) {
    if (p.rows < 1 || p.nh < 1 || p.seq < 1) return hipErrorInvalidValue;
    const int64_t waves = ((int64_t) p.rows * p.nh + 3) / 4;
    launch_kernel(qkv_scatter_kernel, dim3((unsigned) ((waves + 3) / 4)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_qkv_scatter2(const QkvScatter &p0, const QkvScatter &p1, hipStream_t s) {
    for (const QkvScatter *p : {&p0, &p1})
        if (p->rows < 1 || p->nh < 1 || p->seq < 1) return hipErrorInvalidValue;
    const int64_t waves = ((int64_t) p0.rows * p0.nh + 3) / 4 + ((int64_t) p1.rows * p1.nh + 3) / 4;
    launch_kernel(qkv_scatter2_kernel, dim3((unsigned) ((waves + 3) / 4)), dim3(256), 0, s, p0, p1);
    return hipGetLastError();
}

// ---- glue of the reference graph (src/mmdit.cpp:150-200, :285-289)

// y = bf16(silu(x)) (silu before the bf16 conversion of a BF16 mul_mat's src1)
__global__ void silu_bf16_kernel(const float *x, uint16_t *y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = f32_to_bf16_bits(v / (1.0f + expf(-v)));
}

// y[i] = a[i] + b[i] (f32)
__global__ void add_f32_kernel(const float *a, const float *b, float *y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

// mean over the S rows of each batch item: x [B][S][H] -> y [B][H]; the sum
// in double rounded to fp32, then divided by S (ggml_mean, src/mmdit.cpp:186)
// 64 columns per workgroup: wave w sums rows [w S / 4, (w + 1) S / 4) in
// double, then the four partial sums are added in order (a sum of at most a
// few thousand floats of similar size is exact in double in either order)
__global__ __launch_bounds__(256) void row_mean_kernel(const float *x, int S, int H, float *y) {
    __shared__ double part[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int b = blockIdx.y, c = blockIdx.x * 64 + lane;
    const int r0 = (int) ((int64_t) S * w / 4), r1 = (int) ((int64_t) S * (w + 1) / 4);
    double s = 0.0;
    if (c < H)
        for (int i = r0; i < r1; ++i) s += (double) x[((int64_t) b * S + i) * H + c];
    part[w][lane] = s;
    __syncthreads();
    if (w == 0 && c < H)
        y[(int64_t) b * H + c] = (float) (((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]) / (float) S;
}

// extended_c[b][t] = sync[b][idx(t)] + g[b], idx(t) = floor((t + 0.5) S / T)
// (ggml_get_rows with the nearest-exact index of src/mmdit.cpp:319, then the
// broadcast add of global_c, :196)
__global__ void sync_extend_kernel(const float *sync, int S, int T, int H, const float *g, float *y) {
    const int t = blockIdx.x, b = blockIdx.y;
    const int idx = min((int) floorf(((float) t + 0.5f) * (float) S / (float) T), S - 1);
    const float *src = sync + ((int64_t) b * S + idx) * H;
    const float *gb = g + (int64_t) b * H;
    float *dst = y + ((int64_t) b * T + t) * H;
    for (int c = threadIdx.x; c < H; c += blockDim.x) dst[c] = src[c] + gb[c];
}

// y[r][c] = x[r][c] + pe[(r % period)][c]
__global__ void add_period_rows_kernel(const float *x, int64_t rows, int cols, const float *pe, int period, float *y) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols;
    const int c = (int) (i % cols);
    y[i] = x[i] + pe[(r % period) * cols + c];
}

hipError_t launch_transpose_ct(const float *x, int B, int C, int T, float *y, hipStream_t s) {
    const int64_t n = (int64_t) B * C * T;
    launch_kernel(transpose_ct_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, B, C, T, y);
    return hipGetLastError();
}

hipError_t launch_add_period_rows(const float *x, int64_t rows, int cols, const float *pe, int period, float *y,
                                  hipStream_t s) {
    launch_kernel(add_period_rows_kernel, dim3(blocks_for(rows * cols, 256)), dim3(256), 0, s, x, rows, cols, pe,
                  period, y);
    return hipGetLastError();
}

hipError_t launch_silu_bf16(const float *x, uint16_t *y, int64_t n, hipStream_t s) {
    launch_kernel(silu_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_add_f32(const float *a, const float *b, float *y, int64_t n, hipStream_t s) {
    launch_kernel(add_f32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, a, b, y, n);
    return hipGetLastError();
}

hipError_t launch_row_mean(const float *x, int B, int S, int H, float *y, hipStream_t s) {
    launch_kernel(row_mean_kernel, dim3((H + 63) / 64, B), dim3(256), 0, s, x, S, H, y);
    return hipGetLastError();
}

hipError_t launch_sync_extend(const float *sync, int B, int S, int T, int H, const float *g, float *y, hipStream_t s) {
    launch_kernel(sync_extend_kernel, dim3(T, B), dim3(256), 0, s, sync, S, T, H, g, y);
    return hipGetLastError();
}

hipError_t launch_proj_f32_cm(const uint16_t *w, const float *bias, const float *x, int T, int N, int K, int M,
                              float *y, int64_t ld_y, float *tmp, hipStream_t s) {
    if (N < 1 || M < 1 || K < 8 || K % 8 || T < 1 || N % T) return hipErrorInvalidValue;
    if (K == 64) {
        launch_kernel(proj_f32_rows_kernel<64, 16>, dim3((unsigned) ((M + 63) / 64), (unsigned) ((N + 15) / 16)),
                      dim3(256), 0, s, w, bias, x, (int64_t) K, N, M, y, ld_y, T);
        return hipGetLastError();
    }
    // other widths: token-major copy in tmp ([N][K] f32), then the row kernels
    const int64_t n = (int64_t) N * K;
    launch_kernel(transpose_ct_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, s, x, N / T, K, T, tmp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_proj_f32(w, bias, tmp, K, N, K, M, y, ld_y, s);
}

hipError_t launch_im2col_1d(const float *x, int64_t sp, int64_t sc, int64_t sn, int IW, int IC, int KW, int OW, int N,
                           int s0, int p0, int d0, void *dst, int dst_type, int64_t ld, hipStream_t s) {
    const int64_t total = (int64_t) IC * KW * OW * N;
    if (total < 1) return hipErrorInvalidValue;
    const dim3 grid(blocks_for(total, 256)), block(256);
    switch (dst_type) {
        case (int) Elt::F32:
            launch_kernel(im2col_1d_kernel<Elt::F32>, grid, block, 0, s, x, sp, sc, sn, IW, IC, KW, OW, N, s0, p0, d0, dst, ld);
            break;
        case (int) Elt::F16:
            launch_kernel(im2col_1d_kernel<Elt::F16>, grid, block, 0, s, x, sp, sc, sn, IW, IC, KW, OW, N, s0, p0, d0, dst, ld);
            break;
        case (int) Elt::BF16:
            launch_kernel(im2col_1d_kernel<Elt::BF16>, grid, block, 0, s, x, sp, sc, sn, IW, IC, KW, OW, N, s0, p0, d0, dst, ld);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_cast_rows_bf16(const float *x, int64_t ld_x, int64_t ld_b, int rows_per_b, int64_t rows, int cols,
                                 uint16_t *y, hipStream_t s) {
    if (rows < 1 || cols < 4 || cols % 4 || rows_per_b < 1 || ld_x % 4 || ld_b % 4) return hipErrorInvalidValue;
    const int64_t n = rows * (cols / 4);
    launch_kernel(cast_rows_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, ld_x, ld_b, rows_per_b, rows, cols, y);
    return hipGetLastError();
}

hipError_t launch_cast_rows_split3(const float *x, int64_t ld_x, int64_t ld_b, int rows_per_b, int64_t rows, int cols,
                                   uint16_t *y, hipStream_t s) {
    if (rows < 1 || cols < 4 || cols % 4 || rows_per_b < 1 || ld_x % 4 || ld_b % 4) return hipErrorInvalidValue;
    const int64_t n = rows * (cols / 4);
    launch_kernel(cast_rows_split3_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, ld_x, ld_b, rows_per_b, rows,
                  cols, y);
    return hipGetLastError();
}

hipError_t launch_conv_pack(const void *w, int es, int64_t s0, int64_t s1, int64_t s2, int KW, int IC, int OC, void *dst,
                            hipStream_t s) {
    const int64_t total = (int64_t) KW * IC * OC;
    if (total < 1) return hipErrorInvalidValue;
    const dim3 grid(blocks_for(total, 256)), block(256);
    if (es == 4)
        launch_kernel(conv_pack_kernel<uint32_t>, grid, block, 0, s, (const uint32_t *) w, s0, s1, s2, KW, IC, OC,
                      (uint32_t *) dst);
    else if (es == 2)
        launch_kernel(conv_pack_kernel<uint16_t>, grid, block, 0, s, (const uint16_t *) w, s0, s1, s2, KW, IC, OC,
                      (uint16_t *) dst);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_rms_norm_q8(const float *x, int64_t ldx, const float *w, float eps, int8_t *qx, float *dx,
                              int64_t rows, int n, hipStream_t s) {
    if (rows < 1 || ldx % 4 || ((uintptr_t) x & 15) || ((uintptr_t) w & 15) || ((uintptr_t) qx & 3))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned) ((rows + 3) / 4)), blk(256);
    switch (n) {
        case 1024: launch_kernel(rms_norm_q8_kernel<4>, grid, blk, 0, s, x, ldx, w, eps, qx, dx, rows); break;
        case 2048: launch_kernel(rms_norm_q8_kernel<8>, grid, blk, 0, s, x, ldx, w, eps, qx, dx, rows); break;
        case 4096: launch_kernel(rms_norm_q8_kernel<16>, grid, blk, 0, s, x, ldx, w, eps, qx, dx, rows); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_conv_small_oc(const float *x, int T, int IC, int KW, int OC, const float *w, const float *bias,
                                 int pad, float *y, int64_t ld_y, hipStream_t s) {
    constexpr int PW = 256;
    if (T < 1 || pad < 0 || ld_y < T || !x || !w || !y) return hipErrorInvalidValue;
    const dim3 grid((unsigned) (((T + PW - 1) / PW + 3) / 4));
    if (IC == 128 && KW == 7 && OC == 2)
        launch_kernel((conv_small_oc_kernel<2, 7, 2>), grid, dim3(256), 0, s, x, T, w, bias, pad, y, ld_y, PW);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_silu_mul_slices(const float *a, const float *b, int S, int64_t stride, float *y, int64_t n,
                                  hipStream_t s) {
    if (S < 1 || (S > 1 && stride < n)) return hipErrorInvalidValue;
    launch_kernel(silu_mul_slices_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, a, b, S, stride, y, n);
    return hipGetLastError();
}

hipError_t launch_sum_slices(const float *p, int S, int64_t stride, const float *bias, int64_t N, int M, float *y,
                             int64_t ld_y, hipStream_t s) {
    if (S < 1 || N < 1 || M < 4 || M % 4 || ld_y % 4 || stride % 4 || (S > 1 && stride < N * M) ||
        ((uintptr_t) p & 15) || ((uintptr_t) y & 15) || (bias && ((uintptr_t) bias & 15)))
        return hipErrorInvalidValue;
    const int64_t n = N * (M / 4);
    launch_kernel(sum_slices_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, S, stride, bias, N, M, y, ld_y);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *a, const float *b, float *y, int64_t n, hipStream_t s) {
    launch_kernel(silu_mul_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, a, b, y, n);
    return hipGetLastError();
}

hipError_t launch_silu_inplace(float *x, int64_t n, hipStream_t s) {
    launch_kernel(silu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, n);
    return hipGetLastError();
}

hipError_t launch_timestep_embed(const float *freq, const TimeVals &tv, int B, int H, float *temb, hipStream_t s) {
    launch_kernel(timestep_embed_kernel, dim3(blocks_for((int64_t) B * (H / 2), 256)), dim3(256), 0, s, freq, tv,
                       B, H, temb);
    return hipGetLastError();
}

hipError_t launch_cfg_euler(const float *flow2, int64_t n, float cfg, float dt, float *x, float *x2, float *flow0,
                            hipStream_t s) {
    launch_kernel(cfg_euler_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, flow2, n, cfg, dt, x, x2, flow0);
    return hipGetLastError();
}

}  // namespace tsk
