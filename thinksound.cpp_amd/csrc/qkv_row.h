// qkv_row.h — the attention operands from one token's q / k / v features of
// one head (the QKV epilogue of the Q8_0 driver, mmdit.cpp:67-90): shared by
// the scatter kernel over f32 rows and the Q8_0 GEMM's epilogue, so that both
// paths compile to the same arithmetic.
#pragma once

#include "tsk_common.h"
#include "tsk_internal.h"

namespace tsk {

// Token n (row n = b * seq + s of the stream) of head h, section sec (0 q,
// 1 k, 2 v), held by one 16-lane row of the wave: lane sl of the row holds
// features 4 sl .. 4 sl + 3 in x (every lane of the wave takes part, one
// (token, head) per row). q and k get RMSNorm(eps) * w, RoPE from rope_cs
// (when rope) and, for q, the factor q_scale, then go to fp16 in
// [B][nh][Ntot][64] at token tok_off + s; v goes to fp16 in vt, as such rows
// (v_rows) or as V^T [B][nh][64][ldv] at vt_pos(tok_off + s). No product is contracted into an FMA or into the fp16
// conversion, so every caller rounds the same way.
__device__ __forceinline__ void qkv_row_store(const QkvScatter &p, int sec, int h, int n, const float (&x)[4], int sl) {
#pragma clang fp contract(off)
    const int b = n / p.seq, s = n - b * p.seq, tok = p.tok_off + s;
    const int64_t bh = (int64_t) b * p.nh + h;
    if (sec == 2) {
        if (p.v_rows) {
            const uint16_t o4[4] = {f32_to_f16_bits(x[0]), f32_to_f16_bits(x[1]), f32_to_f16_bits(x[2]),
                                    f32_to_f16_bits(x[3])};
            u32x2 w2;
            __builtin_memcpy(&w2, o4, 8);
            *(u32x2 *) (p.vt + (bh * p.Ntot + tok) * 64 + 4 * sl) = w2;
        } else {
            uint16_t *col = p.vt + (bh * 64 + 4 * sl) * p.ldv + vt_pos(tok);
#pragma unroll
            for (int e = 0; e < 4; ++e) col[(int64_t) e * p.ldv] = f32_to_f16_bits(x[e]);
        }
        return;
    }
    const float *wp = (sec ? p.kn_w : p.qn_w) + 4 * sl;
    const float w[4] = {wp[0], wp[1], wp[2], wp[3]};
    const float sq = ((x[0] * x[0] + x[1] * x[1]) + x[2] * x[2]) + x[3] * x[3];
    const float sc = 1.0f / sqrtf(row16_sum(sq) / 64.0f + p.eps);
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = x[e] * sc * w[e];
    if (p.rope) {
        // pairs (4 sl, 4 sl + 1), (4 sl + 2, 4 sl + 3): (cos, sin) at the even, odd index
        const float *cp = p.rope_cs + (int64_t) s * 64 + 4 * sl;
        const float cs[4] = {cp[0], cp[1], cp[2], cp[3]};
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2) {
            const float e0 = y[2 * q2], o0 = y[2 * q2 + 1], c = cs[2 * q2], sn = cs[2 * q2 + 1];
            y[2 * q2] = e0 * c - o0 * sn;
            y[2 * q2 + 1] = e0 * sn + o0 * c;
        }
    }
    uint16_t o4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float v = sec == 0 ? y[e] * p.q_scale : y[e];
        // v is rounded to fp32 before its conversion to fp16: without the
        // barrier the compiler may fold the last product into the conversion
        // (one v_fma_mix rounding) in one caller and not in another
        asm volatile("" : "+v"(v));
        o4[e] = f32_to_f16_bits(v);
    }
    u32x2 w2;
    __builtin_memcpy(&w2, o4, 8);
    *(u32x2 *) ((sec ? p.k : p.q) + (bh * p.Ntot + tok) * 64 + 4 * sl) = w2;
}

}  // namespace tsk
