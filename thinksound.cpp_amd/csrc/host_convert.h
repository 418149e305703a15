// host_convert.h — host-side conversions of weights at upload: fp32 -> bf16
// / fp16 bits (round to nearest even), ggml's reference Q8_0 quantizer, and
// Q8_0 blocks -> the split planes the Q8_0 GEMMs read.
#pragma once

#include <math.h>
#include <stdint.h>
#include <string.h>

namespace tsk {

// fp32 -> bf16 bits, RNE; NaN stays a (quiet) NaN
inline uint16_t host_bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 64u);
    return (uint16_t) ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

// fp32 -> fp16 bits, RNE (GGML_FP32_TO_FP16 of a Q8_0 block scale)
inline uint16_t host_f16_bits(float f) {
    const _Float16 h = (_Float16) f;
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}

inline float host_f16_value(uint16_t b) {
    _Float16 h;
    memcpy(&h, &b, 2);
    return (float) h;
}

// quantize_row_q8_0_ref of ggml: per 32 values d = amax / 127 (stored fp16),
// q = round-half-away(x * (1 / d)); nblocks blocks of 34 bytes
inline void q8_quantize_ref(const float *x, int64_t nblocks, uint8_t *blocks) {
    for (int64_t bi = 0; bi < nblocks; ++bi) {
        const float *v = x + bi * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t *blk = blocks + bi * 34;
        const uint16_t h = host_f16_bits(d);
        memcpy(blk, &h, 2);
        for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t) (int8_t) roundf(v[j] * id);
    }
}

// Q8_0 blocks of M rows of K values -> int8 plane q [M][K] and fp16 scale
// plane d [M][K / 32] (bit-preserving)
inline void q8_blocks_to_planes(const uint8_t *blocks, int64_t M, int64_t K, int8_t *q, uint16_t *d) {
    const int64_t KB = K / 32;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t kb = 0; kb < KB; ++kb) {
            const uint8_t *blk = blocks + (m * KB + kb) * 34;
            memcpy(&d[m * KB + kb], blk, 2);
            memcpy(&q[m * K + kb * 32], blk + 2, 32);
        }
}

}  // namespace tsk
