// tsk_common.h — shared device types and helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tsk/tsk.h"

namespace tsk {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

constexpr int kWave = 64;

// ---- scalar conversions (round to nearest even) -------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t) h << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((x >> 16) | 64u);
    return (uint16_t) ((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16) f;              // v_cvt_f16_f32: RNE
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float) __builtin_bit_cast(_Float16, h);
}

// Element-type tags used by the kernels' templates.
enum class Elt : int { F32 = 0, F16 = 1, BF16 = 30 };

template <Elt E> struct EltInfo;
template <> struct EltInfo<Elt::F32>  { typedef float    storage; static constexpr int bytes = 4; };
template <> struct EltInfo<Elt::F16>  { typedef uint16_t storage; static constexpr int bytes = 2; };
template <> struct EltInfo<Elt::BF16> { typedef uint16_t storage; static constexpr int bytes = 2; };

template <Elt E> __device__ __forceinline__ float load_as_f32(const void *p, int64_t i) {
    if constexpr (E == Elt::F32) return ((const float *) p)[i];
    else if constexpr (E == Elt::F16) return f16_bits_to_f32(((const uint16_t *) p)[i]);
    else return bf16_bits_to_f32(((const uint16_t *) p)[i]);
}
template <Elt E> __device__ __forceinline__ void store_from_f32(void *p, int64_t i, float v) {
    if constexpr (E == Elt::F32) ((float *) p)[i] = v;
    else if constexpr (E == Elt::F16) ((uint16_t *) p)[i] = f32_to_f16_bits(v);
    else ((uint16_t *) p)[i] = f32_to_bf16_bits(v);
}

// GELU, tanh form: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3),
// tanh(u) = 1 - 2 / (exp(2u) + 1), the quotient through the hardware
// reciprocal (v_rcp_f32, within 1 ulp; an IEEE division is ten instructions
// per element in every GELU epilogue). exp(2u) = inf gives t = 1, exp(2u) = 0
// gives t = -1.
__device__ __forceinline__ float gelu_tanh_f(float x) {
    const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * u) + 1.0f);
    return 0.5f * x * (1.0f + t);
}

// RoPE angle of pair i at position p: p * theta_scale^i as a running product
// (the order ggml's rope evaluates it in)
__device__ __forceinline__ float rope_theta(float p, float theta_scale, int pair) {
    float th = p;
    for (int j = 0; j < pair; ++j) th *= theta_scale;
    return th;
}

// 64-lane reductions without LDS: DPP steps inside each 16-lane row (swaps
// within quads, the half-row and the row mirrors), then v_permlane16_swap and
// v_permlane32_swap pair the rows. Each step combines the same two values in
// either order, so every lane ends with the same bits. The whole wave must be
// active.
__device__ __forceinline__ float dpp_f(float v, int ctrl_id) {
    switch (ctrl_id) {
        case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
        case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
        case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
        default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
    }
}
// sum over each 16-lane row (every lane of the row gets the sum); all 16
// lanes of a row must be active
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v += dpp_f(v, i);
    return v;
}
// the other 16-lane row of the same 32-lane half (rows 0 <-> 1, 2 <-> 3): {own, other} in either order
__device__ __forceinline__ float row_pair_sum(float v) {
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
}
__device__ __forceinline__ float row_pair_max(float v) {
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
}
// the same lane of the other 32-lane half
__device__ __forceinline__ float half_pair_sum(float v) {
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
}
__device__ __forceinline__ float half_pair_max(float v) {
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v = fmaxf(v, dpp_f(v, i));
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

}  // namespace tsk
