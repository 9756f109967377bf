// af_device.h — device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace af {

typedef _Float16 f16;

__device__ __forceinline__ float h2f(uint16_t h) { return float(__builtin_bit_cast(f16, h)); }
// fp32 -> fp16, round to nearest even (v_cvt_f16_f32 under the default mode).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, f16(f)); }

// OCP E4M3FN encode (bias 7, max 448 = 0x7E, 0x7F NaN, no infinities), round to
// nearest even. The input must already be clamped to +-448.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x43e00000u) return sign | 0x7eu;  // 448
    if (a < 0x3c800000u) {                      // below 2^-6: quantum 2^-9
        const float v = __builtin_bit_cast(float, a) * 512.0f;
        return sign | uint32_t(__builtin_rintf(v));  // 8 lands on 2^-6 (e=1, m=0)
    }
    const int e = int(a >> 23) - 127;
    const uint32_t mant = a & 0x7fffffu;
    uint32_t m3 = mant >> 20;
    const uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3 += 1;  // carry bumps the exponent
    return sign | ((uint32_t(e + 7) << 3) + m3);
}

// Quantiser convention of tools/quantize_weights.py:249-260: divide by the
// scale (IEEE), clamp to +-448, cast to e4m3fn (round to nearest even).
__device__ __forceinline__ uint32_t quantize_fp8(uint16_t h, float scale) {
    float v = h2f(h) / scale;
    v = fminf(fmaxf(v, -448.0f), 448.0f);
    return e4m3_encode(v);
}

// RoPE rotation of one fp16 pair (x, y) by (c, s): separately rounded fp32
// products and sums, then fp16 round-to-nearest-even (the reference's
// rope_kernel arithmetic, src/kernel/rope.cu:34-35; no FMA contraction).
__device__ __forceinline__ void rope_rotate(uint16_t x, uint16_t y, float c, float s, uint16_t& xo,
                                            uint16_t& yo) {
#pragma clang fp contract(off)
    const float xf = h2f(x), yf = h2f(y);
    const float xc = xf * c;
    const float ys = yf * s;
    const float xs = xf * s;
    const float yc = yf * c;
    xo = f2h(xc - ys);
    yo = f2h(xs + yc);
}

// 2^x on v_exp_f32 (1 ulp; flushes below 2^-126, 2^-inf = 0).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- cross-lane reductions (wave64) -----------------------------------------
// DPP move of v (row_mask, bank_mask all lanes; bound_ctrl: a source lane
// outside the row would read 0, which none of the controls used here has).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Cross-row exchanges of gfx950 (VALU, no LDS round trip). With a = b = v on
// entry, v_permlane16_swap leaves rows (v0, v0, v2, v2) in a and (v1, v1, v3, v3)
// in b (rows of 16 lanes); v_permlane32_swap leaves (lo, lo) in a and (hi, hi)
// in b (halves of 32 lanes). Written as inline asm with both operands
// read-write: the compiler's builtin returns the first result for both. The
// s_nop provides the two wait states the swap needs after a VALU write.
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Sum / max over the four 16-lane rows of values that are uniform per row.
__device__ __forceinline__ float rows_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap16(a, b);
    v = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    a = b = __builtin_bit_cast(uint32_t, v);
    swap32(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float rows_max(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap16(a, b);
    v = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = b = __builtin_bit_cast(uint32_t, v);
    swap32(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x128>(v);
    return rows_sum(v);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x128>(v));
    return rows_max(v);
}

}  // namespace af
