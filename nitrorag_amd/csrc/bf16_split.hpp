// fp32 values as exact sums of bf16 numbers, for fp32-accurate products on
// gfx950's bf16 matrix cores.
//
// A finite fp32 v (not below 2^-102 in magnitude unless zero) is hi + mid +
// lo exactly, where hi is the upper 16 bits of v (a bf16 truncation), mid
// the upper 16 bits of v - hi, and lo = v - hi - mid: each part keeps 8
// significant bits of what is left, 24 in all.  The product of two bf16
// numbers is exact in fp32, so sum_i parts_i * parts_j accumulated in fp32
// by v_mfma_f32_*_bf16 keeps fp32 accuracy when the dropped cross terms are
// below fp32 resolution (an int8 factor is exact in one part).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nitro {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float upper16(float v) { return __uint_as_float(__float_as_uint(v) & 0xffff0000u); }

// Elements (a, b) as a bf16 pair: the upper 16 bits of each (bytes 2, 3 of a
// then bytes 2, 3 of b; v_perm_b32 numbers the second operand's bytes 0-3 and
// the first's 4-7).
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// The three parts of v, each as a bf16 bit pattern.
__device__ __forceinline__ void split_parts(float v, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
    const float r1 = v - upper16(v);
    const float r2 = r1 - upper16(r1);
    hi = (uint16_t)(__float_as_uint(v) >> 16);
    mid = (uint16_t)(__float_as_uint(r1) >> 16);
    lo = (uint16_t)(__float_as_uint(r2) >> 16);
}

// Eight values as three bf16x8 operands: hi, mid, lo.
__device__ __forceinline__ void split3(const float (&v)[8], bf16x8& hi, bf16x8& mid, bf16x8& lo) {
    u32x4 h, m, l;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const float a = v[2 * p], b = v[2 * p + 1];
        const float ar = a - upper16(a), br = b - upper16(b);
        const float al = ar - upper16(ar), bl = br - upper16(br);
        h[p] = bf16_pair(a, b);
        m[p] = bf16_pair(ar, br);
        l[p] = bf16_pair(al, bl);
    }
    hi = __builtin_bit_cast(bf16x8, h);
    mid = __builtin_bit_cast(bf16x8, m);
    lo = __builtin_bit_cast(bf16x8, l);
}

// Eight values as two bf16x8 operands, hi and mid (each a truncation): v
// minus hi + mid is below 2^-16 |v| (16 significant bits kept).  For factors
// whose products need only that (the attention weights, each added into a
// sum of thousands of terms: a relative error of 2^-16 per weight moves the
// output by about 1e-5 of its size).
__device__ __forceinline__ void split2(const float (&v)[8], bf16x8& hi, bf16x8& mid) {
    u32x4 h, m;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const float a = v[2 * p], b = v[2 * p + 1];
        h[p] = bf16_pair(a, b);
        m[p] = bf16_pair(a - upper16(a), b - upper16(b));
    }
    hi = __builtin_bit_cast(bf16x8, h);
    mid = __builtin_bit_cast(bf16x8, m);
}

}  // namespace nitro
