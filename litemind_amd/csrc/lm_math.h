// lm_math.h -- scalar math shared by the gfx950 kernels and host code.
//
// LiteMind computes softmax and SiLU with std::exp(float) (src/Gemm.cpp:216,
// :229), which resolves to the C library's expf.  On this platform that is
// glibc 2.35, whose expf is the ARM Optimized Routines algorithm
// (math/expf.c + math/exp2f_data.c, adopted as sysdeps/ieee754/flt-32/e_expf.c
// in glibc 2.27): x * 32/ln2 = k + r, exp(x) = 2^(k/32) * p(r) with a 32-entry
// table of 2^(i/32) and a cubic in double precision.  On x86-64 glibc selects
// the build compiled with -mfma, where GCC fuses the range reduction
// (kd = fma(InvLn2N, x, Shift), r = fma(InvLn2N, x, -kd)).
//
// lm::expf_ref restates that published algorithm with the fused reduction
// spelled out, so the GPU produces the same softmax weights as LiteMind bit for
// bit.  The 2^(i/32) table below is computed from the definition (correctly
// rounded 2^(i/32) in double, minus i << 47), not copied.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define LM_HD __host__ __device__
#else
#define LM_HD
#endif

namespace lm {

LM_HD inline double bits_double(uint64_t u) { return __builtin_bit_cast(double, u); }
LM_HD inline uint64_t double_bits(double d) { return __builtin_bit_cast(uint64_t, d); }
LM_HD inline uint32_t float_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
LM_HD inline float bits_float(uint32_t u) { return __builtin_bit_cast(float, u); }

// BF16 bits -> float: shift into the high half (src/Gemm.cpp:18-20).
LM_HD inline float widen_bf16(uint16_t bits) { return bits_float(static_cast<uint32_t>(bits) << 16); }

// 2^(i/32) as double bits, with i << 47 subtracted so adding k << 47 scales by 2^(k/32).
// A select tree over the five index bits: on the GPU the index differs from
// lane to lane, so a switch would compile to a tree of divergent branches that
// every wave walks in full, and a table in memory would put a load behind the
// kernel's weight stream in the in-order memory queue.
LM_HD inline uint64_t exp2_table(uint32_t i) {
    const bool b0 = (i & 1u) != 0, b1 = (i & 2u) != 0, b2 = (i & 4u) != 0, b3 = (i & 8u) != 0,
               b4 = (i & 16u) != 0;
    const uint64_t v0 = b0 ? 0x3fefd9b0d3158574ull : 0x3ff0000000000000ull;
    const uint64_t v1 = b0 ? 0x3fef9301d0125b51ull : 0x3fefb5586cf9890full;
    const uint64_t v2 = b0 ? 0x3fef54873168b9aaull : 0x3fef72b83c7d517bull;
    const uint64_t v3 = b0 ? 0x3fef1e9df51fdee1ull : 0x3fef387a6e756238ull;
    const uint64_t v4 = b0 ? 0x3feef1a7373aa9cbull : 0x3fef06fe0a31b715ull;
    const uint64_t v5 = b0 ? 0x3feece086061892dull : 0x3feedea64c123422ull;
    const uint64_t v6 = b0 ? 0x3feeb42b569d4f82ull : 0x3feebfdad5362a27ull;
    const uint64_t v7 = b0 ? 0x3feea47eb03a5585ull : 0x3feeab07dd485429ull;
    const uint64_t v8 = b0 ? 0x3fee9f75e8ec5f74ull : 0x3feea09e667f3bcdull;
    const uint64_t v9 = b0 ? 0x3feea589994cce13ull : 0x3feea11473eb0187ull;
    const uint64_t v10 = b0 ? 0x3feeb737b0cdc5e5ull : 0x3feeace5422aa0dbull;
    const uint64_t v11 = b0 ? 0x3feed503b23e255dull : 0x3feec49182a3f090ull;
    const uint64_t v12 = b0 ? 0x3feeff76f2fb5e47ull : 0x3feee89f995ad3adull;
    const uint64_t v13 = b0 ? 0x3fef3720dcef9069ull : 0x3fef199bdd85529cull;
    const uint64_t v14 = b0 ? 0x3fef7c97337b9b5full : 0x3fef5818dcfba487ull;
    const uint64_t v15 = b0 ? 0x3fefd0765b6e4540ull : 0x3fefa4afa2a490daull;
    const uint64_t w0 = b1 ? v1 : v0;
    const uint64_t w1 = b1 ? v3 : v2;
    const uint64_t w2 = b1 ? v5 : v4;
    const uint64_t w3 = b1 ? v7 : v6;
    const uint64_t w4 = b1 ? v9 : v8;
    const uint64_t w5 = b1 ? v11 : v10;
    const uint64_t w6 = b1 ? v13 : v12;
    const uint64_t w7 = b1 ? v15 : v14;
    const uint64_t x0 = b2 ? w1 : w0;
    const uint64_t x1 = b2 ? w3 : w2;
    const uint64_t x2 = b2 ? w5 : w4;
    const uint64_t x3 = b2 ? w7 : w6;
    const uint64_t y0 = b3 ? x1 : x0;
    const uint64_t y1 = b3 ? x3 : x2;
    return b4 ? y1 : y0;
}

// expf as glibc 2.35 computes it on an FMA-capable x86-64 host (see the header),
// with the 2^(i/32) entry (exp2_table's value for i = ki % 32) supplied by
// `table`: the select tree above, or a copy of it that a kernel keeps in LDS.
template <class Table>
LM_HD inline float expf_with(float x, Table table) {
    const uint32_t abstop = (float_bits(x) >> 20) & 0x7ffu;
    if (abstop >= (float_bits(88.0f) >> 20)) {
        if (float_bits(x) == float_bits(-__builtin_inff())) {
            return 0.0f;
        }
        if (abstop >= (float_bits(__builtin_inff()) >> 20)) {
            return x + x;
        }
        if (x > 0x1.62e42ep6f) {
            return __builtin_inff();
        }
        if (x < -0x1.9fe368p6f) {
            return 0.0f;
        }
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = static_cast<double>(x);
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = double_bits(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = table(static_cast<uint32_t>(ki % 32u));
    t += ki << 47;
    const double s = bits_double(t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

LM_HD inline float expf_ref(float x) { return expf_with(x, exp2_table); }

// silu(g) * u with LiteMind's rounding steps: g / (1 + exp(-g)), then * u (src/Gemm.cpp:225-231).
LM_HD inline float silu_mul_ref(float g, float u) {
    const float denom = 1.0f + expf_ref(-g);
    const float s = g / denom;
    return s * u;
}

}  // namespace lm
