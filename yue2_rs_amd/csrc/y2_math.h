// y2_math.h -- scalar math shared by the HIP kernels and the host runtime.
//
// Every function here is deterministic IEEE arithmetic (+, -, *, /, sqrt,
// fma, rint, conversions) with an explicit evaluation order, so the host and
// the device produce the same bits.  All sources are compiled with
// -ffp-contract=off: a fused multiply-add happens only where fma() is
// written.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define Y2_HD __host__ __device__ __forceinline__

namespace y2 {

Y2_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
Y2_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
Y2_HD uint64_t d2u(double f) { return __builtin_bit_cast(uint64_t, f); }
Y2_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// round_bf16 of src/tensor.rs:645-652: round to nearest even at bit 16,
// NaN becomes a quiet NaN with the payload's top bits.
// On the device this is the gfx950 conversion v_cvt_pk_bf16_f32 (round to
// nearest even under the kernels' default mode, denormals kept, NaN quieted
// with its top bits kept: the same bits for all 2^32 inputs, checked
// exhaustively against the integer form), two instructions where the integer
// form takes seven -- it is inlined at every rounding of the decode step.
Y2_HD float rb(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
    return u2f((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v) << 16);
#else
    const uint32_t b = f2u(v);
    const uint32_t nan = (b & 0xffff0000u) | 0x00400000u;
    const uint32_t rne = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
    return u2f((b & 0x7fffffffu) > 0x7f800000u ? nan : rne);
#endif
}
// BF16 bits of a value that is already BF16-exact.
Y2_HD uint16_t bf16_bits(float v) { return (uint16_t)(f2u(v) >> 16); }
Y2_HD float bf16_lo(uint32_t pair) { return u2f(pair << 16); }
Y2_HD float bf16_hi(uint32_t pair) { return u2f(pair & 0xffff0000u); }
Y2_HD float bf16(uint16_t b) { return u2f((uint32_t)b << 16); }

// exp of an f32 argument, rounded once to f32.  Cody-Waite reduction
// x = n ln2 + r (ln2 = 43-bit head + tail, |r| <= ln2/2), e^r from the
// Taylor series to degree 13 in double precision, exact scaling by 2^n.
// The double result is within ~2^-52 relative of e^x, so the f32 result is
// the correctly rounded exp except within ~2^-52 of a rounding midpoint.
Y2_HD float expf_cr(float xf) {
    if (xf != xf) return xf + xf;
    if (xf > 89.0f) return __builtin_huge_valf();
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double n = __builtin_rint(x * 0x1.71547652b82fep+0);
    double r = __builtin_fma(-n, 0x1.62e42fefa3800p-1, x);
    r = __builtin_fma(-n, 0x1.ef35793c76730p-45, r);
    double p = 0x1.6124613a86d09p-33;           // 1/13!
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);  // 1/12!
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);  // 1/11!
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);  // 1/10!
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);  // 1/9!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);  // 1/8!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);  // 1/7!
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);  // 1/6!
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);   // 1/5!
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);   // 1/4!
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);   // 1/3!
    p = __builtin_fma(p, r, 0x1.0000000000000p-1);   // 1/2!
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    const int64_t ni = (int64_t)n;
    return (float)(p * u2d((uint64_t)(ni + 1023) << 52));
}

// log(m) for m in [sqrt(1/2), sqrt(2)): 2 atanh(s), s = (m-1)/(m+1), series
// 2 s^(2j+1)/(2j+1) to j = 11.
Y2_HD double log_core(double m) {
    const double f1 = m - 1.0;
    const double s = f1 / (2.0 + f1);
    const double z = s * s;
    double p = 0x1.642c8590b2164p-4;            // 2/23
    p = __builtin_fma(p, z, 0x1.8618618618618p-4);  // 2/21
    p = __builtin_fma(p, z, 0x1.af286bca1af28p-4);  // 2/19
    p = __builtin_fma(p, z, 0x1.e1e1e1e1e1e1ep-4);  // 2/17
    p = __builtin_fma(p, z, 0x1.1111111111111p-3);  // 2/15
    p = __builtin_fma(p, z, 0x1.3b13b13b13b14p-3);  // 2/13
    p = __builtin_fma(p, z, 0x1.745d1745d1746p-3);  // 2/11
    p = __builtin_fma(p, z, 0x1.c71c71c71c71cp-3);  // 2/9
    p = __builtin_fma(p, z, 0x1.2492492492492p-2);  // 2/7
    p = __builtin_fma(p, z, 0x1.999999999999ap-2);  // 2/5
    p = __builtin_fma(p, z, 0x1.5555555555555p-1);  // 2/3
    return __builtin_fma(s * z, p, s + s);
}

// Split a positive normal double u = m 2^k with m in [sqrt(1/2), sqrt(2)).
Y2_HD double split_log_arg(double u, int* k) {
    const uint64_t bits = d2u(u);
    int e = (int)((bits >> 52) & 0x7ff) - 1022;
    double f = u2d((bits & 0x000fffffffffffffull) | 0x3fe0000000000000ull);  // [0.5, 1)
    if (f < 0x1.6a09e667f3bcdp-1) {
        f = f + f;
        e -= 1;
    }
    *k = e;
    return f;
}

// log1p in double precision (replaces Rust f64::ln_1p):
// u = 1 + x, correction c = (x - (u - 1)) / u, log u = k ln2 + log m.
Y2_HD double log1p_d(double x) {
    if (x == 0.0) return x;
    if (x != x) return x + x;
    if (x <= -1.0) return x == -1.0 ? -__builtin_huge_val() : __builtin_nan("");
    if (x == __builtin_huge_val()) return x;
    const double u = 1.0 + x;
    const double c = (x - (u - 1.0)) / u;
    int k;
    const double m = split_log_arg(u, &k);
    const double lm = log_core(m);
    const double kd = (double)k;
    return __builtin_fma(kd, 0x1.62e42fefa3800p-1, lm + __builtin_fma(kd, 0x1.ef35793c76730p-45, c));
}

// SiLU with the reference's rounding points (src/tensor.rs:661-686):
// rb(g / (1 + exp(-g))).
Y2_HD float silu_rb(float g) { return rb(g / (1.0f + expf_cr(-g))); }

// RMSNorm scale from an f32 sum of squares (src/tensor.rs:1144-1147).
Y2_HD float norm_scale_from_sum(float sum, int n, float eps) {
    return rb(1.0f / __builtin_sqrtf(sum / (float)n + eps));
}

// Order-preserving key of f32::total_cmp.
Y2_HD int32_t total_key(float f) {
    const int32_t b = (int32_t)f2u(f);
    return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

}  // namespace y2
