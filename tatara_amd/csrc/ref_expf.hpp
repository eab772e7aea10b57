// exp as the reference's CPU path evaluates it: Rust's f32::exp calls glibc's
// expf on linux-gnu.  ref_expf restates glibc's published method (ARM
// optimized-routines: x / ln2 * 32 = k + r, exp(x) = 2^(k/32) * p(r) with a
// cubic p in double, the FMA build glibc selects on x86-64 CPUs with FMA);
// the 2^(i/32) table entries are 2^(i/32) rounded to double.  The result
// equals glibc's on every non-NaN float, so sigmoids built on it (progress
// buckets, the losses) are bit-identical to the reference's CPU values.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tatara {
namespace {

__constant__ uint64_t c_exp2_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};
// entry i holds the bits of 2^(i/32) minus (i << 52) / 32, so that adding
// k << 47 to it scales by 2^(k/32) in exponent-and-table form

__device__ __forceinline__ float ref_expf(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_huge_valf();
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = c_exp2_tab[ki % 32] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double zz = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(zz, r2, y);
    y = y * s;
    return (float)y;
}

}  // namespace
}  // namespace tatara
