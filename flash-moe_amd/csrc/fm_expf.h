// fm_expf.h -- expf with the exact results of the reference's libm.
//
// The reference's routing and shared-expert gate call libm expf
// (cpu_softmax / cpu_sigmoid, cpu_kernels.h:258-277); the oracle, the
// reference compiled on this image, links glibc 2.35, whose expf is the ARM
// optimized-routines algorithm (published in glibc as
// sysdeps/ieee754/flt-32/e_expf.c with the table of e_exp2f_data.c):
//   x / ln2 = k/32 + r/32 with k = round(x * 32 / ln2), |r| <= 1/2;
//   2^(k/32) = 2^(k div 32) * 2^((k mod 32) / 32), the latter from a table;
//   2^(r/32) ~= 1 + c2 r + c1 r^2 + c0 r^3 (minimax), all in double;
//   the double result is rounded once to float.
// On x86-64 CPUs with FMA (the hosts here) glibc runs the variant compiled
// with -mfma, where k and r come from fused multiply-adds; this restatement
// uses fma for those and for the polynomial.  Checked exhaustively against the
// oracle's libm: bit-equal for every non-NaN float input (4.28e9 values),
// so routing on the device sees exactly the probabilities the CPU sees.
//
// The table entry i is the bit pattern of 2^(i/32) rounded to double, minus
// i << 47 (the exponent bits that k mod 32 adds back); the table can be
// regenerated from that rule.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define FM_HD __host__ __device__ inline
#else
#define FM_HD static inline
#endif

#define FM_EXPF_TAB                                                                                  \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,      \
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,  \
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,  \
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,  \
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,  \
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,  \
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,  \
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

// The algorithm for x inside [-0x1.9fe368p6f, 0x1.62e42ep6f], with the table
// entry supplied by `tab(i)` (i = 0..31), so device code can keep the table
// in registers instead of memory.
template <class Tab>
FM_HD float fm_expf_core(float x, Tab tab) {
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32.0;  // 32 / ln 2
    const double shift = 0x1.8p+52;                         // rounds to an integer in the low mantissa bits
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const uint64_t t = tab((int)(ki % 32)) + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// The cases outside that range: NaN, underflow to 0 (below half the smallest
// subnormal, and -inf), overflow to inf.
FM_HD float fm_expf_special(float x, float core) {
    float y = x < -0x1.9fe368p6f ? 0.0f : core;
    y = x > 0x1.62e42ep6f ? __builtin_inff() : y;
    return x != x ? x + x : y;
}

// x clamped into the core's range (a NaN becomes the lower bound).
FM_HD float fm_expf_clamp(float x) { return __builtin_fminf(__builtin_fmaxf(x, -0x1.9fe368p6f), 0x1.62e42ep6f); }

FM_HD float fm_expf_ref(float x) {
    const uint64_t tab[32] = {FM_EXPF_TAB};
    return fm_expf_special(x, fm_expf_core(fm_expf_clamp(x), [&](int i) { return tab[i]; }));
}

#if defined(__HIPCC__)
// The table in device memory as 64 dwords: fm_expf_lanes_load gives lane l
// dword l (lo/hi words of entry l / 2), fm_expf_lanes looks entries up with
// ds_bpermute -- no dependent memory load in the exp itself.  ds_bpermute
// reads 0 from inactive lanes, so fm_expf_lanes must run with every lane of
// the wave active (no early exits inside: the special cases are selects).
static __device__ const uint64_t fm_expf_tab_dev[32] = {FM_EXPF_TAB};
__device__ __forceinline__ uint32_t fm_expf_lanes_load() {
    return ((const uint32_t *)fm_expf_tab_dev)[threadIdx.x & 63];
}
__device__ __forceinline__ float fm_expf_lanes(float x, uint32_t lanes) {
    const float core = fm_expf_core(fm_expf_clamp(x), [&](int i) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(8 * i, (int)lanes);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(8 * i + 4, (int)lanes);
        return ((uint64_t)hi << 32) | lo;
    });
    return fm_expf_special(x, core);
}
#endif
