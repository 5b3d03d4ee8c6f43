// fm_device.h -- gfx950 device helpers shared by the quantized-expert kernels.
//
// Dequant arithmetic.  The reference computes, per row,
//   sum_g sum_{i in g} (code_i * s_g + b_g) * x_i          (cpu_kernels.h:199-232)
// which equals  sum_g ( s_g * sum_{i in g} code_i x_i  +  b_g * sum_{i in g} x_i ).
// The kernels use the second form: codes are exact small integers, so the
// inner dot runs on v_dot2_f32_f16 (two fp16 products, fp32 accumulate) with
// codes unpacked by the fp16 "magic exponent" trick (OR the nibbles into the
// mantissa of 1024.0h, then one packed fp16 FMA makes them exact integers),
// and the per-group scale/bias are applied once per group in fp32.
// That is ~1.6 VALU ops per 4-bit code instead of ~3 for cvt+fma, which is
// what keeps an HBM-rate matvec under the CU's vector issue budget.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 fm_h2 __attribute__((ext_vector_type(2)));
typedef float fm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t fm_u4 __attribute__((ext_vector_type(4)));

#define FM_DEV __device__ __forceinline__

FM_DEV float fm_bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet).
FM_DEV uint16_t fm_f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

FM_DEV fm_h2 fm_as_h2(uint32_t u) { return __builtin_bit_cast(fm_h2, u); }
FM_DEV uint32_t fm_h2_bits(fm_h2 h) { return __builtin_bit_cast(uint32_t, h); }

FM_DEV fm_h2 fm_pack_h2(float lo, float hi) {
    fm_h2 r;
    r.x = (_Float16)lo;
    r.y = (_Float16)hi;
    return r;
}

FM_DEV float fm_dot2(fm_h2 a, fm_h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// (1024 + m*c) -> c exactly, for a code field whose lowest bit sits at mantissa
// bit log2(m).  One v_pk_add_f16 (m == 1) or v_pk_fma_f16.
template <int M>
FM_DEV fm_h2 fm_magic_norm(uint32_t masked) {
    fm_h2 v = fm_as_h2(masked | 0x64006400u);
    if constexpr (M == 1) {
        const fm_h2 off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
        return v + off;
    } else {
        const fm_h2 sc = {(_Float16)(1.0f / M), (_Float16)(1.0f / M)};
        const fm_h2 off = {(_Float16)(-1024.0f / M), (_Float16)(-1024.0f / M)};
        return __builtin_elementwise_fma(v, sc, off);
    }
}

// ---- x layout per group --------------------------------------------------
// A lane owns whole 64-element groups.  For one group it keeps 32 fp16 pairs
// ordered to match the code pairs the unpack produces:
//  4-bit word p (elements 8p..8p+7): pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7)
//  2-bit word p (elements 16p..16p+15): pairs (x_n, x_{n+8}), n = 0..7
// plus the fp32 group sum for the bias term.
struct FmXGroup {
    fm_h2 q[32];
    float sum;
};

template <int BITS>
FM_DEV void fm_load_xgroup(const float *__restrict__ xg, FmXGroup &g) {
    float s = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int p = 0; p < 8; p++) {
            fm_f4 a = *(const fm_f4 *)(xg + 8 * p);
            fm_f4 b = *(const fm_f4 *)(xg + 8 * p + 4);
            g.q[4 * p + 0] = fm_pack_h2(a.x, b.x);
            g.q[4 * p + 1] = fm_pack_h2(a.y, b.y);
            g.q[4 * p + 2] = fm_pack_h2(a.z, b.z);
            g.q[4 * p + 3] = fm_pack_h2(a.w, b.w);
            s += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        }
    } else {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            fm_f4 a0 = *(const fm_f4 *)(xg + 16 * p);
            fm_f4 a1 = *(const fm_f4 *)(xg + 16 * p + 4);
            fm_f4 b0 = *(const fm_f4 *)(xg + 16 * p + 8);
            fm_f4 b1 = *(const fm_f4 *)(xg + 16 * p + 12);
            g.q[8 * p + 0] = fm_pack_h2(a0.x, b0.x);
            g.q[8 * p + 1] = fm_pack_h2(a0.y, b0.y);
            g.q[8 * p + 2] = fm_pack_h2(a0.z, b0.z);
            g.q[8 * p + 3] = fm_pack_h2(a0.w, b0.w);
            g.q[8 * p + 4] = fm_pack_h2(a1.x, b1.x);
            g.q[8 * p + 5] = fm_pack_h2(a1.y, b1.y);
            g.q[8 * p + 6] = fm_pack_h2(a1.z, b1.z);
            g.q[8 * p + 7] = fm_pack_h2(a1.w, b1.w);
            s += ((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w)) +
                 ((b0.x + b0.y) + (b0.z + b0.w)) + ((b1.x + b1.y) + (b1.z + b1.w));
        }
    }
    g.sum = s;
}

// sum over one group of code_i * x_i, for one 4-bit word (8 codes).
FM_DEV float fm_dot_word4(uint32_t w, const fm_h2 *q, float acc) {
    uint32_t t = w >> 8;
    acc = fm_dot2(fm_magic_norm<1>(w & 0x000F000Fu), q[0], acc);
    acc = fm_dot2(fm_magic_norm<16>(w & 0x00F000F0u), q[1], acc);
    acc = fm_dot2(fm_magic_norm<1>(t & 0x000F000Fu), q[2], acc);
    acc = fm_dot2(fm_magic_norm<16>(t & 0x00F000F0u), q[3], acc);
    return acc;
}

// one 2-bit word (16 codes): pairs (c_n, c_{n+8}).
FM_DEV float fm_dot_word2(uint32_t w, const fm_h2 *q, float acc) {
    uint32_t t = w >> 10;
    acc = fm_dot2(fm_magic_norm<1>(w & 0x00030003u), q[0], acc);
    acc = fm_dot2(fm_magic_norm<4>(w & 0x000C000Cu), q[1], acc);
    acc = fm_dot2(fm_magic_norm<16>(w & 0x00300030u), q[2], acc);
    acc = fm_dot2(fm_magic_norm<64>(w & 0x00C000C0u), q[3], acc);
    acc = fm_dot2(fm_magic_norm<256>(w & 0x03000300u), q[4], acc);
    acc = fm_dot2(fm_magic_norm<1>(t & 0x00030003u), q[5], acc);
    acc = fm_dot2(fm_magic_norm<4>(t & 0x000C000Cu), q[6], acc);
    acc = fm_dot2(fm_magic_norm<16>(t & 0x00300030u), q[7], acc);
    return acc;
}

// Raw words of one group: 8 (4-bit) or 4 (2-bit) uint32 = 32 / 16 bytes.
struct FmWGroup {
    fm_u4 a, b;
};

template <int BITS>
FM_DEV void fm_load_wgroup(const uint32_t *__restrict__ wg, FmWGroup &w) {
    w.a = __builtin_nontemporal_load((const fm_u4 *)wg);
    if constexpr (BITS == 4) w.b = __builtin_nontemporal_load((const fm_u4 *)wg + 1);
}

// s * sum(code*x) + b * sum(x) for one group.
template <int BITS>
FM_DEV float fm_group_dot(const FmWGroup &w, const FmXGroup &x, float s, float b) {
    float acc0 = 0.f, acc1 = 0.f;
    if constexpr (BITS == 4) {
        acc0 = fm_dot_word4(w.a.x, &x.q[0], acc0);
        acc1 = fm_dot_word4(w.a.y, &x.q[4], acc1);
        acc0 = fm_dot_word4(w.a.z, &x.q[8], acc0);
        acc1 = fm_dot_word4(w.a.w, &x.q[12], acc1);
        acc0 = fm_dot_word4(w.b.x, &x.q[16], acc0);
        acc1 = fm_dot_word4(w.b.y, &x.q[20], acc1);
        acc0 = fm_dot_word4(w.b.z, &x.q[24], acc0);
        acc1 = fm_dot_word4(w.b.w, &x.q[28], acc1);
    } else {
        acc0 = fm_dot_word2(w.a.x, &x.q[0], acc0);
        acc1 = fm_dot_word2(w.a.y, &x.q[8], acc1);
        acc0 = fm_dot_word2(w.a.z, &x.q[16], acc0);
        acc1 = fm_dot_word2(w.a.w, &x.q[24], acc1);
    }
    return __builtin_fmaf(s, acc0 + acc1, b * x.sum);
}

// Sum over aligned groups of L lanes (L in {16, 32, 64}); every lane of the
// group receives the total.
template <int L>
FM_DEV float fm_lane_sum(float v) {
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

FM_DEV float fm_silu_mul(float g, float u) {
    float sg = g / (1.0f + expf(-g));
    return sg * u;
}

FM_DEV float fm_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
