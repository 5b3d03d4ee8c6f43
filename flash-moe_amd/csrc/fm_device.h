// fm_device.h -- gfx950 device helpers shared by the quantized-expert kernels.
//
// Dequant arithmetic.  The reference computes, per row,
//   sum_g sum_{i in g} (code_i * s_g + b_g) * x_i          (cpu_kernels.h:199-232)
// which equals  sum_g ( s_g * sum_{i in g} code_i x_i  +  b_g * sum_{i in g} x_i ).
// The kernels use the second form.  Codes are small integers, so the inner dot
// runs on v_dot2_f32_f16 (two fp16 products, fp32 accumulate) fed straight
// from the packed word: a nibble masked in place, with the fp16 exponent field
// left at zero, IS the fp16 subnormal code * 2^-24 (or * 2^-20 for the nibble
// at bits 4..7) -- exact, no conversion instruction at all.  The 2^-24 is
// folded into the group scale and the 2^4 factors into the fp16 copy of x.
// Per 4-bit word (8 codes): one shift, four ANDs, four dot2 = 1.1 VALU ops per
// code, which keeps an HBM-rate stream under the CU's vector issue budget.
// (fp16 denormals are preserved: the kernels run with denorm mode 16/64 = 3.)
//
// Operand range.  x enters the dot products as fp16, so every 64-element group
// is first scaled by a power of two 2^e chosen from the group's largest |x|
// (fm_group_shift: max |x| * 2^e lands in [2^14, 2^15)).  The field factors
// (down to 2^-8 for 2-bit fields) then still leave every value of the group
// inside fp16's normal range, whatever the magnitude of x (1e-6 or 3e4): the
// fp16 rounding error is at most 2^-12 of the group's largest |x|.  The
// inverse 2^(24-e) -- with the 2^24 of the subnormal codes -- multiplies the
// group scale in the fold; the group sum stays unscaled fp32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fm_expf.h"

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

// ---- x layout per group --------------------------------------------------
// A lane owns whole 64-element groups.  For one group it keeps 32 fp16 pairs
// ordered (and pre-scaled by 2^-log2(m)) to match the code pairs:
//  4-bit word p (elements 8p..8p+7):  (x0,x4) (x1,x5)/16 (x2,x6) (x3,x7)/16
//  2-bit word p (elements 16p..+15):  (x_n, x_{n+8}) / 4^(n mod 5 ... see fm_dot_word2)
// plus the fp32 group sum for the bias term.
struct FmXGroup {
    fm_h2 q[32];
    float sum;
    float inv;  // 2^(24 - e): the group's operand scale 2^e undone, codes' 2^-24 folded in
};

// 2^e as a float, e in [-126, 127] (exact).
FM_DEV float fm_exp2i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// Shift e for a group whose largest magnitude is amax: amax * 2^e in [2^14, 2^15)
// (clamped to [-100, 100]: all-zero or subnormal groups take 2^100, which keeps
// 2^(24 - e) a normal float).
FM_DEV int fm_group_shift(float amax) {
    const int E = (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127;
    return min(max(14 - E, -100), 100);
}

template <int BITS>
FM_DEV void fm_load_xgroup(const float *__restrict__ xg, FmXGroup &g) {
    float s = 0.f, mx = 0.f;
#pragma unroll
    for (int p = 0; p < 16; p++) {
        const fm_f4 a = *(const fm_f4 *)(xg + 4 * p);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
    }
    const int e = fm_group_shift(mx);
    const float f = fm_exp2i(e);
    g.inv = fm_exp2i(24 - e);
    if constexpr (BITS == 4) {
        const float f16 = f * 0.0625f;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            fm_f4 a = *(const fm_f4 *)(xg + 8 * p);
            fm_f4 b = *(const fm_f4 *)(xg + 8 * p + 4);
            g.q[4 * p + 0] = fm_pack_h2(a.x * f, b.x * f);
            g.q[4 * p + 1] = fm_pack_h2(a.y * f16, b.y * f16);
            g.q[4 * p + 2] = fm_pack_h2(a.z * f, b.z * f);
            g.q[4 * p + 3] = fm_pack_h2(a.w * f16, b.w * f16);
            s += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        }
    } else {
        // code field n of a 2-bit word sits at bit 2n (n <= 4) or 2(n-5) after >> 10
        float m[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
        for (int i = 0; i < 8; i++) m[i] *= f;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            fm_f4 a0 = *(const fm_f4 *)(xg + 16 * p);
            fm_f4 a1 = *(const fm_f4 *)(xg + 16 * p + 4);
            fm_f4 b0 = *(const fm_f4 *)(xg + 16 * p + 8);
            fm_f4 b1 = *(const fm_f4 *)(xg + 16 * p + 12);
            g.q[8 * p + 0] = fm_pack_h2(a0.x * m[0], b0.x * m[0]);
            g.q[8 * p + 1] = fm_pack_h2(a0.y * m[1], b0.y * m[1]);
            g.q[8 * p + 2] = fm_pack_h2(a0.z * m[2], b0.z * m[2]);
            g.q[8 * p + 3] = fm_pack_h2(a0.w * m[3], b0.w * m[3]);
            g.q[8 * p + 4] = fm_pack_h2(a1.x * m[4], b1.x * m[4]);
            g.q[8 * p + 5] = fm_pack_h2(a1.y * m[5], b1.y * m[5]);
            g.q[8 * p + 6] = fm_pack_h2(a1.z * m[6], b1.z * m[6]);
            g.q[8 * p + 7] = fm_pack_h2(a1.w * m[7], b1.w * m[7]);
            s += ((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w)) +
                 ((b0.x + b0.y) + (b0.z + b0.w)) + ((b1.x + b1.y) + (b1.z + b1.w));
        }
    }
    g.sum = s;
}

// fm_load_xgroup for all G groups of x by a whole workgroup: four adjacent
// threads per group, 16 elements each (loop over 4 G thread slots; G a
// multiple of 16 keeps every wave's lanes in step for the shuffles, other G
// leave whole 4-thread groups idle together).  Same values as fm_load_xgroup.
template <int BITS>
FM_DEV void fm_stage_xgroups(const float *__restrict__ x, uint32_t G, FmXGroup *xs) {
    for (uint32_t i = threadIdx.x; i < ((4 * G + 63) & ~63u); i += blockDim.x) {
        const uint32_t g = i >> 2, qq = i & 3;
        const bool live = g < G;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const fm_f4 t = live ? *(const fm_f4 *)(x + 64 * g + 16 * qq + 4 * j) : (fm_f4){0.f, 0.f, 0.f, 0.f};
            v[4 * j] = t.x;
            v[4 * j + 1] = t.y;
            v[4 * j + 2] = t.z;
            v[4 * j + 3] = t.w;
        }
        float mx = 0.f, sm = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
#pragma unroll
        for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        sm += __shfl_xor(sm, 1, 64);
        sm += __shfl_xor(sm, 2, 64);
        if (!live) continue;
        const int e = fm_group_shift(mx);
        const float f = fm_exp2i(e);
        FmXGroup &o = xs[g];
        if constexpr (BITS == 4) {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float m = (j & 1) ? 0.0625f * f : f;
                    o.q[4 * (2 * qq + h) + j] = fm_pack_h2(v[8 * h + j] * m, v[8 * h + 4 + j] * m);
                }
        } else {
            const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
            for (int n = 0; n < 8; n++) o.q[8 * qq + n] = fm_pack_h2(v[n] * (mt[n] * f), v[8 + n] * (mt[n] * f));
        }
        if (qq == 0) {
            o.sum = sm;
            o.inv = fm_exp2i(24 - e);
        }
    }
}

// sum over one 4-bit word of code_i * x_i * 2^-24 (8 codes, 9 VALU ops).
FM_DEV float fm_dot_word4(uint32_t w, const fm_h2 *q, float acc) {
    uint32_t t = w >> 8;
    acc = fm_dot2(fm_as_h2(w & 0x000F000Fu), q[0], acc);
    acc = fm_dot2(fm_as_h2(w & 0x00F000F0u), q[1], acc);
    acc = fm_dot2(fm_as_h2(t & 0x000F000Fu), q[2], acc);
    acc = fm_dot2(fm_as_h2(t & 0x00F000F0u), q[3], acc);
    return acc;
}

// one 2-bit word (16 codes): pairs (c_n, c_{n+8}), times 2^-24.
FM_DEV float fm_dot_word2(uint32_t w, const fm_h2 *q, float acc) {
    uint32_t t = w >> 10;
    acc = fm_dot2(fm_as_h2(w & 0x00030003u), q[0], acc);
    acc = fm_dot2(fm_as_h2(w & 0x000C000Cu), q[1], acc);
    acc = fm_dot2(fm_as_h2(w & 0x00300030u), q[2], acc);
    acc = fm_dot2(fm_as_h2(w & 0x00C000C0u), q[3], acc);
    acc = fm_dot2(fm_as_h2(w & 0x03000300u), q[4], acc);
    acc = fm_dot2(fm_as_h2(t & 0x00030003u), q[5], acc);
    acc = fm_dot2(fm_as_h2(t & 0x000C000Cu), q[6], acc);
    acc = fm_dot2(fm_as_h2(t & 0x00300030u), q[7], acc);
    return acc;
}

// Raw words of one group: 8 (4-bit) or 4 (2-bit) uint32 = 32 / 16 bytes.
struct FmWGroup {
    fm_u4 a, b;
};

// Global-address-space loads.  Pointers that pass through LDS (staged slot
// descriptors) lose their address space; a flat load would then share the LDS
// wait counter, so every LDS access or cross-lane op would wait for all
// in-flight weight prefetches.  These force global_load_* instead.
#define FM_GLOBAL __attribute__((address_space(1)))
FM_DEV fm_u4 fm_ldg_u4_nt(const void *p) { return __builtin_nontemporal_load((const FM_GLOBAL fm_u4 *)p); }
FM_DEV fm_u4 fm_ldg_u4(const void *p) { return *(const FM_GLOBAL fm_u4 *)p; }
FM_DEV uint16_t fm_ldg_u16(const void *p) { return *(const FM_GLOBAL uint16_t *)p; }
FM_DEV float fm_ldg_f32(const void *p) { return *(const FM_GLOBAL float *)p; }
FM_DEV fm_f4 fm_ldg_f4(const void *p) { return *(const FM_GLOBAL fm_f4 *)p; }

template <int BITS>
FM_DEV void fm_load_wgroup(const uint32_t *__restrict__ wg, FmWGroup &w) {
    w.a = fm_ldg_u4_nt(wg);
    if constexpr (BITS == 4) w.b = fm_ldg_u4_nt(wg + 4);
}

// s * sum(code*x) + b * sum(x) for one group (the dot carries codes * 2^-24).
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
    return __builtin_fmaf(s * x.inv, acc0 + acc1, b * x.sum);  // codes carried * 2^-24, x * 2^e
}

// DPP lane moves (GFX9 encodings): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_ror:4 = 0x124, row_ror:8 = 0x128, wave_shl:1 = 0x130.
template <int CTRL>
FM_DEV int fm_dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
FM_DEV float fm_dpp_f(float v) { return __int_as_float(fm_dpp_i<CTRL>(__float_as_int(v))); }

// Sum over aligned segments of L lanes (L in {16, 32, 64}).  The total is
// valid in the FIRST lane of each segment (for L == 16: in every lane).
// In-row steps are DPP adds; the cross-row steps are v_readlane into SGPRs,
// so no LDS crossbar (ds_bpermute / ds_swizzle) round trips are involved.
template <int L>
FM_DEV float fm_lane_sum(float v) {
    v += fm_dpp_f<0xB1>(v);
    v += fm_dpp_f<0x4E>(v);
    v += fm_dpp_f<0x124>(v);
    v += fm_dpp_f<0x128>(v);
    if constexpr (L == 32) {
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
        v += (threadIdx.x & 32) ? r3 : r1;
    } else if constexpr (L == 64) {
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
        const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
        v = (v + r1) + (r2 + r3);
    }
    return v;
}

// Max over each aligned 16-lane DPP row (valid in every lane of the row).
FM_DEV float fm_row16_max(float v) {
    v = fmaxf(v, fm_dpp_f<0xB1>(v));
    v = fmaxf(v, fm_dpp_f<0x4E>(v));
    v = fmaxf(v, fm_dpp_f<0x124>(v));
    v = fmaxf(v, fm_dpp_f<0x128>(v));
    return v;
}

FM_DEV float fm_silu_mul(float g, float u) {
    float sg = g / (1.0f + expf(-g));
    return sg * u;
}

// cpu_sigmoid (cpu_kernels.h:258-260) with the reference libm's expf: bit-equal.
FM_DEV float fm_sigmoid(float x) { return 1.0f / (1.0f + fm_expf_ref(-x)); }
