// fm_mfma_dev.h -- MFMA operand builders and slot lookups shared by the
// decode kernels (fm_decode_mfma.hip, fm_decode_ring.hip).
#pragma once
#include "fm_decode.h"

typedef _Float16 fmm_h8 __attribute__((ext_vector_type(8)));
typedef float fmm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t fmm_u2 __attribute__((ext_vector_type(2)));

#define FMM_H 4096             // hidden size this kernel is specialised for
#define FMM_MAXI 1024          // largest intermediate size (k of the down rows)
#define FMM_GH (FMM_H / 64)    // input groups of a gate/up row
#define FMM_GI (FMM_MAXI / 64) // input groups of a down row (max)
#define FMM_BLOCKS_PER_CU 3
#define FMM_TS 68  // words per row of a wave's transpose buffer (64 + 4 pad: no bank conflicts)

// One packed word -> the B operand of one MFMA (8 subnormal fp16 codes).
// 4-bit: [c0 c4 c1' c5' c2 c6 c3' c7'] (' = field *16); 2-bit: half h of the
// word's 16 codes, pairs n = 4h..4h+3 of the fm_dot_word2 layout.
template <int BITS>
FM_DEV fmm_h8 fmm_codes(uint32_t w, int h) {
    uint32_t r0, r1, r2, r3;
    if constexpr (BITS == 4) {
        const uint32_t t = w >> 8;
        r0 = w & 0x000F000Fu;
        r1 = w & 0x00F000F0u;
        r2 = t & 0x000F000Fu;
        r3 = t & 0x00F000F0u;
    } else if (h == 0) {
        r0 = w & 0x00030003u;
        r1 = w & 0x000C000Cu;
        r2 = w & 0x00300030u;
        r3 = w & 0x00C000C0u;
    } else {
        const uint32_t t = w >> 10;
        r0 = w & 0x03000300u;
        r1 = t & 0x00030003u;
        r2 = t & 0x000C000Cu;
        r3 = t & 0x00300030u;
    }
    fm_u4 v = {r0, r1, r2, r3};
    return __builtin_bit_cast(fmm_h8, v);
}

FM_DEV fmm_h8 fmm_lds_op(const fm_h2 *p) { return __builtin_bit_cast(fmm_h8, *(const fm_u4 *)p); }

// One 64-element group of v (fp32, in LDS), scaled by f = 2^e -> operand row
// layout for BITS, 32 pairs; this call writes pair e.
FM_DEV void fmm_build_pair(const float *v, int bits, int e, float f, fm_h2 *dst) {
    if (bits == 4) {
        const int p = e >> 2, j = e & 3;
        const float m = (j & 1) ? 0.0625f * f : f;
        dst[e] = fm_pack_h2(v[8 * p + j] * m, v[8 * p + 4 + j] * m);
    } else {
        const int p = e >> 3, n = e & 7;
        // pair n: (x_n, x_{n+8}) / 4^(field position of code n in the word)
        const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
        dst[e] = fm_pack_h2(v[16 * p + n] * (mt[n] * f), v[16 * p + 8 + n] * (mt[n] * f));
    }
}

// Sum over the 16 lanes of each DPP row (result valid in every lane).
FM_DEV float fmm_row_sum(float v) {
    v += fm_dpp_f<0xB1>(v);
    v += fm_dpp_f<0x4E>(v);
    v += fm_dpp_f<0x124>(v);
    v += fm_dpp_f<0x128>(v);
    return v;
}

FM_DEV uint32_t fmm_comp(const fm_u4 &v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }

// Fold: lane (row n, q) holds D[4q+v][n] = dot of row n with group g0+4q+v;
// ginv4 undoes each group's operand scale (and the codes' 2^-24).
FM_DEV float fmm_fold(const fmm_f4 &d, fmm_u2 sc, fmm_u2 bi, const float *gsum4, const float *ginv4) {
    const float s0 = __uint_as_float(sc.x << 16), s1 = __uint_as_float(sc.x & 0xffff0000u);
    const float s2 = __uint_as_float(sc.y << 16), s3 = __uint_as_float(sc.y & 0xffff0000u);
    const float b0 = __uint_as_float(bi.x << 16), b1 = __uint_as_float(bi.x & 0xffff0000u);
    const float b2 = __uint_as_float(bi.y << 16), b3 = __uint_as_float(bi.y & 0xffff0000u);
    const fm_f4 gi = *(const fm_f4 *)ginv4, gs = *(const fm_f4 *)gsum4;
    float r = __builtin_fmaf(s0 * gi.x, d[0], b0 * gs.x);
    r += __builtin_fmaf(s1 * gi.y, d[1], b1 * gs.y);
    r += __builtin_fmaf(s2 * gi.z, d[2], b2 * gs.z);
    r += __builtin_fmaf(s3 * gi.w, d[3], b3 * gs.w);
    return r;
}

// Sum over the four lanes n, n+16, n+32, n+48 (valid in every lane).
FM_DEV float fmm_q_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Copy 16-byte runs into LDS with the vector memory DMA path (lane l's run
// lands at lds + 16 l).  Written as inline assembly so that the compiler's
// wait counts ignore it: they then only ever over-wait (these loads are older
// than every load it counts after them), and the issuing wave waits for the
// copy itself with an explicit vmcnt.  m0 (the DMA's LDS base) is restored.
FM_DEV void fmc_dma16(void *lds, const void *g) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"((uint32_t)(uintptr_t)lds), "v"(g)
                 : "memory");
}

typedef __attribute__((address_space(4))) const uint32_t fmc_cu32;
typedef __attribute__((address_space(4))) const uint64_t fmc_cu64;
// Loads through the constant address space: wave-uniform addresses become
// scalar loads (memory written by earlier launches only).
FM_DEV uint32_t fmc_ld32(const void *p) { return *(fmc_cu32 *)p; }
FM_DEV uint64_t fmc_ld64(const void *p) { return *(fmc_cu64 *)p; }

// Slot k (wave-uniform) resolved with scalar loads: idx / weight, then the
// pool's blob address and bit width.  With rsel (fused routing) the expert
// and its probability come from LDS and the weight is p * winv.
FM_DEV FmSlot fmc_slot(const FmDecodeArgs &a, int k, const int *rsel = nullptr, const int *rp = nullptr,
                       float winv = 1.f) {
    if (!a.pool_mode || k >= a.K) return a.slot[k];
    FmSlot s;
    int e;
    float w;
    if (rsel) {
        e = __builtin_amdgcn_readfirstlane(rsel[k]);
        w = __int_as_float(__builtin_amdgcn_readfirstlane(rp[k])) * winv;
    } else {
        e = (int)fmc_ld32(a.idx + k);
        w = __uint_as_float(fmc_ld32(a.wdev + k));
    }
    if (e < 0 || (uint32_t)e >= a.pool_n) {
        s.valid = 0;
        s.bits = 4;
        s.weight = 0.f;
        return s;
    }
    const char *blob = (const char *)fmc_ld64(a.pool_blobs + e);
    const uintptr_t bp = (uintptr_t)(a.pool_bits + e);
    const int bits = (int)((fmc_ld32((const void *)(bp & ~(uintptr_t)3)) >> (8 * (bp & 3))) & 0xffu);
    const uint64_t *off = bits == 2 ? a.off2 : a.off4;
    s.gw = (const uint32_t *)(blob + off[0]);
    s.gs = (const uint16_t *)(blob + off[1]);
    s.gb = (const uint16_t *)(blob + off[2]);
    s.uw = (const uint32_t *)(blob + off[3]);
    s.us = (const uint16_t *)(blob + off[4]);
    s.ub = (const uint16_t *)(blob + off[5]);
    s.dw = (const uint32_t *)(blob + off[6]);
    s.ds = (const uint16_t *)(blob + off[7]);
    s.db = (const uint16_t *)(blob + off[8]);
    s.bits = bits;
    s.weight = w;
    s.valid = blob != nullptr && (bits == 2 || bits == 4);
    return s;
}
