// fm_decode_mfma.hip -- the decode step (K routed experts + shared expert) with
// every expert dot product on the matrix cores.
//
// Same contract as the eager kernel in fm_decode.hip (CMD3 of
// layer_forward.h:3895-3993: gate/up, SwiGLU, down, weighted combine into the
// residual, one launch), restructured so the packed codes feed
// v_mfma_f32_16x16x32_f16 directly:
//
//  * codes are the B operand (one row per lane column): a masked nibble with a
//    zero fp16 exponent field IS the subnormal code*2^-24 (code*2^-20 for the
//    field at bits 4-7), so one shift and four ANDs turn a packed word into
//    the operand (no conversion, no dot instructions);
//  * the input vector is the A operand, but only in the operand row m that
//    equals the group index mod 16 -- every other row is zero.  D[m][row] thus
//    accumulates, over 32 MFMAs, the 16 per-group dot products of 16 weight
//    rows separately, and the per-(row, group) scale/bias fold happens once per
//    16 groups:  acc_row += s_g * 2^24 * D[g mod 16][row] + b_g * sum(x_g).
//    In the D layout a lane holds four consecutive groups of one row, so the
//    fold reads 8-byte scale/bias runs.
//
// Work split (one 256-thread workgroup = 4 wavefronts, all resident):
//  A  block b < S*I/16: 16 gate/up rows of slot b/(I/16); wave w takes the
//     w-th 1024-code quarter of the row (H = 4096); the 4 partial gate/up
//     sums meet in LDS, the block applies SwiGLU and publishes 16 tagged
//     activations.
//  B  block b < S*H/64: 64 down rows of slot b/(H/64), 16 per wave, k = I.
//     The block waits for its slot's I tagged activations, then streams.
//  C  the blocks of the last slot also combine their 64 rows over all slots
//     in the slot order of cpu_vec_madd (layer_forward.h:1257, 1295-1305).
// Hand-off polls re-issue their loads back to back (no sleep between rounds:
// each round is a memory round trip; sleeping only added latency).
// Every wave issues all of its gate/up loads before computing, so that stream
// is in flight from the first microsecond; down-projection loads follow once
// the wave's own gate/up work is done.
#include "fm_decode.h"
#include "fm_mfma_dev.h"
#include "fm_route_dev.h"
#include "fm_route_cu.h"

#include <stdlib.h>

#ifndef FM_DX_MARK
#define FM_DX_MARK(n)
#endif

#define FMM_MAXS 136  // slots of one launch: 8 tokens x (16 routed + shared)
#define FMM_TAB 1024  // pools up to this many experts: the blob/bits tables are staged in LDS

template <int NSLOT>  // slot table entries (the one-pass instance needs few: keeps 3 blocks per CU)
struct __attribute__((aligned(16))) FmmLds {
    fm_h2 xq[2][FMM_GH][32];  // x as MFMA operand rows: [4-bit | 2-bit layout][group][32 pairs]
    fm_h2 aq[2][FMM_GI][32];  // the B slot's activations, same layouts
    fm_h2 zero[32];           // zero operand rows (128 B)
    float xsum[FMM_GH];       // per-group sums of x
    float xinv[FMM_GH];       // per-group 2^(24 - e): x operands carry x * 2^e
    float asum[FMM_GI];       // per-group sums of the activations
    float ainv[FMM_GI];       // per-group 2^(24 - e) of the activation operands
    union {
        float act[FMM_MAXI];            // staged activations (fp32)
        const char *tab[FMM_TAB / 2];   // prologue: pool blob table, first half
    };
    const char *tab2[FMM_TAB / 2];      // prologue: pool blob table, second half
    uint8_t tbits[FMM_TAB];             // prologue: pool bit widths
    float part[4][16][2];     // per-wave partial gate/up sums of the A rows
    float ylast[64];          // this block's rows of the last slot's y
    uint32_t tr[4][16 * FMM_TS];  // per-wave transpose buffers
    FmSlot sd[NSLOT];
};

// fm_pool_slot with the blob / bits tables read from their LDS copies.
FM_DEV FmSlot fm_pool_slot_tab(const FmDecodeArgs &a, int e, float w, const char *const *t1, const char *const *t2,
                               const uint8_t *tb) {
    FmSlot s;
    if (e < 0 || (uint32_t)e >= a.pool_n) {
        s.valid = 0;
        s.bits = 4;
        s.weight = 0.f;
        return s;
    }
    const char *blob = e < FMM_TAB / 2 ? t1[e] : t2[e - FMM_TAB / 2];
    const int bits = tb[e];
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



// Registers of one unit: 16 rows x 64 words per piece (4-bit: 2 pieces,
// 2-bit: 1), loaded row-contiguously, plus the lane's scale/bias runs.
struct FmmCodes {
    fm_u4 c[8];
};

// The code loads of fmm_issue alone (scales and biases loaded elsewhere),
// issued on every path: with !ok every lane reads the first 256 bytes of
// `dummy` instead, so the number of loads in flight never depends on a branch
// (the compiler's wait counts stay exact instead of falling back to "wait for
// everything").  bits must be 2 or 4 either way.
// NG (16 or 8): groups of the unit.  With 8 groups a 4-bit row run is one
// piece (4 loads) and a 2-bit one half a piece (lanes n >= 8 repeat lane n - 8).
template <int NG = 16>
FM_DEV void fmm_issue_codes(const uint32_t *W, int bits, uint32_t row0, uint32_t in_dim, uint32_t g0, bool ok,
                            FmmCodes &cd, int lane, const void *dummy, int pmask = 3) {
    const int n = lane & 15, kq = lane >> 4;
    const uint32_t G = in_dim / 64, wpg = 2 * bits, wpr = ok ? G * wpg : 0;
    if (!ok) {
        W = (const uint32_t *)dummy;
        row0 = g0 = 0;
    }
    // always 8 loads (4 with 8 groups): a 2-bit row piece is 4 of them, its
    // other 4 repeat the same addresses (cache hits) so the load count never
    // depends on bits
    const int nw = (NG == 8 && bits == 2) ? (n & 7) : n;
#pragma unroll
    for (int p = 0; p < NG / 8; p++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t row = row0 + 4 * j + kq;
            const uint32_t po = (ok && bits == 4) ? g0 * wpg + 64 * p : (ok ? g0 * wpg : 0);
            // pieces outside pmask read the dummy (same load count, cache hits)
            cd.c[4 * p + j] = fm_ldg_u4_nt(((pmask >> p) & 1) ? W + (size_t)row * wpr + po + 4 * nw
                                                               : (const uint32_t *)dummy);
        }
    }
}

// The scale / bias runs of fmm_issue (lane (n, kq): row row0 + n, groups
// g0 + 4 kq .. + 3), branch-free like fmm_issue_codes.
// With NG = 8 the lanes kq >= 2 hold no group of the unit: zero.
template <int NG = 16>
FM_DEV void fmm_issue_sb(const uint16_t *S, const uint16_t *B, uint32_t row0, uint32_t in_dim, uint32_t g0, bool ok,
                         fmm_u2 &sc, fmm_u2 &bi, int lane, const void *dummy) {
    const int n = lane & 15, kq = lane >> 4;
    const bool mine = ok && 4 * kq < NG;
    const size_t o = mine ? (size_t)(row0 + n) * (in_dim / 64) + g0 + 4 * kq : 0;
    sc = *(const FM_GLOBAL fmm_u2 *)(mine ? S + o : (const uint16_t *)dummy);
    bi = *(const FM_GLOBAL fmm_u2 *)(mine ? B + o : (const uint16_t *)dummy);
    if (NG == 8 && !mine) sc = bi = (fmm_u2){0u, 0u};
}

// Issue the loads of 16 rows x 16 groups (groups g0 .. g0+15) of one matrix.
// Load j of piece p: lane l reads row row0 + 4j + l/16, words 64p + 4(l%16)
// .. +3 of the unit -- every instruction covers four 256-byte row runs.  The
// scale/bias runs follow the MFMA layout: lane (n, kq) takes row row0 + n,
// groups g0 + 4kq .. g0 + 4kq + 3.
FM_DEV void fmm_issue(const uint32_t *W, const uint16_t *S, const uint16_t *B, int bits, uint32_t row0,
                      uint32_t in_dim, uint32_t g0, bool ok, FmmCodes &cd, fmm_u2 &sc, fmm_u2 &bi, int lane) {
    if (!ok) return;
    const int n = lane & 15, kq = lane >> 4;
    const uint32_t G = in_dim / 64;
    const uint32_t wpg = 2 * bits;  // words per group
    const uint32_t wpr = G * wpg;   // words per row
#pragma unroll
    for (int p = 0; p < 2; p++) {
        if (p == 1 && bits != 4) break;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t row = row0 + 4 * j + kq;
            cd.c[4 * p + j] = fm_ldg_u4_nt(W + (size_t)row * wpr + g0 * wpg + 64 * p + 4 * n);
        }
    }
    sc = *(const FM_GLOBAL fmm_u2 *)(S + (size_t)(row0 + n) * G + g0 + 4 * kq);
    bi = *(const FM_GLOBAL fmm_u2 *)(B + (size_t)(row0 + n) * G + g0 + 4 * kq);
}


// 32 MFMAs over 16 groups: D[m][row] += x_op[m] . codes.  Each piece passes
// through the wave's LDS transpose buffer T: written as loaded (row runs),
// read back so lane (n, kq) holds row n's words 16h + 4kq .. +3 (h = 0..3).
// 4-bit: word s of read h of piece p is MFMA (chunk 2p + h/2, i = 4(h%2) + s),
//        group 4c + 2(i/4) + kq/2 of the unit, word 4(kq%2) + i%4 of it;
// 2-bit: read h is chunk c = h: group 4c + kq, MFMA i uses word i/2, half i%2.
// The x operand row m carries group g0 + m and is non-zero only in the slot
// that holds that group.  The LDS x operand of step j+1 is read during step
// j; scheduling barriers keep the compiler from hoisting further reads.
template <int BITS, int NG = 16>  // NG = 8: groups 0..7 only (16 MFMAs)
FM_DEV void fmm_mma(const FmmCodes &cd, const fm_h2 *xq_grp0, const fm_h2 *zero, uint32_t *T, fmm_f4 &d0,
                    fmm_f4 &d1, int lane) {
    const int m = lane & 15, kq = lane >> 4;
    auto src_of = [&](int j) -> const fm_h2 * {
        const int c = j >> 3, i = j & 7;
        if constexpr (BITS == 4) {
            const bool on = (kq >> 1) == (m & 1) && c == (m >> 2) && (i >> 2) == ((m >> 1) & 1);
            return on ? xq_grp0 + 32 * m + 16 * (kq & 1) + 4 * (i & 3) : zero;
        } else {
            const bool on = kq == (m & 3) && c == (m >> 2);
            return on ? xq_grp0 + 32 * m + 4 * i : zero;
        }
    };
    if constexpr (BITS == 4) {
        // A lane's operand is non-zero in 4 of the 32 steps only, always with
        // pairs of its own group m: keep those 4 quads in registers and select
        // per step (no LDS operand traffic in the loop).
        fmm_h8 xv[4];
#pragma unroll
        for (int s = 0; s < 4; s++) xv[s] = fmm_lds_op(xq_grp0 + 32 * m + 16 * (kq & 1) + 4 * s);
        const fmm_h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
        const bool kq_on = (kq >> 1) == (m & 1);
#pragma unroll
        for (int p = 0; p < NG / 8; p++) {
#pragma unroll
            for (int j = 0; j < 4; j++) *(fm_u4 *)&T[(4 * j + kq) * FMM_TS + 4 * m] = cd.c[4 * p + j];
            fm_u4 v[4];
#pragma unroll
            for (int h = 0; h < 4; h++) v[h] = *(const fm_u4 *)&T[m * FMM_TS + 16 * h + 4 * kq];
#pragma unroll
            for (int jj = 0; jj < 16; jj++) {
                const int j = 16 * p + jj;
                const int c = j >> 3, i = j & 7;
                const bool on = kq_on && c == (m >> 2) && (i >> 2) == ((m >> 1) & 1);
                const fmm_h8 xo = on ? xv[i & 3] : z;
                const fmm_h8 co = fmm_codes<4>(fmm_comp(v[2 * (c & 1) + (i >> 2)], i & 3), 0);
                if (i & 1)
                    d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d1, 0, 0, 0);
                else
                    d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d0, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return;
    }
    constexpr int NP = BITS == 4 ? 2 : 1;
    fmm_h8 xo = fmm_lds_op(src_of(0));
#pragma unroll
    for (int p = 0; p < NP; p++) {
#pragma unroll
        for (int j = 0; j < 4; j++) *(fm_u4 *)&T[(4 * j + kq) * FMM_TS + 4 * m] = cd.c[4 * p + j];
        fm_u4 v[4];
#pragma unroll
        for (int h = 0; h < 4; h++) v[h] = *(const fm_u4 *)&T[m * FMM_TS + 16 * h + 4 * kq];
        constexpr int NJ = 2 * NG / NP;
#pragma unroll
        for (int jj = 0; jj < NJ; jj++) {
            const int j = p * NJ + jj;
            const int c = j >> 3, i = j & 7;
            fmm_h8 xn = xo;
            if (j + 1 < 32) xn = fmm_lds_op(src_of(j + 1));
            fmm_h8 co;
            if constexpr (BITS == 4)
                co = fmm_codes<4>(fmm_comp(v[2 * (c & 1) + (i >> 2)], i & 3), 0);
            else
                co = fmm_codes<2>(fmm_comp(v[c], i >> 1), i & 1);
            if (i & 1)
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d1, 0, 0, 0);
            else
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d0, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            xo = xn;
        }
    }
}

// fmm_mma<4, NG> with the x operand read from LDS: lanes whose row m carries
// the group of a block of 4 steps read their own 4 operand quads, the others
// a zero run (one address select per block instead of 4 v_cndmask a step; the
// next block's quads are read while the current block's MFMAs run).  For one
// wave alone (the last item's down rows, on the step's critical path) this
// measured 29 ns a step against 36 ns.  `zero` must hold 16 zero pairs.
// P0 .. P1 - 1: the pieces (8 groups each) computed.
template <int NG = 16, int P0 = 0, int P1 = NG / 8>
FM_DEV void fmm_mma_l4(const FmmCodes &cd, const fm_h2 *xq_grp0, const fm_h2 *zero, uint32_t *T, fmm_f4 &d0,
                       fmm_f4 &d1, int lane) {
    const int m = lane & 15, kq = lane >> 4;
    const bool kq_on = (kq >> 1) == (m & 1);
    const fm_h2 *own = xq_grp0 + 32 * m + 16 * (kq & 1);
    auto blk_src = [&](int blk) -> const fm_h2 * {
        const int c = blk >> 1, h = blk & 1;
        return (kq_on && c == (m >> 2) && h == ((m >> 1) & 1)) ? own : zero;
    };
    constexpr int NB = 4 * P1;  // blocks of 4 steps
    fmm_h8 xa[4], xb[4];
    {
        const fm_h2 *sp = blk_src(4 * P0);
#pragma unroll
        for (int s = 0; s < 4; s++) xa[s] = fmm_lds_op(sp + 4 * s);
    }
#pragma unroll
    for (int p = P0; p < P1; p++) {
#pragma unroll
        for (int j = 0; j < 4; j++) *(fm_u4 *)&T[(4 * j + kq) * FMM_TS + 4 * m] = cd.c[4 * p + j];
        fm_u4 v[4];
#pragma unroll
        for (int h = 0; h < 4; h++) v[h] = *(const fm_u4 *)&T[m * FMM_TS + 16 * h + 4 * kq];
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            const int blk = 4 * p + bb;
            if (blk + 1 < NB) {
                const fm_h2 *sp = blk_src(blk + 1);
#pragma unroll
                for (int s = 0; s < 4; s++) xb[s] = fmm_lds_op(sp + 4 * s);
            }
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int j = 4 * blk + s;
                const int c = j >> 3, i = j & 7;
                const fmm_h8 co = fmm_codes<4>(fmm_comp(v[2 * (c & 1) + (i >> 2)], i & 3), 0);
                if (i & 1)
                    d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s], co, d1, 0, 0, 0);
                else
                    d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s], co, d0, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int s = 0; s < 4; s++) xa[s] = xb[s];
        }
    }
}


// A slot descriptor read from LDS is the same in every lane: keep it in scalar registers.
FM_DEV FmSlot fmm_uniform(const FmSlot &v) {
    FmSlot r;
    const uint32_t *src = (const uint32_t *)&v;
    uint32_t *dst = (uint32_t *)&r;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(FmSlot) / 4); i++) dst[i] = __builtin_amdgcn_readfirstlane(src[i]);
    return r;
}

typedef __attribute__((address_space(4))) const FmDecodeArgs FmmCArgs;
// The launch arguments in the kernarg segment, opaque to the optimiser.
FM_DEV const FmDecodeArgs *fmm_args() {
    FmmCArgs *p = (FmmCArgs *)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return (const FmDecodeArgs *)p;
}

// MP (multi-pass): the grid is smaller than the work and blocks loop over
// items; the loop costs the compiler ~24 registers, so that instance runs two
// blocks per CU (no spills) while the one-pass instance keeps three.
template <bool MP>
__global__ __launch_bounds__(256, MP ? 2 : FMM_BLOCKS_PER_CU) void fm_decode_mfma_kernel(FmDecodeArgs a_) {
    const FmDecodeArgs &a = a_;
    __shared__ FmmLds<MP ? FMM_MAXS : FM_MAX_SLOTS> L;
    const int tid = threadIdx.x;
    const uint32_t H = a.hidden, I = a.inter;
    const uint32_t tilesA = I / 16, tilesB = H / 64;
    const int spt = a.spt;
    // Work items: item i is A tile i and B tile i (slot i / tiles).  The grid
    // is a whole number of slots' tiles and every block takes items b, b + grid,
    // ...: the items of one slot always run in the same pass, so a block only
    // ever waits for blocks that are resident in that pass (or done).
    const uint32_t nitems = (uint32_t)a.S * (tilesA > tilesB ? tilesA : tilesB);
    const uint32_t b0 = blockIdx.x;
    auto token_of = [&](uint32_t item) -> int {
        const uint32_t k = item / tilesA;
        return (int)((k < (uint32_t)a.S ? k : 0) / spt);
    };

    FM_DX_MARK(0);
    // this call's tag: loaded first, needed only after the prologue
    const uint32_t ep_ld = fm_epoch_load(a);
    // x first: thread t holds elements 16*(t%4) .. +15 of group t/4.  Loaded
    // before the slot lookup and the weights, so its latency overlaps theirs.
    fm_f4 xr[4];
    auto load_x = [&](uint32_t item) {
        const float *xp = a.x + (size_t)token_of(item) * H + 16 * tid;
#pragma unroll
        for (int j = 0; j < 4; j++) xr[j] = fm_ldg_f4(xp + 4 * j);
    };
    load_x(b0);
    // Slots of every token.  A pool of up to FMM_TAB experts has its blob/bits
    // tables staged in LDS together with idx / weights (independent loads, one
    // round trip) instead of the dependent chain idx -> table entry.
    const bool tab = a.pool_mode && a.pool_n <= FMM_TAB;
    const int sT = tid < a.S ? tid / spt : 0, sK = tid < a.S ? tid % spt : 0;
    const bool routed = tid < a.S && sK < a.K;
    int e_k = 0;
    float w_k = 0.f;
    if (a.pool_mode && b0 == 0) {
        for (int i = tid; i < a.ntok * a.K; i += 256) {
            const int e = a.idx[i];
            if (e < 0 || (uint32_t)e >= a.pool_n) atomicOr(a.err, FM_STATUS_BAD_EXPERT);  // skipped (invalid slot)
        }
    }
    if (tab) {
        if (routed) {
            e_k = a.idx[sT * a.K + sK];
            w_k = a.wdev[sT * a.K + sK];
        }
        for (uint32_t e = tid; e < a.pool_n; e += 256) {
            const char *p = (const char *)a.pool_blobs[e];
            if (e < FMM_TAB / 2)
                L.tab[e] = p;
            else
                L.tab2[e - FMM_TAB / 2] = p;
            L.tbits[e] = a.pool_bits[e];
        }
        __syncthreads();
        if (routed) {
            L.sd[tid] = fm_pool_slot_tab(a, e_k, w_k, L.tab, L.tab2, L.tbits);
        } else if (tid < a.S) {
            L.sd[tid] = a.slot[sK];
        }
    } else if (tid < a.S) {
        L.sd[tid] = fm_get_slot(a, sK, sT);
    }
    if (tid < 32) L.zero[tid] = fm_as_h2(0u);
    __syncthreads();
    const uint32_t ep = fm_epoch_tag(ep_ld);

    // gate/up codes of the current item: the multi-pass instance loads the
    // next item's during the current item's down phase (the registers are
    // free once the activations are published), so the activation wait and
    // the down rows of one pass overlap the gate/up latency of the next
    FmmCodes cg, cu;
    fmm_u2 sg = {0, 0}, bg = {0, 0}, su = {0, 0}, bu = {0, 0};
    for (uint32_t b = b0; b < nitems; b += gridDim.x) {
    // The arguments are re-read from the kernarg segment per item (scalar
    // loads): hoisted out of the loop they would all stay live in registers.
    const FmDecodeArgs &a = MP ? *fmm_args() : a_;
    // the thread index is made opaque per item too, so that no per-lane
    // address arithmetic is hoisted out of the loop
    int tid = threadIdx.x;
    if constexpr (MP) asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wv = tid >> 6, n = lane & 15, q = lane >> 4;
    const int spt = a.spt;
    const uint32_t H = a.hidden, I = a.inter, GI = I / 64, tilesA = I / 16, tilesB = H / 64;
    const bool hasA = b < (uint32_t)a.S * tilesA;
    const bool hasB = b < (uint32_t)a.S * tilesB;
    const int kA = hasA ? (int)(b / tilesA) : 0;
    const int kB = hasB ? (int)(b / tilesB) : 0;
    const int tokB = kB / spt;  // token of the B slot (the combine's token)
    const FmSlot sA = MP ? fmm_uniform(L.sd[kA]) : L.sd[kA];
    FmSlot sB;
    if constexpr (!MP) sB = L.sd[kB];
    const bool doA = hasA && sA.valid;
    // ---- this item's gate/up loads (multi-pass: issued during the previous item) ----
    const uint32_t rowA0 = (b % tilesA) * 16;
    FmmCodes cdn;
    fmm_u2 sdn = {0, 0}, bdn = {0, 0};
    if (!MP || b == b0) {
        fmm_issue(sA.gw, sA.gs, sA.gb, sA.bits, rowA0, H, 16 * wv, doA, cg, sg, bg, lane);
        fmm_issue(sA.uw, sA.us, sA.ub, sA.bits, rowA0, H, 16 * wv, doA, cu, su, bu, lane);
    }
    const uint32_t rowB0 = (b % tilesB) * 64 + 16 * wv;

    FM_DX_MARK(1);
    // ---- x operand rows in both layouts, and the group sums ----
    {
        const int g = tid >> 2, qq = tid & 3;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[4 * j] = xr[j].x;
            v[4 * j + 1] = xr[j].y;
            v[4 * j + 2] = xr[j].z;
            v[4 * j + 3] = xr[j].w;
        }
        // the group's operand scale 2^e (its 4 threads are adjacent lanes)
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
        // 4-bit words 2qq, 2qq+1: pair j of word p = (x_{8p+j}, x_{8p+4+j}) * (j odd ? 1/16 : 1)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float m = (j & 1) ? 0.0625f * f : f;
                L.xq[0][g][4 * (2 * qq + h) + j] = fm_pack_h2(v[8 * h + j] * m, v[8 * h + 4 + j] * m);
            }
        // 2-bit word qq: pair n = (x_n, x_{n+8}) / 4^(field position of code n)
        const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
        for (int n = 0; n < 8; n++) L.xq[1][g][8 * qq + n] = fm_pack_h2(v[n] * (mt[n] * f), v[8 + n] * (mt[n] * f));
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 4) s += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if (qq == 0) {
            L.xsum[g] = s;
            L.xinv[g] = fm_exp2i(24 - ex);
        }
    }
    __syncthreads();

    FM_DX_MARK(2);
    // ---- A: gate/up partials of 16 rows over this wave's 16 groups ----
    if (doA) {
        fmm_f4 g0 = {0, 0, 0, 0}, g1 = g0, u0 = g0, u1 = g0;
        const fm_h2 *xq = &L.xq[sA.bits == 4 ? 0 : 1][16 * wv][0];
        if (sA.bits == 4) {
            fmm_mma_l4(cg, xq, L.zero, L.tr[wv], g0, g1, lane);
            fmm_mma_l4(cu, xq, L.zero, L.tr[wv], u0, u1, lane);
        } else {
            fmm_mma<2>(cg, xq, L.zero, L.tr[wv], g0, g1, lane);
            fmm_mma<2>(cu, xq, L.zero, L.tr[wv], u0, u1, lane);
        }
        const float *gs4 = &L.xsum[16 * wv + 4 * q], *gi4 = &L.xinv[16 * wv + 4 * q];
        float pg = fmm_fold(g0 + g1, sg, bg, gs4, gi4);
        float pu = fmm_fold(u0 + u1, su, bu, gs4, gi4);
        pg = fmm_q_sum(pg);
        pu = fmm_q_sum(pu);
        if (lane < 16) {
            L.part[wv][n][0] = pg;
            L.part[wv][n][1] = pu;
        }
    }
    FM_DX_MARK(3);
    __syncthreads();
    if (doA && tid < 16) {
        const float g = (L.part[0][tid][0] + L.part[1][tid][0]) + (L.part[2][tid][0] + L.part[3][tid][0]);
        const float u = (L.part[0][tid][1] + L.part[1][tid][1]) + (L.part[2][tid][1] + L.part[3][tid][1]);
        fm_put_tagged(&a.act2[(size_t)kA * I + rowA0 + tid], fm_silu_mul(g, u), ep);
    }

    FM_DX_MARK(4);
    // Down-projection loads are issued only now: their data is useless before
    // the slot's activations exist, and issuing them early would only delay
    // other waves' gate/up data.
    if constexpr (MP) sB = fmm_uniform(L.sd[kB]);  // read only now: fewer registers live during A
    const bool doB = hasB && sB.valid;
    fmm_issue(sB.dw, sB.ds, sB.db, sB.bits, rowB0, I, 0, doB, cdn, sdn, bdn, lane);
    if constexpr (MP) {
        // the next item's x and gate/up rows, behind this item's down rows
        const uint32_t bn = b + gridDim.x;
        if (bn < nitems) {
            load_x(bn);
            const bool hasAn = bn < (uint32_t)a.S * tilesA;
            const int kAn = hasAn ? (int)(bn / tilesA) : 0;
            const FmSlot sAn = fmm_uniform(L.sd[kAn]);
            const bool doAn = hasAn && sAn.valid;
            const uint32_t rowAn = (bn % tilesA) * 16;
            fmm_issue(sAn.gw, sAn.gs, sAn.gb, sAn.bits, rowAn, H, 16 * wv, doAn, cg, sg, bg, lane);
            fmm_issue(sAn.uw, sAn.us, sAn.ub, sAn.bits, rowAn, H, 16 * wv, doAn, cu, su, bu, lane);
        }
    }
    // ---- B: stage the slot's activations, then 16 down rows per wave ----
    if (doB) {
        constexpr int MAXQ = FMM_MAXI / 256;
        uint64_t t[MAXQ];
        const uint64_t *src = a.act2 + (size_t)kB * I;
#pragma unroll
        for (int j = 0; j < MAXQ; j++) {
            const uint32_t i = j * 256 + tid;
            t[j] = i < I ? fm_get_tagged(src + i) : ((uint64_t)ep << 32);
        }
        uint32_t it = 0;
        do {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < MAXQ; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
            if (__all(ready)) break;
#pragma unroll
            for (int j = 0; j < MAXQ; j++) {
                const uint32_t i = j * 256 + tid;
                if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(src + i);
            }
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
#pragma unroll
        for (int j = 0; j < MAXQ; j++) {
            const uint32_t i = j * 256 + tid;
            if (i < I) L.act[i] = __uint_as_float((uint32_t)t[j]);
        }
    }
    __syncthreads();
    if (doB) {
        // per group (16 threads x 4 elements): sum, operand scale 2^e, and the
        // operand rows (2 pairs per thread)
        const int lay = sB.bits == 4 ? 0 : 1;
        for (uint32_t g = tid >> 4; g < GI; g += 16) {
            const float *ag = L.act + 64 * g + 4 * (tid & 15);
            float s = (ag[0] + ag[1]) + (ag[2] + ag[3]);
            float mx = fmaxf(fmaxf(fabsf(ag[0]), fabsf(ag[1])), fmaxf(fabsf(ag[2]), fabsf(ag[3])));
            s = fmm_row_sum(s);
            mx = fm_row16_max(mx);
            const int ex = fm_group_shift(mx);
            const float f = fm_exp2i(ex);
            if ((tid & 15) == 0) {
                L.asum[g] = s;
                L.ainv[g] = fm_exp2i(24 - ex);
            }
            fmm_build_pair(L.act + 64 * g, sB.bits, 2 * (tid & 15), f, &L.aq[lay][g][0]);
            fmm_build_pair(L.act + 64 * g, sB.bits, 2 * (tid & 15) + 1, f, &L.aq[lay][g][0]);
        }
    }
    __syncthreads();
    FM_DX_MARK(5);
    const bool last = hasB && a.mode == 0 && kB % spt == spt - 1;
    if (doB) {
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        const fm_h2 *aq = &L.aq[sB.bits == 4 ? 0 : 1][0][0];
        if (sB.bits == 4)
            fmm_mma_l4(cdn, aq, L.zero, L.tr[wv], d0, d1, lane);
        else
            fmm_mma<2>(cdn, aq, L.zero, L.tr[wv], d0, d1, lane);
        float y = fmm_fold(d0 + d1, sdn, bdn, &L.asum[4 * q], &L.ainv[4 * q]);
        y = fmm_q_sum(y);
        const uint32_t row = rowB0 + n;
        if (lane < 16) {
            if (a.mode == 1)
                a.expert_out[(size_t)kB * H + row] = y;
            else if (!last)
                fm_put_tagged(&a.y2[(size_t)kB * H + row], y, ep);
            else
                L.ylast[16 * wv + n] = y;
        }
    } else if (last && lane < 16) {
        L.ylast[16 * wv + n] = 0.f;
    }

    FM_DX_MARK(6);
    // ---- C: the blocks of a token's last slot combine their 64 rows over the token's slots ----
    if (last) {
        __syncthreads();
        if (wv == 0) {
            // one wavefront gathers every other slot's y for the 64 rows with
            // one batch of coherent loads, re-polling only what is not ready
            const uint32_t row = (b % tilesB) * 64 + lane;
            const int k0 = tokB * spt;  // the token's first slot
            uint64_t t[FM_MAX_SLOTS - 1];
#pragma unroll
            for (int k = 0; k < FM_MAX_SLOTS - 1; k++)
                t[k] = (k < spt - 1 && L.sd[k0 + k].valid) ? fm_get_tagged(&a.y2[(size_t)(k0 + k) * H + row])
                                                         : ((uint64_t)ep << 32);
            uint32_t it = 0;
            do {
                bool ready = true;
#pragma unroll
                for (int k = 0; k < FM_MAX_SLOTS - 1; k++) ready &= (uint32_t)(t[k] >> 32) == ep;
                if (__all(ready)) break;
#pragma unroll
                for (int k = 0; k < FM_MAX_SLOTS - 1; k++)
                    if ((uint32_t)(t[k] >> 32) != ep) t[k] = fm_get_tagged(&a.y2[(size_t)(k0 + k) * H + row]);
            } while (++it < FM_SPIN_MAX);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
            const float sw =
                (a.has_shared || a.shared_y) ? (a.shared_score ? fm_sigmoid(a.shared_score[tokB]) : a.shared_w_host)
                                             : 0.f;
            const float yl = L.ylast[lane];
            float moe = 0.f;
#pragma unroll
            for (int k = 0; k < FM_MAX_SLOTS; k++) {
                if (k < a.K && L.sd[k0 + k].valid) {
                    const float yk = k == spt - 1 ? yl : __uint_as_float((uint32_t)t[k < FM_MAX_SLOTS - 1 ? k : 0]);
                    moe = __fadd_rn(moe, __fmul_rn(L.sd[k0 + k].weight, yk));
                }
            }
            const size_t orow = (size_t)tokB * H + row;
            float o = a.h_mid ? __fadd_rn(a.h_mid[orow], moe) : moe;
            if (a.has_shared) o = __fadd_rn(o, __fmul_rn(sw, yl));
            else if (a.shared_y) o = __fadd_rn(o, __fmul_rn(sw, a.shared_y[orow]));
            a.out[orow] = o;
            if (a.out_bf16) a.out_bf16[orow] = fm_f32_to_bf16(o);
            if (a.norm_w) {
                // next layer's input RMS norm (cpu_kernels.h:235-246): every
                // combining block publishes the sum of squares of its 64 rows,
                // then reduces all of them in the same fixed order
                const uint32_t j = b % tilesB;
                const float sq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fm_lane_sum<64>(o * o))));
                if (lane == 0) fm_put_tagged(&a.ss2[j], sq, ep);
                uint64_t v = lane < (int)tilesB ? fm_get_tagged(&a.ss2[lane]) : ((uint64_t)ep << 32);
                uint32_t it = 0;
                while (!__all((uint32_t)(v >> 32) == ep) && ++it < FM_SPIN_MAX) {
                    if ((uint32_t)(v >> 32) != ep) v = fm_get_tagged(&a.ss2[lane]);
                }
                if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
                const float part = lane < (int)tilesB ? __uint_as_float((uint32_t)v) : 0.f;
                const float tot = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fm_lane_sum<64>(part))));
                const float inv = 1.0f / sqrtf(tot / (float)H + a.norm_eps);
                a.normed[row] = o * inv * fm_bf16_to_f32(a.norm_w[row]);
            }
        }
    }
    FM_DX_MARK(7);
    // the ends of the hand-off chains: combining items (mode 0) or every down
    // item (mode 1, per-slot outputs) count towards publishing the next epoch
    if (tid == 0 && (a.mode == 0 ? last : hasB))
        fm_epoch_finish(a, ep, (uint32_t)(a.mode == 0 ? a.ntok : a.S) * tilesB);
    __syncthreads();  // LDS of this item is reused by the next
    if constexpr (!MP) break;
    }
}

// ------------------------------------------------ one workgroup per CU ----
// The single-token step with ONE 768-thread workgroup per CU holding up to
// three work items (item = A tile + B tile of one slot, as above; item i of
// workgroup g is g + i * grid).  A CU's vector memory requests are served in
// issue order, so one workgroup per CU decides that order itself:
//   x (once per CU, not once per item), then every item's gate/up rows (the
//   issue itself blocks while the CU's request queue is full: the last item's
//   waves finish issuing ~9 us in), then each item's down rows as soon as its
//   own activations are published -- the last item's copied into LDS by item
//   0's waves at that point, ahead of the other items' down rows.
// The gate/up bytes thus arrive first everywhere, and the down bytes stream
// while the slots' activations are still being completed.  Slot descriptors come
// from wave-uniform scalar loads (idx -> pool tables), which do not queue
// behind the vector stream.  The four waves of an item synchronise through an
// LDS counter, so items progress independently of each other.
#define FMC_NG 3                  // items per workgroup (FMC_THREADS = 256 FMC_NG)
static_assert(FMC_THREADS == 256 * FMC_NG, "three 4-wave items per workgroup");

struct __attribute__((aligned(16))) FmcItem {
    fm_h2 aq[2][FMM_GI][32];      // the item's activations as MFMA operand rows
    float asum[FMM_GI];
    float ainv[FMM_GI];
    float act[FMM_MAXI];          // staged activations (fp32)
    float part[4][16][2];         // per-wave partial gate/up sums
    float ylast[64];              // combine: this item's rows of the last slot's y
    uint32_t tr[4][16 * FMM_TS];  // per-wave transpose buffers
    uint32_t scl[4][16][FMM_GH / 2];  // gate/up scales and biases of the 16 rows (bf16 pairs)
    float cw[FM_MAX_SLOTS];       // combine: every slot's weight
    float sw;                     // combine: the shared expert's sigmoid gate
    uint32_t cvalid;              // combine: bit k = slot k is valid
    uint32_t sync;                // the item's 4-wave barrier counter
};

#ifndef FMC_DN_HELP
#define FMC_DN_HELP 1  // item 0's waves take half of the last item's down MMA (see fm_decode_cu_kernel)
#endif

#ifndef FMC_DN_LDS
#define FMC_DN_LDS 1  // the last item's down rows copied into LDS early (see fm_decode_cu_kernel)
#endif


struct __attribute__((aligned(16))) FmcLds {
    fm_h2 xq[2][FMM_GH][32];
    fm_h2 zero[32];
    float xsum[FMM_GH];
    float xinv[FMM_GH];
    uint32_t xready;              // count of item 0's waves that built the x operands
    uint32_t dn_ready;            // count of item 0's waves whose copy of the last item's down rows landed
    uint32_t hlp_go;              // the last item's activation operands are built (its helpers may start)
    uint32_t hlp_done[4];         // helper wave w has written hy[w]
    float hy[4][16];              // helper wave w: groups 8..15 of the last item's wave-w down rows
    FmcItem it[FMC_NG];
    union {
        // the routing scratch is dead once every wave has passed the
        // prologue; the down-row copy starts later (after item 0's
        // activations), and never on the CU whose idle wave group writes
        // the slot-order outputs (it holds no last item)
        uint32_t dn[4][16 * FMM_MAXI / 8];     // last item: each wave's 16 down rows (4-bit: 128 words a row)
        FmcRoute rt;
    };
    uint16_t dsb[4][2][16 * FMM_GI];       // ... and their scales / biases
    int rsel[FM_MAX_K];           // fused routing: expert of routed slot k (descending probability)
    int rp[FM_MAX_K];             // ... and its probability bits
};


// Slot of item position q when the combining slot S - 1 sits at position cs.
FM_DEV int fmc_slot_at(int q, int S, int cs) { return q == cs ? S - 1 : (q == S - 1 ? cs : q); }

// Barrier of the 4 waves of one item: an LDS counter that only grows (target
// += 4 per use).  Waits on LDS operations only -- the item's weight loads stay
// in flight across it.
FM_DEV void fmc_item_sync(uint32_t *ctr, uint32_t &target) {
    target += 4;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
        __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");
}

// NG = input groups of one wave's share of a row (16: hidden 4096 / inter 1024;
// 8: hidden 2048 / inter 512).  hidden = 256 NG, inter = hidden / 4, so the
// gate/up tiles (16 rows) and the down tiles (64 rows) of a slot pair up.
template <int NG, bool RT>  // RT: routing fused into the launch (FmDecodeArgs::route_logits)
__global__ __launch_bounds__(FMC_THREADS, 1) void fm_decode_cu_kernel(FmDecodeArgs a) {
    __shared__ FmcLds L;
    const int tid = threadIdx.x, lane = tid & 63;
    const int grp = __builtin_amdgcn_readfirstlane(tid >> 8);  // the wave's item
    const int wv = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    const int gt = tid & 255;  // thread within the item
    const int n = lane & 15, q = lane >> 4;
    constexpr uint32_t H = 256 * NG, I = 64 * NG, GI = NG, GH = 4 * NG, TILES = 4 * NG;  // TILES == I / 16
    static_assert(H <= FMM_H && I <= FMM_MAXI, "LDS is sized for hidden 4096 / inter 1024");
    const uint32_t item = blockIdx.x + gridDim.x * (uint32_t)grp;
    const bool has = item < (uint32_t)a.S * TILES;
    // Item positions q = item / TILES hold slot q, except that the combining
    // slot S - 1 trades places with position S - grid / TILES: with m =
    // (S TILES - 1) / grid, the workgroups from S TILES - m grid on hold m
    // items (the others m + 1), and that position is their item m - 1.  They
    // finish their own streams first, so the combine there waits only for the
    // other slots' outputs (measured with m = 2: 1 us off the config-2 step;
    // with m = 1, where that item is the CU's first, 0.5 us slower: kept off;
    // compiled for the 16-group instance only, the 8-group one lost 0.45 us
    // to the extra code even with the placement off)
    const uint32_t STI = (uint32_t)a.S * TILES, G = gridDim.x, m = (STI - 1) / G;
    const int cs = (NG == 16 && a.mode == 0 && m >= 2 && G % TILES == 0 && STI + TILES <= (m + 1) * G) ? a.S - (int)(G / TILES)
                                                                                          : a.S - 1;
    const int k = has ? fmc_slot_at((int)(item / TILES), a.S, cs) : 0;  // the item's slot
    const uint32_t tile = item % TILES;

    FM_DX_MARK(0);
    // counters first (no load is in flight yet, so this barrier is cheap)
    if (tid < FMC_NG) L.it[tid].sync = 0;
    if (tid < 4) L.hlp_done[tid] = 0;
    if (RT && tid < FMC_THREADS / 8) L.rt.ck[tid] = 0;
    if (tid == 0) {
        L.xready = L.dn_ready = L.hlp_go = 0;
        if constexpr (RT) {
            L.rt.ncand = L.rt.pconv = 0;  // fused routing: candidate count, p written into pb
            L.rt.vk = -1;                 // ... and the first probability left out (none)
        }
    }
    __syncthreads();
    const uint32_t ep_ld = fm_epoch_load(a);
    constexpr bool fused = RT;
    float lgq[FMC_THREADS / 64];
    uint32_t etab = 0;  // exp table in lanes (fm_expf_lanes), loaded with the logits
    if constexpr (RT) {
        etab = fm_expf_lanes_load();
#pragma unroll
        for (int q = 0; q < FMC_THREADS / 64; q++)
            lgq[q] = 64 * q + lane < a.route_E ? a.route_logits[64 * q + lane] : -INFINITY;
    }
    // x: every wave loads elements 16 t .. 16 t + 15 of its item-relative
    // thread t (items 1 and 2 hit the lines item 0 brings into the CU's
    // cache); item 0 turns them into operand rows below
    fm_f4 xr[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xr[j] = fm_ldg_f4(a.x + 16 * (gt < (int)GH * 4 ? gt : 0) + 4 * j);
    float winv = 1.f;
    if constexpr (RT) winv = fmc_route(a, L, lgq, etab);
    if (fused && blockIdx.x == gridDim.x - 1 && grp == FMC_NG - 1 && wv == 0) {
        // the idle wave group of the last CU, right after the routing (the
        // launch guarantees it holds no item, so its CU makes no down-row
        // copy over the routing scratch):
        // cpu_topk's slot order by serial replay, then cpu_normalize_weights
        // (sequential sum over the slots) -- bit-equal to fm_route_kernel
        // (issue priority raised: the replay is a long dependent chain that
        // would otherwise queue behind the MFMA waves sharing its SIMD)
        __builtin_amdgcn_s_setprio(3);
        // p with cpu_softmax's sum (index order), bit-equal to the reference:
        // scaled inside the replay unless the prologue already wrote p
        const float pinv = L.rt.pconv ? 0.f : 1.0f / fm_serial_sum((const float *)L.rt.pb, a.route_E);
        FM_DX_MARK(13);
        fm_topk_serial(L.rt.pb, a.route_E, a.K, L.rt, pinv);
        FM_DX_MARK(14);
        __builtin_amdgcn_s_setprio(0);
        fm_wave_lds_sync();
        if (lane < a.K) {
            float sm = 0.f;
            for (int kk = 0; kk < a.K; kk++) sm += L.rt.s_val[kk];
            const float v = L.rt.s_val[lane];
            a.route_idx[lane] = L.rt.s_id[lane];
            a.route_w[lane] = sm > 0.f ? v * (1.0f / sm) : v;
        }
    }
    const int *rsel = RT ? L.rsel : nullptr;
    const FmSlot s = fmc_slot(a, k, rsel, L.rp, winv);
    const bool doA = has && s.valid;
    // The last item's down rows: item 0's waves copy them into LDS right
    // after publishing their own activations, so they queue behind the gate/up
    // stream instead of behind the last item's own activation wait.
    const uint32_t item_l = blockIdx.x + gridDim.x * (uint32_t)(FMC_NG - 1);
    const bool has_l = item_l < (uint32_t)a.S * TILES;
    const int k_l = has_l ? fmc_slot_at((int)(item_l / TILES), a.S, cs) : 0;
    // (the 8-group instance only: with the combining slot on the two-item CUs
    // the 16-group step measured 0.2 us faster without the copy)
    constexpr bool DNL = FMC_DN_LDS && NG == 8;
    // The last item's down MMA (on the step's critical path: its activations
    // arrive last) is split with item 0's waves, idle by then: item 0's wave w
    // computes groups 8..15 of the last item's wave-w rows from codes it loads
    // right after its own down rows, and hands the partial sums over in LDS.
    // Only for 4-bit slots (one wave per SIMD becomes two).
    constexpr bool HLP = FMC_DN_HELP && NG == 16;
    const FmSlot s_l = ((DNL || HLP) && grp == 0) ? fmc_slot(a, k_l, rsel, L.rp, winv) : s;
    const bool help0 = HLP && grp == 0 && has_l && s_l.valid && s_l.bits == 4;
    const bool help2 = HLP && grp == FMC_NG - 1 && doA && s.bits == 4;
    const bool dn_lds = DNL && (grp == 0 ? has_l && s_l.valid : (grp == FMC_NG - 1 && doA));
    // Every gate/up load of the item.  Loads issue in order and block while
    // the CU's request queue is full, so a wave issues its down rows only
    // after its activations are published (a blocked issue would hold back
    // the gate/up compute behind it).
    const uint32_t rowA0 = tile * 16, rowB0 = tile * 64 + 16 * wv;
    FmmCodes cg, cu, cdn;
    fmm_u2 sdn = {0, 0}, bdn = {0, 0}, scl[4] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
    const int bits = doA ? s.bits : 4;
    fmm_issue_codes<NG>(s.gw, bits, rowA0, H, NG * wv, doA, cg, lane, a.x);
    fmm_issue_codes<NG>(s.uw, bits, rowA0, H, NG * wv, doA, cu, lane, a.x);
    // the tile's gate/up scales and biases: 16 rows x 64 groups = 2 KB per
    // array, contiguous; wave wv loads rows 4 wv .. 4 wv + 3 of each (full
    // lines) and the item shares them through LDS
    {
        const uint16_t *arr[4] = {s.gs, s.gb, s.us, s.ub};
#pragma unroll
        for (int j = 0; j < 4; j++)
            scl[j] = *(const FM_GLOBAL fmm_u2 *)((doA && lane < (int)GH) ? arr[j] + (size_t)(rowA0 + 4 * wv) * GH + 4 * lane
                                                                         : (const uint16_t *)a.x);
    }
    FM_DX_MARK(1);
    const bool last = has && a.mode == 0 && k == a.S - 1;
    if (last && wv == 0) {
        // the combine's slot weights, fetched now (scalar loads) so that the
        // combine itself waits for nothing but the other slots' outputs
        uint32_t vm = 0;
#pragma unroll
        for (int kk = 0; kk < FM_MAX_SLOTS; kk++) {
            if (kk < a.S) {
                const FmSlot sk = fmc_slot(a, kk, rsel, L.rp, winv);
                if (lane == 0) L.it[grp].cw[kk] = sk.weight;
                vm |= sk.valid ? 1u << kk : 0u;
            }
        }
        if (lane == 0) L.it[grp].cvalid = vm;
        // the shared expert's gate, off the combine's critical path
        const float swv = (a.has_shared || a.shared_y)
                              ? (a.shared_score ? fm_sigmoid(a.shared_score[0]) : a.shared_w_host)
                              : 0.f;
        if (lane == 0) L.it[grp].sw = swv;
    }
    // item 0 turns x into MFMA operand rows (both layouts), group sums and
    // scales; the other items wait for them on an LDS flag, not a barrier
    if (grp == 0) {
        if (tid < 32) L.zero[tid] = fm_as_h2(0u);
        const int g = tid >> 2, qq = tid & 3;
        const bool gok = g < (int)GH;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[4 * j] = xr[j].x;
            v[4 * j + 1] = xr[j].y;
            v[4 * j + 2] = xr[j].z;
            v[4 * j + 3] = xr[j].w;
        }
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float m = (j & 1) ? 0.0625f * f : f;
                if (gok) L.xq[0][g][4 * (2 * qq + h) + j] = fm_pack_h2(v[8 * h + j] * m, v[8 * h + 4 + j] * m);
            }
        const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
        for (int n2 = 0; n2 < 8; n2++)
            if (gok) L.xq[1][g][8 * qq + n2] = fm_pack_h2(v[n2] * (mt[n2] * f), v[8 + n2] * (mt[n2] * f));
        float sm = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
        sm += __shfl_xor(sm, 1, 64);
        sm += __shfl_xor(sm, 2, 64);
        if (qq == 0 && gok) {
            L.xsum[g] = sm;
            L.xinv[g] = fm_exp2i(24 - ex);
        }
    }
    {
        uint32_t xr_target = 0;
        if (grp == 0) {
            fmc_item_sync(&L.xready, xr_target);  // item 0's 4 waves have written the operands
        } else {
            while (__hip_atomic_load(&L.xready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 4)
                __builtin_amdgcn_s_sleep(1);
            asm volatile("" ::: "memory");
        }
    }
    const uint32_t ep = fm_epoch_tag(ep_ld);
    FmcItem &T = L.it[grp];
    uint32_t phase = 0;
    FM_DX_MARK(2);

    // ---- A: gate/up partials of 16 rows over this wave's 16 groups ----
    if (doA) {
        fmm_f4 g0 = {0, 0, 0, 0}, g1 = g0, u0 = g0, u1 = g0;
        const fm_h2 *xq = &L.xq[s.bits == 4 ? 0 : 1][NG * wv][0];
        if (s.bits == 4 && grp == FMC_NG - 1) {
            // the last item's gate/up MMA (its data arrives last) with the x
            // operand from LDS: shorter per step when it runs alone on a SIMD
            fmm_mma_l4<NG>(cg, xq, L.zero, T.tr[wv], g0, g1, lane);
            fmm_mma_l4<NG>(cu, xq, L.zero, T.tr[wv], u0, u1, lane);
        } else if (s.bits == 4) {
            fmm_mma<4, NG>(cg, xq, L.zero, T.tr[wv], g0, g1, lane);
            fmm_mma<4, NG>(cu, xq, L.zero, T.tr[wv], u0, u1, lane);
        } else {
            fmm_mma<2, NG>(cg, xq, L.zero, T.tr[wv], g0, g1, lane);
            fmm_mma<2, NG>(cu, xq, L.zero, T.tr[wv], u0, u1, lane);
        }
        // scale runs: GH / 4 lanes per row (4 groups = 2 words each)
        if (lane < (int)GH) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                *(fmm_u2 *)&T.scl[j][4 * wv + lane / (GH / 4)][2 * (lane % (GH / 4))] = scl[j];
        }
        fmc_item_sync(&T.sync, phase);
        // lane (row n, q) folds groups NG wv + 4 q .. + 3 of row n (NG = 8: q < 2 only)
        const bool qok = 4 * q < NG;
        const int c0 = (NG / 2) * wv + 2 * (qok ? q : 0);
        const fmm_u2 sg = *(const fmm_u2 *)&T.scl[0][n][c0], bg = *(const fmm_u2 *)&T.scl[1][n][c0];
        const fmm_u2 su = *(const fmm_u2 *)&T.scl[2][n][c0], bu = *(const fmm_u2 *)&T.scl[3][n][c0];
        const float *gs4 = &L.xsum[NG * wv + 4 * (qok ? q : 0)], *gi4 = &L.xinv[NG * wv + 4 * (qok ? q : 0)];
        float pg = qok ? fmm_fold(g0 + g1, sg, bg, gs4, gi4) : 0.f;
        float pu = qok ? fmm_fold(u0 + u1, su, bu, gs4, gi4) : 0.f;
        pg = fmm_q_sum(pg);
        pu = fmm_q_sum(pu);
        if (lane < 16) {
            T.part[wv][n][0] = pg;
            T.part[wv][n][1] = pu;
        }
    }
    FM_DX_MARK(3);
    fmc_item_sync(&T.sync, phase);
    if (doA && gt < 16) {
        const float g = (T.part[0][gt][0] + T.part[1][gt][0]) + (T.part[2][gt][0] + T.part[3][gt][0]);
        const float u = (T.part[0][gt][1] + T.part[1][gt][1]) + (T.part[2][gt][1] + T.part[3][gt][1]);
        fm_put_tagged(&a.act2[(size_t)k * I + rowA0 + gt], fm_silu_mul(g, u), ep);
    }
    if (dn_lds && grp == 0) {
        // wave wv copies the last item's wave wv rows: 16 rows x (NG groups x
        // 2 bits words), contiguous, then their scales and biases (NG x 2
        // bytes a row)
        const int bl = s_l.bits;
        const uint32_t rows0 = (item_l % TILES) * 64 + 16 * wv, wpr = NG * 2 * bl;
        const char *src = (const char *)(s_l.dw + (size_t)rows0 * wpr);
        const int runs = 16 * wpr * 4 / 1024;  // 1 KB per instruction
        for (int r = 0; r < runs; r++) fmc_dma16(&L.dn[wv][256 * r], src + 1024 * r + 16 * lane);
        if (lane < NG * 2) {  // 16 rows x NG bf16 = 32 NG bytes
            fmc_dma16(&L.dsb[wv][0][0], (const char *)(s_l.ds + (size_t)rows0 * NG) + 16 * lane);
            fmc_dma16(&L.dsb[wv][1][0], (const char *)(s_l.db + (size_t)rows0 * NG) + 16 * lane);
        }
    }
    // the down rows (queue behind every gate/up request of the CU); the last
    // item's come from LDS (its loads read the dummy, so the count of loads in
    // flight is the same on every path)
    const bool dn_glob = doA && !(dn_lds && grp == FMC_NG - 1);
    fmm_issue_codes<NG>(s.dw, bits, rowB0, I, 0, dn_glob, cdn, lane, a.x, help2 ? 1 : 3);
    fmm_issue_sb<NG>(s.ds, s.db, rowB0, I, 0, dn_glob, sdn, bdn, lane, a.x);
    // item 0's share of the last item's down rows (piece 1: groups 8..15)
    FmmCodes chl;
    fmm_u2 sdh = {0, 0}, bdh = {0, 0};
    if constexpr (HLP) {
        const uint32_t rowBl = (item_l % TILES) * 64 + 16 * wv;
        fmm_issue_codes<NG>(s_l.dw, 4, rowBl, I, 0, help0, chl, lane, a.x, 2);
        fmm_issue_sb<NG>(s_l.ds, s_l.db, rowBl, I, 0, help0, sdh, bdh, lane, a.x);
    }
    if (dn_lds && grp == 0) {
        // the copy is older than the NG / 2 + 2 loads just issued
        static_assert(NG / 2 + 2 <= 15, "vmcnt immediate");
        __builtin_amdgcn_s_waitcnt((NG / 2 + 2) | (0x7 << 4) | (0xF << 8));
        if (lane == 0) __hip_atomic_fetch_add(&L.dn_ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    FM_DX_MARK(4);

    // ---- B: the slot's activations (every A tile of the slot), then 16 down rows per wave ----
    if (doA) {
        constexpr int MAXQ = I / 256;
        uint64_t t[MAXQ];
        const uint64_t *src = a.act2 + (size_t)k * I;
#pragma unroll
        for (int j = 0; j < MAXQ; j++) t[j] = fm_get_tagged(src + j * 256 + gt);
        uint32_t it = 0;
        do {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < MAXQ; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
            if (__all(ready)) break;
#pragma unroll
            for (int j = 0; j < MAXQ; j++)
                if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(src + j * 256 + gt);
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
#pragma unroll
        for (int j = 0; j < MAXQ; j++) T.act[j * 256 + gt] = __uint_as_float((uint32_t)t[j]);
    }
    fmc_item_sync(&T.sync, phase);
    if (doA && gt < 16 * (int)GI) {
        // per group (16 threads x 4 elements): sum, operand scale 2^e, operand rows
        const int lay = s.bits == 4 ? 0 : 1;
        const uint32_t g = gt >> 4;
        const float *ag = T.act + 64 * g + 4 * (gt & 15);
        float sm = (ag[0] + ag[1]) + (ag[2] + ag[3]);
        float mx = fmaxf(fmaxf(fabsf(ag[0]), fabsf(ag[1])), fmaxf(fabsf(ag[2]), fabsf(ag[3])));
        sm = fmm_row_sum(sm);
        mx = fm_row16_max(mx);
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
        if ((gt & 15) == 0) {
            T.asum[g] = sm;
            T.ainv[g] = fm_exp2i(24 - ex);
        }
        fmm_build_pair(T.act + 64 * g, s.bits, 2 * (gt & 15), f, &T.aq[lay][g][0]);
        fmm_build_pair(T.act + 64 * g, s.bits, 2 * (gt & 15) + 1, f, &T.aq[lay][g][0]);
    }
    fmc_item_sync(&T.sync, phase);
    FM_DX_MARK(5);
    if (help2 && wv == 0 && lane == 0) __hip_atomic_fetch_add(&L.hlp_go, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (dn_lds && grp == FMC_NG - 1) {
        // this item's down rows from LDS, in the lane layout of fmm_issue_codes / fmm_issue_sb
        uint32_t it = 0;
        while (__hip_atomic_load(&L.dn_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 4 && ++it < FM_SPIN_MAX)
            __builtin_amdgcn_s_sleep(1);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        asm volatile("" ::: "memory");
        const uint32_t wpr = NG * 2 * s.bits;
        const int nw = (NG == 8 && s.bits == 2) ? (n & 7) : n;
#pragma unroll
        for (int p = 0; p < NG / 8; p++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t po = s.bits == 4 ? 64 * p : 0;
                cdn.c[4 * p + j] = *(const fm_u4 *)&L.dn[wv][(4 * j + q) * wpr + po + 4 * nw];
            }
        if (4 * q < NG) {
            sdn = *(const fmm_u2 *)&L.dsb[wv][0][n * NG + 4 * q];
            bdn = *(const fmm_u2 *)&L.dsb[wv][1][n * NG + 4 * q];
        } else {
            sdn = bdn = (fmm_u2){0u, 0u};
        }
    }
    if (doA) {
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        const fm_h2 *aq = &T.aq[s.bits == 4 ? 0 : 1][0][0];
        if (help2)
            fmm_mma_l4<NG, 0, 1>(cdn, aq, L.zero, T.tr[wv], d0, d1, lane);
        else if (s.bits == 4)
            fmm_mma_l4<NG>(cdn, aq, L.zero, T.tr[wv], d0, d1, lane);
        else
            fmm_mma<2, NG>(cdn, aq, L.zero, T.tr[wv], d0, d1, lane);
        const bool qok = 4 * q < NG && !(help2 && q >= 2);
        float y = qok ? fmm_fold(d0 + d1, sdn, bdn, &T.asum[4 * (qok ? q : 0)], &T.ainv[4 * (qok ? q : 0)]) : 0.f;
        y = fmm_q_sum(y);  // with the helper: (q0 + q1) here, (q2 + q3) from it -- the same sum
        if (help2) {
            uint32_t it = 0;
            while (__hip_atomic_load(&L.hlp_done[wv], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0 &&
                   ++it < FM_SPIN_MAX)
                __builtin_amdgcn_s_sleep(1);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
            asm volatile("" ::: "memory");
            y += L.hy[wv][n];
        }
        const uint32_t row = rowB0 + n;
        if (lane < 16) {
            if (a.mode == 1)
                a.expert_out[(size_t)k * H + row] = y;
            else if (!last)
                fm_put_tagged(&a.y2[(size_t)k * H + row], y, ep);
            else
                T.ylast[16 * wv + n] = y;
        }
    } else if (last && lane < 16) {
        T.ylast[16 * wv + n] = 0.f;
    }
    FM_DX_MARK(6);

    // ---- C: the items of the last slot combine their 64 rows over every slot ----
    if (last) {
        fmc_item_sync(&T.sync, phase);
        if (wv == 0) {
            const uint32_t row = tile * 64 + lane;
            const int spt = a.S;
            // every slot's weight and validity, fetched at the start
            const uint32_t cv = T.cvalid;
            uint64_t t[FM_MAX_SLOTS - 1];
#pragma unroll
            for (int kk = 0; kk < FM_MAX_SLOTS - 1; kk++)
                t[kk] = (kk < spt - 1 && ((cv >> kk) & 1u)) ? fm_get_tagged(&a.y2[(size_t)kk * H + row])
                                                            : ((uint64_t)ep << 32);
            uint32_t it = 0;
            do {
                bool ready = true;
#pragma unroll
                for (int kk = 0; kk < FM_MAX_SLOTS - 1; kk++) ready &= (uint32_t)(t[kk] >> 32) == ep;
                if (__all(ready)) break;
#pragma unroll
                for (int kk = 0; kk < FM_MAX_SLOTS - 1; kk++)
                    if ((uint32_t)(t[kk] >> 32) != ep) t[kk] = fm_get_tagged(&a.y2[(size_t)kk * H + row]);
            } while (++it < FM_SPIN_MAX);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
            const float sw = T.sw;
            const float yl = T.ylast[lane];
            float moe = 0.f;
#pragma unroll
            for (int kk = 0; kk < FM_MAX_SLOTS; kk++) {
                if (kk < a.K && ((cv >> kk) & 1u)) {
                    const float yk =
                        kk == spt - 1 ? yl : __uint_as_float((uint32_t)t[kk < FM_MAX_SLOTS - 1 ? kk : 0]);
                    moe = __fadd_rn(moe, __fmul_rn(T.cw[kk], yk));
                }
            }
            float o = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
            if (a.has_shared) o = __fadd_rn(o, __fmul_rn(sw, yl));
            else if (a.shared_y) o = __fadd_rn(o, __fmul_rn(sw, a.shared_y[row]));
            a.out[row] = o;
            if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(o);
            if (a.norm_w) {
                // next layer's input RMS norm (cpu_kernels.h:235-246): every
                // combining item publishes the sum of squares of its 64 rows,
                // then reduces all of them in the same fixed order
                const float sq =
                    __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fm_lane_sum<64>(o * o))));
                if (lane == 0) fm_put_tagged(&a.ss2[tile], sq, ep);
                uint64_t v = lane < (int)TILES ? fm_get_tagged(&a.ss2[lane]) : ((uint64_t)ep << 32);
                uint32_t it2 = 0;
                while (!__all((uint32_t)(v >> 32) == ep) && ++it2 < FM_SPIN_MAX) {
                    if ((uint32_t)(v >> 32) != ep) v = fm_get_tagged(&a.ss2[lane]);
                }
                if (it2 >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
                const float part = lane < (int)TILES ? __uint_as_float((uint32_t)v) : 0.f;
                const float tot =
                    __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fm_lane_sum<64>(part))));
                const float inv = 1.0f / sqrtf(tot / (float)H + a.norm_eps);
                a.normed[row] = o * inv * fm_bf16_to_f32(a.norm_w[row]);
            }
        }
    }
    if (help0) {
        // item 0's wave wv: groups 8..15 of the last item's wave-wv down rows,
        // once that item's activation operands are built
        uint32_t it = 0;
        while (__hip_atomic_load(&L.hlp_go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0 && ++it < FM_SPIN_MAX)
            __builtin_amdgcn_s_sleep(1);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        asm volatile("" ::: "memory");
        FmcItem &T2 = L.it[FMC_NG - 1];
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        fmm_mma_l4<NG, 1, 2>(chl, &T2.aq[0][0][0], L.zero, T.tr[wv], d0, d1, lane);
        const int qh = q >= 2 ? q : 2;
        float yh = q >= 2 ? fmm_fold(d0 + d1, sdh, bdh, &T2.asum[4 * qh], &T2.ainv[4 * qh]) : 0.f;
        yh = fmm_q_sum(yh);
        if (lane < 16) L.hy[wv][n] = yh;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): hy is written
        if (lane == 0) __hip_atomic_fetch_add(&L.hlp_done[wv], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    FM_DX_MARK(7);
    if (a.pool_mode && !fused && blockIdx.x == 0 && tid < a.K) {
        const int e = a.idx[tid];
        if (e < 0 || (uint32_t)e >= a.pool_n) atomicOr(a.err, FM_STATUS_BAD_EXPERT);  // skipped (invalid slot)
    }
    // Publishing the next epoch.  With the last slot valid, the combining
    // item of tile 0 has, through its waits, observed every tag user: each
    // wave of a valid slot read the epoch before its first weight load
    // returned (loads return in order), which precedes its item's activation
    // publish, and the combine waited on the outputs of every valid slot,
    // each computed after all of that slot's activations arrived.  Otherwise
    // (an invalid last slot: combine waves that poll without having loaded
    // weights, or mode 1 with no combine) the ends of the hand-off chains
    // count to the last one.
    if (gt == 0 && has) {
        if (a.mode != 0)
            fm_epoch_finish(a, ep, (uint32_t)a.S * TILES);
        else if (last && ((T.cvalid >> (a.S - 1)) & 1u)) {
            if (tile == 0) fm_epoch_publish(a, ep);
        } else if (last)
            fm_epoch_finish(a, ep, TILES);
    }
}

// ------------------------------------------------- few slots (S <= 4) ----
// A step of up to four slots (one routed expert, or a few) leaves most CUs
// idle in the kernels above (64 work items per slot).  Here each of 256
// workgroups (4 waves, one per slot) takes:
//   A  slot w, 16 gate/up rows of tile g / 4, the 1024-input quarter g % 4:
//      partial sums published as tagged words; the quarter-0 workgroup of the
//      tile adds the four quarters (same order as the kernels above), applies
//      SwiGLU and publishes the tile's 16 activations;
//   B  slot w, down rows 16 g .. 16 g + 15 over all 1024 activations;
//   C  the combine of rows 16 g .. + 15 over the slots -- all of them live in
//      this workgroup, so it is local (no output hand-off).
#define FMS_MAXS 4
#define FMS_GRID 256

struct __attribute__((aligned(16))) FmsLds {
    fm_h2 xq[2][16][32];          // x of this workgroup's quarter as operand rows
    float xsum[16], xinv[16];
    fm_h2 zero[32];
    fm_h2 aq[FMS_MAXS][2][FMM_GI][32];  // each slot's activations as operand rows
    float asum[FMS_MAXS][FMM_GI], ainv[FMS_MAXS][FMM_GI];
    float act[FMS_MAXS][FMM_MAXI];
    float y[FMS_MAXS][16];
    float pu[16];                 // one slot: the second half of the down rows
    float ph[4][16];              // one slot: each wave's half of the gate / up partials
    uint32_t tr[4][16 * FMM_TS];
};

__global__ __launch_bounds__(256, 1) void fm_decode_split_kernel(FmDecodeArgs a) {
    __shared__ FmsLds L;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // the wave's slot
    const int n = lane & 15, q = lane >> 4;
    constexpr uint32_t H = FMM_H, I = FMM_MAXI;
    const uint32_t g = blockIdx.x, tile = g >> 2, quarter = g & 3;
    const uint32_t rowA0 = tile * 16, rowB0 = g * 16;
    const bool mine = wv < a.S;
    // one slot (reached only with FMOE_DECODE_NO_SOLO set; fm_decode_solo_kernel
    // runs one slot otherwise): waves 0 and 1 take half of the gate rows' input
    // groups each, waves 2 and 3 half of the up rows', then waves 2 and 3 half
    // of the down rows' inputs each; the four waves share the activation polls
    // and operand rows
    const bool solo = a.S == 1;
    FM_DX_MARK(0);
    const uint32_t ep_ld = fm_epoch_load(a);
    // x of the quarter: 1024 elements, 4 threads per group
    fm_f4 xr[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xr[j] = fm_ldg_f4(a.x + 1024 * quarter + 16 * lane + 4 * j);  // every wave: same lines
    const FmSlot s = fmc_slot(a, mine ? wv : 0);
    const bool doA = mine && s.valid;
    const int bits = s.valid ? s.bits : 4;
    // one slot: waves 0, 1 take the gate rows' input groups 0-7, 8-15 of the
    // quarter, waves 2, 3 the up rows'
    const bool doG = solo ? s.valid && wv < 2 : doA, doU = solo ? s.valid && wv >= 2 : doA;
    const uint32_t gA = 16 * quarter + (solo ? 8 * (wv & 1) : 0);
    const bool doD = solo ? s.valid && wv >= 2 : doA;  // one slot: waves 2, 3 take down groups 0-7, 8-15
    const int ys = solo ? 0 : wv;  // the slot of this wave's down rows
    FmmCodes cg, cu, cdn;
    fmm_u2 sg, bg, su, bu, sdn, bdn;
    if (solo) {
        fmm_issue_codes<8>(s.gw, bits, rowA0, H, gA, doG, cg, lane, a.x);
        fmm_issue_sb<8>(s.gs, s.gb, rowA0, H, gA, doG, sg, bg, lane, a.x);
        fmm_issue_codes<8>(s.uw, bits, rowA0, H, gA, doU, cu, lane, a.x);
        fmm_issue_sb<8>(s.us, s.ub, rowA0, H, gA, doU, su, bu, lane, a.x);
    } else {
        fmm_issue_codes(s.gw, bits, rowA0, H, gA, doG, cg, lane, a.x);
        fmm_issue_sb(s.gs, s.gb, rowA0, H, gA, doG, sg, bg, lane, a.x);
        fmm_issue_codes(s.uw, bits, rowA0, H, gA, doU, cu, lane, a.x);
        fmm_issue_sb(s.us, s.ub, rowA0, H, gA, doU, su, bu, lane, a.x);
    }
    if (solo) {
        fmm_issue_codes<8>(s.dw, bits, rowB0, I, 8 * (wv & 1), doD, cdn, lane, a.x);
        fmm_issue_sb<8>(s.ds, s.db, rowB0, I, 8 * (wv & 1), doD, sdn, bdn, lane, a.x);
    } else {
        fmm_issue_codes(s.dw, bits, rowB0, I, 0, doD, cdn, lane, a.x);
        fmm_issue_sb(s.ds, s.db, rowB0, I, 0, doD, sdn, bdn, lane, a.x);
    }
    if (tid < 64) {  // wave 0 builds the quarter's 16 operand groups
        const int gg = tid >> 2, qq = tid & 3;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[4 * j] = xr[j].x;
            v[4 * j + 1] = xr[j].y;
            v[4 * j + 2] = xr[j].z;
            v[4 * j + 3] = xr[j].w;
        }
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float m = (j & 1) ? 0.0625f * f : f;
                L.xq[0][gg][4 * (2 * qq + h) + j] = fm_pack_h2(v[8 * h + j] * m, v[8 * h + 4 + j] * m);
            }
        const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
        for (int n2 = 0; n2 < 8; n2++)
            L.xq[1][gg][8 * qq + n2] = fm_pack_h2(v[n2] * (mt[n2] * f), v[8 + n2] * (mt[n2] * f));
        float sm = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
        sm += __shfl_xor(sm, 1, 64);
        sm += __shfl_xor(sm, 2, 64);
        if (qq == 0) {
            L.xsum[gg] = sm;
            L.xinv[gg] = fm_exp2i(24 - ex);
        }
        if (tid < 32) L.zero[tid] = fm_as_h2(0u);
    }
    __syncthreads();
    FM_DX_MARK(1);
    const uint32_t ep = fm_epoch_tag(ep_ld);
    // ---- A: this quarter's partial gate/up sums of the 16 rows ----
    uint64_t *part = a.p2 + ((size_t)wv * (H / 64) + tile) * 4 * 32;  // [slot][tile][quarter][16 rows][g, u]
    float pg = 0.f, pu = 0.f;
    if (solo && s.valid) {
        // half h of the quarter's 16 groups of the gate (waves 0, 1) or up
        // (waves 2, 3) rows; the four halves meet in LDS
        const int h = wv & 1;
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        const fm_h2 *xq = &L.xq[bits == 4 ? 0 : 1][8 * h][0];
        if (bits == 4)
            fmm_mma_l4<8>(wv < 2 ? cg : cu, xq, L.zero, L.tr[wv], d0, d1, lane);
        else
            fmm_mma<2, 8>(wv < 2 ? cg : cu, xq, L.zero, L.tr[wv], d0, d1, lane);
        FM_DX_MARK(2);
        const bool qok = q < 2;
        const int gq = 8 * h + 4 * (qok ? q : 0);
        const float ph = fmm_q_sum(qok ? fmm_fold(d0 + d1, wv < 2 ? sg : su, wv < 2 ? bg : bu, &L.xsum[gq],
                                                  &L.xinv[gq])
                                       : 0.f);
        if (lane < 16) L.ph[wv][lane] = ph;
        __syncthreads();
        pg = L.ph[0][lane & 15] + L.ph[1][lane & 15];
        pu = L.ph[2][lane & 15] + L.ph[3][lane & 15];
    } else if (doA) {
        fmm_f4 g0 = {0, 0, 0, 0}, g1 = g0, u0 = g0, u1 = g0;
        const fm_h2 *xq = &L.xq[bits == 4 ? 0 : 1][0][0];
        if (bits == 4) {
            fmm_mma_l4(cg, xq, L.zero, L.tr[wv], g0, g1, lane);
            fmm_mma_l4(cu, xq, L.zero, L.tr[wv], u0, u1, lane);
        } else {
            fmm_mma<2>(cg, xq, L.zero, L.tr[wv], g0, g1, lane);
            fmm_mma<2>(cu, xq, L.zero, L.tr[wv], u0, u1, lane);
        }
        FM_DX_MARK(2);
        pg = fmm_q_sum(fmm_fold(g0 + g1, sg, bg, &L.xsum[4 * q], &L.xinv[4 * q]));
        pu = fmm_q_sum(fmm_fold(u0 + u1, su, bu, &L.xsum[4 * q], &L.xinv[4 * q]));
    }
    if (solo ? s.valid && wv == 0 : doA) {
        // lanes 0..15: gate of row n, lanes 16..31: up of row n - 16 (the
        // shuffle runs in the full wave: an inactive source lane reads as 0)
        const float pu_n = __shfl(pu, (lane - 16) & 63, 64);
        const float own = lane < 16 ? pg : pu_n;
        if (quarter != 0 && lane < 32) fm_put_tagged(&part[quarter * 32 + lane], own, ep);
        if (quarter == 0) {
            // the tile's activations: the other three quarters' partials, in the order (q0 + q1) + (q2 + q3)
            uint64_t t[3];
            const bool rd = lane < 32;
#pragma unroll
            for (int j = 0; j < 3; j++) t[j] = rd ? fm_get_tagged(&part[(j + 1) * 32 + lane]) : ((uint64_t)ep << 32);
            uint32_t it = 0;
            do {
                bool ready = true;
#pragma unroll
                for (int j = 0; j < 3; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
                if (__all(ready)) break;
#pragma unroll
                for (int j = 0; j < 3; j++)
                    if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(&part[(j + 1) * 32 + lane]);
            } while (++it < FM_SPIN_MAX);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
            const float p1 = __uint_as_float((uint32_t)t[0]), p2 = __uint_as_float((uint32_t)t[1]);
            const float p3 = __uint_as_float((uint32_t)t[2]);
            const float tot = (own + p1) + (p2 + p3);
            const float up = __shfl(tot, (lane & 15) + 16, 64);
            if (lane < 16) fm_put_tagged(&a.act2[(size_t)wv * I + rowA0 + lane], fm_silu_mul(tot, up), ep);
        }
    }
    FM_DX_MARK(3);
    // ---- B: the slot's 1024 activations, then 16 down rows ----
    if (solo && s.valid) {
        // wave w polls activations 256 w .. 256 w + 255
        const uint64_t *src = a.act2 + 256 * wv;
        uint64_t t[4];
#pragma unroll
        for (int j = 0; j < 4; j++) t[j] = fm_get_tagged(src + 64 * j + lane);
        uint32_t it = 0;
        do {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < 4; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
            if (__all(ready)) break;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(src + 64 * j + lane);
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        FM_DX_MARK(4);
#pragma unroll
        for (int j = 0; j < 4; j++) L.act[0][256 * wv + 64 * j + lane] = __uint_as_float((uint32_t)t[j]);
        __syncthreads();
        // per group (16 threads x 4 elements): sum, operand scale 2^e, operand rows
        const int sb = s.bits, lay = sb == 4 ? 0 : 1;
        const uint32_t gg = tid >> 4;
        const float *ag = &L.act[0][64 * gg + 4 * (tid & 15)];
        float sm = (ag[0] + ag[1]) + (ag[2] + ag[3]);
        float mx = fmaxf(fmaxf(fabsf(ag[0]), fabsf(ag[1])), fmaxf(fabsf(ag[2]), fabsf(ag[3])));
        sm = fmm_row_sum(sm);
        mx = fm_row16_max(mx);
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
        if ((tid & 15) == 0) {
            L.asum[0][gg] = sm;
            L.ainv[0][gg] = fm_exp2i(24 - ex);
        }
        fmm_build_pair(&L.act[0][64 * gg], sb, 2 * (tid & 15), f, &L.aq[0][lay][gg][0]);
        fmm_build_pair(&L.act[0][64 * gg], sb, 2 * (tid & 15) + 1, f, &L.aq[0][lay][gg][0]);
        __syncthreads();
    } else if (!solo && doA) {
        const uint64_t *src = a.act2 + (size_t)wv * I;
        uint64_t t[16];
#pragma unroll
        for (int j = 0; j < 16; j++) t[j] = fm_get_tagged(src + 64 * j + lane);
        uint32_t it = 0;
        do {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < 16; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
            if (__all(ready)) break;
#pragma unroll
            for (int j = 0; j < 16; j++)
                if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(src + 64 * j + lane);
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        FM_DX_MARK(4);
#pragma unroll
        for (int j = 0; j < 16; j++) L.act[wv][64 * j + lane] = __uint_as_float((uint32_t)t[j]);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        // per group (4 lanes x 16 elements): sum, scale 2^e, operand rows
        const int lay = bits == 4 ? 0 : 1;
        const uint32_t gg = lane >> 2, qq = lane & 3;
        const float *ag = &L.act[wv][64 * gg + 16 * qq];
        float sm = 0.f, mx = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            sm += ag[j];
            mx = fmaxf(mx, fabsf(ag[j]));
        }
        sm += __shfl_xor(sm, 1, 64);
        sm += __shfl_xor(sm, 2, 64);
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
        if (qq == 0) {
            L.asum[wv][gg] = sm;
            L.ainv[wv][gg] = fm_exp2i(24 - ex);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) fmm_build_pair(&L.act[wv][64 * gg], bits, 8 * qq + e, f, &L.aq[wv][lay][gg][0]);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
    float y = 0.f;
    if (doD) {
        FM_DX_MARK(5);
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        if (solo) {
            // half h of the 16 groups (NG = 8: lanes q < 2 hold its groups)
            const int h = wv & 1;
            const fm_h2 *aq = &L.aq[0][bits == 4 ? 0 : 1][8 * h][0];
            if (bits == 4)
                fmm_mma_l4<8>(cdn, aq, L.zero, L.tr[wv], d0, d1, lane);
            else
                fmm_mma<2, 8>(cdn, aq, L.zero, L.tr[wv], d0, d1, lane);
            const bool qok = q < 2;
            const int gq = 8 * h + 4 * (qok ? q : 0);
            y = fmm_q_sum(qok ? fmm_fold(d0 + d1, sdn, bdn, &L.asum[0][gq], &L.ainv[0][gq]) : 0.f);
        } else {
            if (bits == 4)
                fmm_mma_l4(cdn, &L.aq[ys][0][0][0], L.zero, L.tr[wv], d0, d1, lane);
            else
                fmm_mma<2>(cdn, &L.aq[ys][1][0][0], L.zero, L.tr[wv], d0, d1, lane);
            y = fmm_q_sum(fmm_fold(d0 + d1, sdn, bdn, &L.asum[ys][4 * q], &L.ainv[ys][4 * q]));
        }
    }
    if (solo && s.valid) {
        if (wv == 3 && lane < 16) L.pu[n] = y;  // the second half, to wave 2
        __syncthreads();
        if (wv == 2) y += L.pu[n];
    }
    if (doD && (!solo || wv == 2) && lane < 16) {
        if (a.mode == 1)
            a.expert_out[(size_t)ys * H + rowB0 + n] = y;
        else
            L.y[ys][n] = y;
    }
    FM_DX_MARK(6);
    __syncthreads();
    // Every wave of a valid slot waited above for the activations of all 64
    // tiles, each published after the tile's four quarters tagged their
    // partials: so every tag user of this call has read the epoch, and one
    // plain store publishes it for the next call (no completion counter).
    if (g == 0 && tid == 0) fm_epoch_publish(a, ep);
    // ---- C: rows 16 g .. + 15 over the slots, in cpu_vec_madd order ----
    if (a.mode == 0 && wv == 0 && lane < 16) {
        const uint32_t row = rowB0 + lane;
        float moe = 0.f;
#pragma unroll
        for (int k = 0; k < FMS_MAXS; k++) {
            if (k < a.K) {
                const FmSlot sk = fmc_slot(a, k);
                if (sk.valid) moe = __fadd_rn(moe, __fmul_rn(sk.weight, L.y[k][lane]));
            }
        }
        float o = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
        const float sw = (a.has_shared || a.shared_y)
                             ? (a.shared_score ? fm_sigmoid(a.shared_score[0]) : a.shared_w_host)
                             : 0.f;
        if (a.has_shared) {
            const FmSlot ss = fmc_slot(a, a.S - 1);
            o = __fadd_rn(o, __fmul_rn(sw, ss.valid ? L.y[a.S - 1][lane] : 0.f));
        } else if (a.shared_y) {
            o = __fadd_rn(o, __fmul_rn(sw, a.shared_y[row]));
        }
        a.out[row] = o;
        if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(o);
    }
    if (a.pool_mode && g == 0 && tid < a.K) {
        const int e = a.idx[tid];
        if (e < 0 || (uint32_t)e >= a.pool_n) atomicOr(a.err, FM_STATUS_BAD_EXPERT);  // skipped (invalid slot)
    }
    FM_DX_MARK(7);
}

// ------------------------------------------------ one slot (config 1) ----
// One expert (or the shared expert alone) with a single cross-workgroup
// hand-off: workgroup g computes gate and up rows 4g .. 4g + 3 over all 4096
// inputs (wave w of 8: input eighth w, 16 MMA steps; the 16 MFMA columns are
// the 4 gate rows, the 4 up rows and 8 zero columns), adds the eighths in LDS
// in the order ((e0 + e1) + (e2 + e3)) + ((e4 + e5) + (e6 + e7)) and publishes
// its 4 activations; every workgroup then polls the 1024 activations and
// computes down rows 16g .. 16g + 15 (waves 6 and 7, half of the inputs each)
// and the combine of those rows.  Eight waves rather than four: one wave's MMA
// steps form a latency chain, and two waves on a SIMD overlap theirs.  (The
// few-slot kernel below hands quarter partials to a reducing workgroup
// first: one more round trip.)
#define FMO_W 8  // waves of the one-slot kernel: one input eighth each in the gate/up MMA
struct __attribute__((aligned(16))) FmoLds {
    fm_h2 xq[2][FMM_GH][32];  // x as operand rows (4-bit | 2-bit layout)
    float xsum[FMM_GH], xinv[FMM_GH];
    fm_h2 zero[32];
    fm_h2 aq[FMM_GI][32];     // the activations as operand rows (the slot's layout)
    float asum[FMM_GI], ainv[FMM_GI];
    float act[FMM_MAXI];
    float ph[FMO_W][8];       // per wave (input eighth): partials of the 4 gate and 4 up rows
    float pu[16];             // the second half of the down rows
    uint32_t tr[FMO_W][16 * FMM_TS];
};

__global__ __launch_bounds__(64 * FMO_W, 1) void fm_decode_solo_kernel(FmDecodeArgs a) {
    __shared__ FmoLds L;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, q = lane >> 4;
    constexpr uint32_t H = FMM_H, I = FMM_MAXI;
    const uint32_t g = blockIdx.x, rowA0 = 4 * g, rowB0 = 16 * g;
    FM_DX_MARK(0);
    const uint32_t ep_ld = fm_epoch_load(a);
    // x: thread t < 256 holds elements 16 t .. 16 t + 15 (group t / 4)
    fm_f4 xr[4];
    const bool xt = tid < 256;
#pragma unroll
    for (int j = 0; j < 4; j++) xr[j] = fm_ldg_f4(a.x + 16 * (xt ? tid : 0) + 4 * j);
    const FmSlot s = fmc_slot(a, 0);
    const bool ok = s.valid;
    const int bits = ok ? s.bits : 4;
    // gate / up codes of input eighth wv (8 groups: one 4-bit piece, half a
    // 2-bit one, whose lanes n >= 8 repeat lane n - 8): MFMA column 4j + kq is
    // gate row rowA0 + kq (j = 0) or up row rowA0 + kq (j = 1); columns 8..15
    // are zero
    FmmCodes cd;
    fmm_u2 sc = {0u, 0u}, bi = {0u, 0u};
    {
        const uint32_t wpg = 2 * bits, wpr = (H / 64) * wpg, g0 = 8 * wv;
        const uint32_t *gw = ok ? s.gw : (const uint32_t *)a.x, *uw = ok ? s.uw : (const uint32_t *)a.x;
        const uint32_t row = ok ? rowA0 + q : 0;
        const uint32_t rw = ok ? wpr : 0;
        const int nw = bits == 2 ? (n & 7) : n;
        const uint32_t po = ok ? g0 * wpg : 0;
        cd.c[0] = fm_ldg_u4_nt(gw + (size_t)row * rw + po + 4 * nw);
        cd.c[1] = fm_ldg_u4_nt(uw + (size_t)row * rw + po + 4 * nw);
#pragma unroll
        for (int j = 2; j < 8; j++) cd.c[j] = (fm_u4){0u, 0u, 0u, 0u};
        // scale / bias runs: lane (n, q) = column n, groups g0 + 4q .. + 3 (q < 2)
        const bool mine = ok && n < 8 && q < 2;
        const uint16_t *S_ = n < 4 ? s.gs : s.us, *B_ = n < 4 ? s.gb : s.ub;
        const size_t o = mine ? (size_t)(rowA0 + (n & 3)) * (H / 64) + g0 + 4 * q : 0;
        const fmm_u2 sv = *(const FM_GLOBAL fmm_u2 *)(mine ? S_ + o : (const uint16_t *)a.x);
        const fmm_u2 bv = *(const FM_GLOBAL fmm_u2 *)(mine ? B_ + o : (const uint16_t *)a.x);
        sc = mine ? sv : (fmm_u2){0u, 0u};
        bi = mine ? bv : (fmm_u2){0u, 0u};
    }
    // down rows rowB0 .. + 15: waves 6, 7 take input groups 0-7, 8-15
    const bool doD = ok && wv >= FMO_W - 2;
    FmmCodes cdn;
    fmm_u2 sdn, bdn;
    fmm_issue_codes<8>(s.dw, bits, rowB0, I, 8 * (wv & 1), doD, cdn, lane, a.x);
    fmm_issue_sb<8>(s.ds, s.db, rowB0, I, 8 * (wv & 1), doD, sdn, bdn, lane, a.x);
    if (xt) {
        // x -> operand rows (both layouts), group sums and scales
        const int gg = tid >> 2, qq = tid & 3;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[4 * j] = xr[j].x;
            v[4 * j + 1] = xr[j].y;
            v[4 * j + 2] = xr[j].z;
            v[4 * j + 3] = xr[j].w;
        }
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float m = (j & 1) ? 0.0625f * f : f;
                L.xq[0][gg][4 * (2 * qq + h) + j] = fm_pack_h2(v[8 * h + j] * m, v[8 * h + 4 + j] * m);
            }
        const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
        for (int n2 = 0; n2 < 8; n2++) L.xq[1][gg][8 * qq + n2] = fm_pack_h2(v[n2] * (mt[n2] * f), v[8 + n2] * (mt[n2] * f));
        float sm = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
        sm += __shfl_xor(sm, 1, 64);
        sm += __shfl_xor(sm, 2, 64);
        if (qq == 0) {
            L.xsum[gg] = sm;
            L.xinv[gg] = fm_exp2i(24 - ex);
        }
        if (tid < 32) L.zero[tid] = fm_as_h2(0u);
    }
    __syncthreads();
    FM_DX_MARK(1);
    const uint32_t ep = fm_epoch_tag(ep_ld);
    // ---- A: eighth wv of the 4 gate and 4 up rows, the eighths added in LDS ----
    if (ok) {
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        const fm_h2 *xq = &L.xq[bits == 4 ? 0 : 1][8 * wv][0];
        if (bits == 4)
            fmm_mma_l4<8>(cd, xq, L.zero, L.tr[wv], d0, d1, lane);
        else
            fmm_mma<2, 8>(cd, xq, L.zero, L.tr[wv], d0, d1, lane);
        const int qq = q < 2 ? q : 0;
        const float f = q < 2 ? fmm_fold(d0 + d1, sc, bi, &L.xsum[8 * wv + 4 * qq], &L.xinv[8 * wv + 4 * qq]) : 0.f;
        const float ph = fmm_q_sum(f);
        if (lane < 8) L.ph[wv][lane] = ph;
    }
    __syncthreads();
    FM_DX_MARK(2);
    if (ok && tid < 4) {
        const float gs = ((L.ph[0][tid] + L.ph[1][tid]) + (L.ph[2][tid] + L.ph[3][tid])) +
                         ((L.ph[4][tid] + L.ph[5][tid]) + (L.ph[6][tid] + L.ph[7][tid]));
        const float us = ((L.ph[0][4 + tid] + L.ph[1][4 + tid]) + (L.ph[2][4 + tid] + L.ph[3][4 + tid])) +
                         ((L.ph[4][4 + tid] + L.ph[5][4 + tid]) + (L.ph[6][4 + tid] + L.ph[7][4 + tid]));
        fm_put_tagged(&a.act2[rowA0 + tid], fm_silu_mul(gs, us), ep);
    }
    FM_DX_MARK(3);
    // ---- B: the 1024 activations (wave w polls its eighth), operand rows ----
    if (ok) {
        constexpr int PQ = FMM_MAXI / (64 * FMO_W);  // words per lane
        const uint64_t *src = a.act2 + (FMM_MAXI / FMO_W) * wv;
        uint64_t t[PQ];
#pragma unroll
        for (int j = 0; j < PQ; j++) t[j] = fm_get_tagged(src + 64 * j + lane);
        uint32_t it = 0;
        do {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < PQ; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
            if (__all(ready)) break;
#pragma unroll
            for (int j = 0; j < PQ; j++)
                if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(src + 64 * j + lane);
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        FM_DX_MARK(4);
#pragma unroll
        for (int j = 0; j < PQ; j++) L.act[(FMM_MAXI / FMO_W) * wv + 64 * j + lane] = __uint_as_float((uint32_t)t[j]);
        // this wave's two groups (its own polled activations) -> operand rows,
        // sums and scales: lanes 0-15 group 2 wv, lanes 16-31 group 2 wv + 1
        // (16 threads x 4 elements a group; lanes 32-63 repeat them, unused)
        fm_wave_lds_sync();
        const uint32_t gg = 2 * wv + ((lane >> 4) & 1), tg = lane & 15;
        const float *ag = &L.act[64 * gg + 4 * tg];
        float sm = (ag[0] + ag[1]) + (ag[2] + ag[3]);
        float mx = fmaxf(fmaxf(fabsf(ag[0]), fabsf(ag[1])), fmaxf(fabsf(ag[2]), fabsf(ag[3])));
        sm = fmm_row_sum(sm);
        mx = fm_row16_max(mx);
        const int ex = fm_group_shift(mx);
        const float f = fm_exp2i(ex);
        if (lane < 32) {
            if (tg == 0) {
                L.asum[gg] = sm;
                L.ainv[gg] = fm_exp2i(24 - ex);
            }
            fmm_build_pair(&L.act[64 * gg], bits, 2 * tg, f, &L.aq[gg][0]);
            fmm_build_pair(&L.act[64 * gg], bits, 2 * tg + 1, f, &L.aq[gg][0]);
        }
        __syncthreads();
    }
    // ---- C: down rows rowB0 .. + 15 (waves 6, 7: halves of the inputs), combine ----
    float y = 0.f;
    if (doD) {
        FM_DX_MARK(5);
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        const int h = wv & 1;
        const fm_h2 *aq = &L.aq[8 * h][0];
        if (bits == 4)
            fmm_mma_l4<8>(cdn, aq, L.zero, L.tr[wv], d0, d1, lane);
        else
            fmm_mma<2, 8>(cdn, aq, L.zero, L.tr[wv], d0, d1, lane);
        const bool qok = q < 2;
        const int gq = 8 * h + 4 * (qok ? q : 0);
        y = fmm_q_sum(qok ? fmm_fold(d0 + d1, sdn, bdn, &L.asum[gq], &L.ainv[gq]) : 0.f);
        if (wv == FMO_W - 1 && lane < 16) L.pu[n] = y;
    }
    __syncthreads();
    FM_DX_MARK(6);
    // every workgroup waited for all 1024 activations, each published after
    // its workgroup's four waves read the epoch: one plain store publishes it
    if (g == 0 && tid == 0) fm_epoch_publish(a, ep);
    if (wv == FMO_W - 2 && lane < 16) {
        const uint32_t row = rowB0 + lane;
        if (ok) y += L.pu[n];
        if (a.mode == 1) {
            if (ok) a.expert_out[row] = y;
        } else {
            const bool routed = a.K >= 1;  // slot 0 is routed (else: the shared expert alone)
            float o = a.h_mid ? a.h_mid[row] : 0.f;
            if (routed) {
                const float moe = ok ? __fmul_rn(s.weight, y) : 0.f;
                o = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
            }
            const float sw = (a.has_shared || a.shared_y)
                                 ? (a.shared_score ? fm_sigmoid(a.shared_score[0]) : a.shared_w_host)
                                 : 0.f;
            if (a.has_shared)
                o = __fadd_rn(o, __fmul_rn(sw, ok ? y : 0.f));
            else if (a.shared_y)
                o = __fadd_rn(o, __fmul_rn(sw, a.shared_y[row]));
            a.out[row] = o;
            if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(o);
        }
    }
    if (a.pool_mode && g == 0 && tid < a.K) {
        const int e = a.idx[tid];
        if (e < 0 || (uint32_t)e >= a.pool_n) atomicOr(a.err, FM_STATUS_BAD_EXPERT);  // skipped (invalid slot)
    }
    FM_DX_MARK(7);
}

// Fused routing needs the one-workgroup-per-CU kernel with the last CU's
// third wave group idle (it writes the slot-order outputs), one logit per
// thread, and the combine.
static bool fmc_route_fits(const FmDecodeArgs &a, uint32_t tiles, int cus) {
    return a.ntok <= 1 && a.mode == 0 && a.pool_mode && a.K >= 1 && a.K <= 64 && a.route_E >= a.K &&
           a.route_E <= FMC_THREADS && (uint32_t)a.S * tiles <= (uint32_t)(FMC_NG * cus) - 1;
}

int fm_launch_decode_mfma(FmDecodeArgs &a, hipStream_t st) {
    if (a.norm_w && a.mode != 0) return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: norm needs the combine");
    // up to 11 slots a token: the row-split kernel where it is enabled
    {
        const int rc = fm_launch_decode_bal(a, st);
        if (rc != FM_ERR_UNSUPPORTED) return rc;
        fm_clear_error();
    }
    const int cus = fm_num_cus();
    if (a.route_logits && !fmc_route_fits(a, a.hidden / 64, cus))
        return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: fused routing does not fit this launch");
    // hidden 2048 / inter 512 (the Qwen3.5-35B-A3B expert shape): the
    // one-workgroup-per-CU kernel with 8-group units, one token whose items
    // fit three per CU
    if (a.hidden == 2048 && a.inter == 512) {
        static int per_cu_8 = -1;
        if (per_cu_8 < 0 &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_8, fm_decode_cu_kernel<8, false>, FMC_THREADS, 0) !=
                hipSuccess)
            per_cu_8 = 0;
        if (a.ntok <= 1 && a.spt == a.S && per_cu_8 >= 1 && (uint32_t)a.S * 32 <= (uint32_t)(FMC_NG * cus) &&
            a.S <= FM_MAX_SLOTS) {
            if (a.route_logits)
                hipLaunchKernelGGL((fm_decode_cu_kernel<8, true>), dim3(cus), dim3(FMC_THREADS), 0, st, a);
            else
                hipLaunchKernelGGL((fm_decode_cu_kernel<8, false>), dim3(cus), dim3(FMC_THREADS), 0, st, a);
            return fm_check_launch("fm_decode_cu_kernel");
        }
        return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: 2048/512 takes one token");
    }
    if (a.hidden != FMM_H || a.inter != FMM_MAXI)
        return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: shape");
    static int per_cu = -1, per_cu_mp = -1;
    if (per_cu < 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fm_decode_mfma_kernel<false>, 256, 0) != hipSuccess)
            per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_mp, fm_decode_mfma_kernel<true>, 256, 0) !=
            hipSuccess)
            per_cu_mp = 0;
    }
    if (a.S > FMM_MAXS || a.spt < 1 || a.S != a.ntok * a.spt)
        return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: %d slots", a.S);
    if (a.ntok > 1 && (a.norm_w || a.mode != 0 || !a.pool_mode))
        return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: several tokens need pool mode and the combine");
    // up to four slots of one token (no fused norm): the split kernel
    if (a.ntok <= 1 && a.S <= FMS_MAXS && !a.norm_w && !a.route_logits) {
        const char *no_split = getenv("FMOE_DECODE_NO_SPLIT");
        if (!(no_split && *no_split)) {
            // one slot: one hand-off (FMOE_DECODE_NO_SOLO set: the few-slot kernel, which tests compare)
            const char *no_solo = getenv("FMOE_DECODE_NO_SOLO");
            if (a.S == 1 && a.ntok <= 1 && !(no_solo && *no_solo)) {
                hipLaunchKernelGGL(fm_decode_solo_kernel, dim3(FMS_GRID), dim3(64 * FMO_W), 0, st, a);
                return fm_check_launch("fm_decode_solo_kernel");
            }
            hipLaunchKernelGGL(fm_decode_split_kernel, dim3(FMS_GRID), dim3(256), 0, st, a);
            return fm_check_launch("fm_decode_split_kernel");
        }
    }
    static int per_cu_c = -1;
    if (per_cu_c < 0 &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_c, fm_decode_cu_kernel<16, false>, FMC_THREADS, 0) != hipSuccess)
        per_cu_c = 0;
    // one token whose items fit three per CU: the one-workgroup-per-CU kernel
    // (FMOE_DECODE_NO_CU set in the environment: the three-workgroup kernel,
    // which tests compare it with)
    const char *no_cu = getenv("FMOE_DECODE_NO_CU");
    if (a.ntok <= 1 && per_cu_c >= 1 && (uint32_t)a.S * (FMM_H / 64) <= (uint32_t)(FMC_NG * cus) &&
        a.S <= FM_MAX_SLOTS && !(no_cu && *no_cu)) {
        if (a.route_logits)
            hipLaunchKernelGGL((fm_decode_cu_kernel<16, true>), dim3(cus), dim3(FMC_THREADS), 0, st, a);
        else
            hipLaunchKernelGGL((fm_decode_cu_kernel<16, false>), dim3(cus), dim3(FMC_THREADS), 0, st, a);
        return fm_check_launch("fm_decode_cu_kernel");
    }
    if (a.route_logits) return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: fused routing needs the per-CU kernel");
    const uint32_t tiles = a.inter / 16 > a.hidden / 64 ? a.inter / 16 : a.hidden / 64;
    const uint32_t items = (uint32_t)a.S * tiles;
    // every block may wait on others: the grid must be resident, and it is a
    // whole number of slots so that a slot's tiles run in one pass
    const uint32_t cap = per_cu > 0 ? (uint32_t)(per_cu * fm_num_cus()) / tiles * tiles : 0;
    if (items <= cap && a.S <= FM_MAX_SLOTS) {
        hipLaunchKernelGGL(fm_decode_mfma_kernel<false>, dim3(items), dim3(256), 0, st, a);
        return fm_check_launch("fm_decode_mfma_kernel");
    }
    const uint32_t cap_mp = per_cu_mp > 0 ? (uint32_t)(per_cu_mp * fm_num_cus()) / tiles * tiles : 0;
    if (cap_mp == 0) return fm_fail(FM_ERR_UNSUPPORTED, "mfma decode: grid");
    hipLaunchKernelGGL(fm_decode_mfma_kernel<true>, dim3(cap_mp), dim3(256), 0, st, a);
    return fm_check_launch("fm_decode_mfma_kernel");
}
