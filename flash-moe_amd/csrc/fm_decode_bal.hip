// fm_decode_bal.hip -- the single-token decode step (K routed experts +
// shared expert: gate/up, SwiGLU, down, weighted combine into the residual;
// CMD3 of layer_forward.h:3895-3993) with the work split evenly over the CUs
// by rows instead of by experts.
//
// One 768-thread workgroup per CU; workgroup c owns, for EVERY slot,
//   * intermediate rows 4c .. 4c + 3 of the gate and up matrices, and
//   * output rows 16c .. 16c + 15 of the down matrix,
// so every CU streams the same number of bytes (hidden 4096 / inter 1024:
// 256 workgroups, 11 slots = 44 gate + 44 up rows of 2 KB and 176 down rows of
// 512 B each).  The down rows are copied into LDS by the vector memory DMA
// path (global_load_lds_dwordx4) right behind the CU's gate/up loads, so the
// whole step's bytes are in flight from the start and no register holds them
// across the wait below.
//
// One hand-off per CU: after its gate/up MMAs, wave 0 stores the CU's 44
// activations (fp32, write-through agent-scope stores), waits for them to
// complete, then stores ONE tagged flag word (the call's epoch, see
// fm_decode.h).  Wave 0 then polls the 256 flags; once all carry the epoch,
// every down wave reads its slot's 1024 activations (4 KB), turns them into
// MFMA operand rows and multiplies them with the 16 down rows in LDS.  The
// combine is local: the CU holds every slot's outputs of its 16 rows, so it
// sums them in slot order (cpu_vec_madd, layer_forward.h:1257, 1295-1305) and
// writes its rows of `out` -- no per-slot outputs cross the chip.
//
// The MFMA scheme is the one of fm_decode_mfma.hip (codes as subnormal fp16
// B operands, x in the operand row of its group), but the weight loads put
// each lane's 16-byte runs straight into the MFMA lane layout (lane (n, kq)
// reads row n's words 16 h + 4 kq of each 64-word piece), so no transpose
// buffer is needed.  Gate/up tiles hold 16 rows: 4 gate + 4 up rows of slot
// 2t, then of slot 2t + 1 (x is the same vector for every slot).  A tile whose
// two slots differ in bit width runs the 4-bit and the 2-bit MMA with the
// other slot's columns masked.
#include "fm_decode.h"
#include "fm_mfma_dev.h"
#include "fm_route_cu.h"

#include <stdlib.h>

#define FMB_THREADS 1024                 // 16 wavefronts
#define FMB_W (FMB_THREADS / 64)
#define FMB_GU (FMC_THREADS / 64)        // waves 0-11: gate/up units, routing, then one down tile each
#define FMB_MAXS 11                      // slots (waves 0 .. S - 1 hold one down tile each)
#define FMB_TILES ((FMB_MAXS + 1) / 2)   // gate/up tiles (two slots each)
static_assert(4 * FMB_TILES <= 2 * FMB_GU && FMB_MAXS <= FMB_GU, "two gate/up units and one down tile per wave");
#ifndef FMB_DN_AFTER_GU
#define FMB_DN_AFTER_GU 1  // the DMA waves start once every gate/up wave has issued its loads
#endif

struct __attribute__((aligned(16))) FmbLds {
    fm_u4 dn[FMB_MAXS][2][4][64];       // each slot's 16 down rows, MFMA lane order [piece][h][lane]
    uint16_t dsb[FMB_MAXS][2][256];     // ... their scales and biases [16 rows][16 groups]
    fm_h2 xq[2][FMM_GH][32];            // x as operand rows: [4-bit | 2-bit layout][group][32 pairs]
    fm_h2 aq[FMB_MAXS][FMM_GI][32];     // each slot's activations as operand rows (its own layout)
    fm_h2 zero[32];
    float xsum[FMM_GH], xinv[FMM_GH];   // per-group sums of x, 2^(24 - e)
    float asum[FMB_MAXS][FMM_GI], ainv[FMB_MAXS][FMM_GI];
    float part[FMB_TILES][4][16];       // gate/up partial sums: [tile][input quarter][tile row]
    float y[FMB_MAXS][16];              // every slot's outputs of the CU's 16 rows
    float cw[FM_MAX_SLOTS];             // combine: slot weights
    float sw;                           // combine: the shared expert's sigmoid gate
    uint32_t cvalid;                    // combine: bit k = slot k valid
    uint32_t xready, pdone, go, ydone;  // LDS hand-offs between the waves
    uint32_t gu_issued, dn_ready;
    FmcRoute rt;                        // fused routing scratch
    int rsel[FM_MAX_K];
    int rp[FM_MAX_K];
};

// Registers of one gate/up unit: a 16-row tile over one quarter (16 groups)
// of the inputs, in MFMA lane order, plus the lane's scale / bias runs.
struct FmbUnit {
    fm_u4 v[2][4];
    fmm_u2 sc, bi;
};

// 2 NG MFMAs over NG groups with the codes already in lane order: v[p][h]
// holds row n's words 64 p + 16 h + 4 kq .. + 3 (2-bit, or NG = 8: p = 0 only;
// 2-bit with NG = 8: h < 2 only).  MASK: lanes
// with !colok contribute zero codes (their column belongs to the other bit
// width of a mixed tile).  4-bit: the x quads of the lane's own group are kept
// in registers and selected per step; 2-bit: read from LDS one step ahead.
template <int BITS, bool MASK, int NG>  // NG: groups of the unit (16: 32 MFMAs, 8: 16)
FM_DEV void fmb_mma(const fm_u4 (&v)[2][4], const fm_h2 *xq_grp0, const fm_h2 *zero, fmm_f4 &d0, fmm_f4 &d1,
                    int lane, bool colok) {
    const int m = lane & 15, kq = lane >> 4;
    if constexpr (BITS == 4) {
        fmm_h8 xv[4];
#pragma unroll
        for (int s = 0; s < 4; s++) xv[s] = fmm_lds_op(xq_grp0 + 32 * m + 16 * (kq & 1) + 4 * s);
        const fmm_h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
        const bool kq_on = (kq >> 1) == (m & 1);
#pragma unroll
        for (int j = 0; j < 2 * NG; j++) {
            const int p = j >> 4, c = j >> 3, i = j & 7;
            const bool on = kq_on && c == (m >> 2) && (i >> 2) == ((m >> 1) & 1);
            const fmm_h8 xo = on ? xv[i & 3] : z;
            uint32_t w = fmm_comp(v[p][2 * (c & 1) + (i >> 2)], i & 3);
            if (MASK) w = colok ? w : 0u;
            const fmm_h8 co = fmm_codes<4>(w, 0);
            if (i & 1)
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d1, 0, 0, 0);
            else
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d0, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        auto src_of = [&](int j) -> const fm_h2 * {
            const int c = j >> 3, i = j & 7;
            return (kq == (m & 3) && c == (m >> 2)) ? xq_grp0 + 32 * m + 4 * i : zero;
        };
        fmm_h8 xo = fmm_lds_op(src_of(0));
#pragma unroll
        for (int j = 0; j < 2 * NG; j++) {
            const int c = j >> 3, i = j & 7;
            fmm_h8 xn = xo;
            if (j + 1 < 2 * NG) xn = fmm_lds_op(src_of(j + 1));
            uint32_t w = fmm_comp(v[0][c], i >> 1);
            if (MASK) w = colok ? w : 0u;
            const fmm_h8 co = fmm_codes<2>(w, i & 1);
            if (i & 1)
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d1, 0, 0, 0);
            else
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, co, d0, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            xo = xn;
        }
    }
}

FM_DEV int fmb_u(int v) { return __builtin_amdgcn_readfirstlane(v); }
FM_DEV uint64_t fmb_u(const void *p) {
    const uint64_t v = (uint64_t)p;
    return (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32);
}

// Word offset of load (p, h) of a lane's run in a row's NG-group span (4-bit:
// 8 words a group, 2-bit: 4): pieces and halves past the span repeat the
// first ones (cache hits), so the number of loads never depends on the width.
template <int NG>
FM_DEV uint32_t fmb_woff(int bits, int p, int h) {
    if (bits == 4) return (NG == 16 ? 64 * p : 0) + 16 * h;
    return NG == 16 ? 16 * h : 16 * (h & 1);
}

// The loads of gate/up unit (tile t, input quarter kq4) for intermediate rows
// RI c .. RI c + RI - 1 (RI = NG / 4): lane (n, kq) takes tile row n = row
// n % RI of the gate (up when (n / RI) odd) matrix of tile slot n / (2 RI).
// Always 8 code loads and 2 scale/bias loads: rows that do not exist or are
// invalid read `dummy`, so the number of loads in flight never depends on a
// branch.
template <int NG>
FM_DEV void fmb_issue_gu(const FmSlot *sl, const bool *ok, uint32_t c, int kq4, FmbUnit &u, int lane,
                         const void *dummy) {
    constexpr int RI = NG / 4, SPT = 8 / RI, GH = 4 * NG;
    const int n = lane & 15, kq = lane >> 4;
    const int hs = n / (2 * RI);
    const bool up = (n / RI) & 1;
    // per-lane selects of wave-uniform values (made opaque first: selects of
    // the struct fields themselves became loads through scratch)
    bool okl = false;
    int bits = 4;
    uint64_t W = 0, Sc = 0, Bi = 0;
#pragma unroll
    for (int j = 0; j < SPT; j++) {
        const bool me = hs == j;
        okl = me ? ok[j] : okl;
        bits = me ? fmb_u(sl[j].bits) : bits;
        W = me ? (up ? fmb_u(sl[j].uw) : fmb_u(sl[j].gw)) : W;
        Sc = me ? (up ? fmb_u(sl[j].us) : fmb_u(sl[j].gs)) : Sc;
        Bi = me ? (up ? fmb_u(sl[j].ub) : fmb_u(sl[j].gb)) : Bi;
    }
    const uint32_t row = RI * c + (n % RI);
    const uint32_t wpg = 2 * bits, wpr = GH * wpg;
    const uint32_t *base = okl ? (const uint32_t *)W + (size_t)row * wpr + NG * kq4 * wpg + 4 * kq
                               : (const uint32_t *)dummy + 4 * kq;
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int h = 0; h < 4; h++) u.v[p][h] = fm_ldg_u4_nt(base + (okl ? fmb_woff<NG>(bits, p, h) : 16 * h));
    const size_t o = (size_t)row * GH + NG * kq4 + 4 * (kq & (NG / 4 - 1));
    u.sc = *(const FM_GLOBAL fmm_u2 *)(okl ? (const uint16_t *)Sc + o : (const uint16_t *)dummy);
    u.bi = *(const FM_GLOBAL fmm_u2 *)(okl ? (const uint16_t *)Bi + o : (const uint16_t *)dummy);
}

// One 16-byte run per lane into LDS (lane l's run lands at lds + 16 l) by the
// vector memory DMA path.  Only the DMA waves issue these, so no other wave's
// compiler-inserted waits are stretched by them; the issuing wave waits for
// its own copies with an explicit vmcnt.
FM_DEV void fmb_dma16(void *lds, const void *g) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

// LDS-counter waits between the waves of the workgroup (bounded: a wait that
// gives up reports FM_STATUS_WAIT_TIMEOUT and lets the kernel finish).
FM_DEV void fmb_wait_lds(const FmDecodeArgs &a, const uint32_t *ctr, uint32_t target) {
    uint32_t it = 0;
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target && ++it < FM_SPIN_MAX)
        __builtin_amdgcn_s_sleep(1);
    if (it >= FM_SPIN_MAX && (threadIdx.x & 63) == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
    asm volatile("" ::: "memory");
}
FM_DEV void fmb_arrive(uint32_t *ctr) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One 64-element group of a vector held 16 values per lane (4 lanes per group,
// lane qq holds elements 16 qq .. 16 qq + 15) -> operand rows of layout `bits`
// (4-bit: pairs 8 qq .. 8 qq + 7 of the fmm_build_pair layout; 2-bit: pairs
// 8 qq .. + 7 of its 2-bit layout), the group's sum and 2^(24 - e).  Lanes
// with !st compute (the shuffles stay within each lane quad) but store nothing.
FM_DEV void fmb_build_group(const float (&v)[16], int qq, int bits, fm_h2 *dst, float *gsum, float *ginv,
                             bool st = true) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    const int ex = fm_group_shift(mx);
    const float f = fm_exp2i(ex);
    if (bits == 4) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float m = (j & 1) ? 0.0625f * f : f;
                if (st) dst[4 * (2 * qq + h) + j] = fm_pack_h2(v[8 * h + j] * m, v[8 * h + 4 + j] * m);
            }
    } else {
        const float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
        for (int n2 = 0; n2 < 8; n2++)
            if (st) dst[8 * qq + n2] = fm_pack_h2(v[n2] * (mt[n2] * f), v[8 + n2] * (mt[n2] * f));
    }
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
    sm += __shfl_xor(sm, 1, 64);
    sm += __shfl_xor(sm, 2, 64);
    if (st && qq == 0) {
        *gsum = sm;
        *ginv = fm_exp2i(24 - ex);
    }
}

// NG: input groups of a quarter of a gate/up row = hidden / 256 (16: hidden
// 4096 / inter 1024; 8: hidden 2048 / inter 512).  With inter = hidden / 4,
// workgroup c owns RI = NG / 4 intermediate rows and RD = NG output rows of
// every slot, and a 16-row gate/up tile holds SPT = 8 / RI slots' rows.
// RT: routing fused into the launch (FmDecodeArgs::route_logits).
// TAG: the activations are handed off as tagged words that each down wave
// polls (no flag round); otherwise as plain words behind one flag per CU.
template <int NG, bool RT, bool TAG>
__global__ __launch_bounds__(FMB_THREADS, 1) void fm_decode_bal_kernel(FmDecodeArgs a) {
    __shared__ FmbLds L;
    constexpr uint32_t H = 256 * NG, I = 64 * NG, GI = NG;
    constexpr int RI = NG / 4, RD = NG, SPT = 8 / RI;
    static_assert(H <= FMM_H && I <= FMM_MAXI, "LDS is sized for hidden 4096 / inter 1024");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, q = lane >> 4;
    const int S = a.S, NT = (S + SPT - 1) / SPT;
    const uint32_t c = blockIdx.x;

    if (RT && tid < FMC_THREADS / 8) L.rt.ck[tid] = 0;
    if (tid == 0) {
        L.xready = L.pdone = L.go = L.ydone = L.gu_issued = L.dn_ready = 0;
        if constexpr (RT) {
            L.rt.ncand = L.rt.pconv = 0;
            L.rt.vk = -1;
        }
    }
    __syncthreads();

    if (wv >= FMB_GU) {
        // ---- DMA waves: every slot's RD down rows into LDS, behind the gate/up loads ----
        float winv = 1.f;
        if constexpr (RT) {
            fmc_route_bystander(L);
            float s = 0.f;
            for (int k = 0; k < a.K; k++) s += __int_as_float(L.rp[k]);
            winv = s > 0.f ? 1.0f / s : 1.0f;
        }
        const int *rsel = RT ? L.rsel : nullptr;
        if (FMB_DN_AFTER_GU) fmb_wait_lds(a, &L.gu_issued, FMB_GU);
        // scale / bias runs of the tile: RD rows x GI groups x 2 B each, 16 B a lane
        constexpr int NSC = RD * GI * 2 / 16;
        for (int sd = wv - FMB_GU; sd < S; sd += FMB_W - FMB_GU) {
            const FmSlot sD = fmc_slot(a, sd, rsel, L.rp, winv);
            const bool okD = sD.valid;
            const uint32_t wpr = GI * 2 * sD.bits;
            const uint32_t *base =
                okD ? sD.dw + (size_t)(RD * c + n % RD) * wpr + 4 * q : (const uint32_t *)a.x + 4 * q;
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int h = 0; h < 4; h++)
                    fmb_dma16(&L.dn[sd][p][h][0], base + (okD ? fmb_woff<NG>(sD.bits, p, h) : 16 * h));
            const bool lsc = lane < 2 * NSC;
            const uint16_t *sb = lane < NSC ? sD.ds : sD.db;
            fmb_dma16(&L.dsb[sd][0][0], (okD && lsc) ? sb + (size_t)RD * c * GI + 8 * (lane % NSC)
                                                      : (const uint16_t *)a.x);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies have landed
        fmb_arrive(&L.dn_ready);
        return;
    }

    // ---- gate/up waves ----
    const uint32_t ep_ld = fm_epoch_load(a);
    float lgq[FMC_THREADS / 64];
    uint32_t etab = 0;
    if constexpr (RT) {
        etab = fm_expf_lanes_load();
#pragma unroll
        for (int j = 0; j < FMC_THREADS / 64; j++)
            lgq[j] = 64 * j + lane < a.route_E ? a.route_logits[64 * j + lane] : -INFINITY;
    }
    // x: the first H / 1024 waves, 16 elements a thread (thread t: elements 16 t .. 16 t + 15)
    constexpr int XT = (int)H / 16, XW = XT / 64;
    fm_f4 xr[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xr[j] = fm_ldg_f4(a.x + 16 * (tid < XT ? tid : 0) + 4 * j);
    // the shared expert's gate input, loaded before the weight stream so that
    // reading it waits for nothing else
    const float sscore = (wv == 0 && a.shared_score) ? a.shared_score[0] : 0.f;
    float winv = 1.f;
    if constexpr (RT) winv = fmc_route(a, L, lgq, etab);
    const int *rsel = RT ? L.rsel : nullptr;

    // gate/up units: wave w takes units w and w + 12 (unit u = tile u / 4, input quarter u % 4)
    const int t0 = wv >> 2, t1 = FMB_GU / 4 + (wv >> 2), kq4 = wv & 3;
    const bool has0 = t0 < NT, has1 = t1 < NT;
    FmSlot s0[SPT], s1[SPT];
    bool ok0[SPT], ok1[SPT];
#pragma unroll
    for (int j = 0; j < SPT; j++) {
        const int k0 = SPT * t0 + j, k1 = SPT * t1 + j;
        s0[j] = fmc_slot(a, has0 && k0 < S ? k0 : 0, rsel, L.rp, winv);
        s1[j] = fmc_slot(a, has1 && k1 < S ? k1 : 0, rsel, L.rp, winv);
        ok0[j] = has0 && k0 < S && s0[j].valid;
        ok1[j] = has1 && k1 < S && s1[j].valid;
    }
    FmbUnit u0, u1;
    fmb_issue_gu<NG>(s0, ok0, c, kq4, u0, lane, a.x);
    fmb_issue_gu<NG>(s1, ok1, c, kq4, u1, lane, a.x);
    if (FMB_DN_AFTER_GU) fmb_arrive(&L.gu_issued);
    // this wave's down slot (waves 0 .. S - 1)
    const int sd = wv;
    const bool down = wv < S;
    const FmSlot sD = fmc_slot(a, down ? sd : 0, rsel, L.rp, winv);
    const bool okD = down && sD.valid;
    if (wv == 0) {
        // the combine's slot weights and validity, and the shared gate
        uint32_t vm = 0;
#pragma unroll
        for (int kk = 0; kk < FM_MAX_SLOTS; kk++) {
            if (kk < S) {
                const FmSlot sk = fmc_slot(a, kk, rsel, L.rp, winv);
                if (lane == 0) L.cw[kk] = sk.weight;
                vm |= sk.valid ? 1u << kk : 0u;
            }
        }
        if (lane == 0) {
            L.cvalid = vm;
            L.sw = (a.has_shared || a.shared_y) ? (a.shared_score ? fm_sigmoid(sscore) : a.shared_w_host) : 0.f;
        }
    }
    // x -> operand rows (both layouts), group sums and scales: the first XW waves
    if (wv < XW) {
        if (tid < 32) L.zero[tid] = fm_as_h2(0u);
        const int g = tid >> 2, qq = tid & 3;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[4 * j] = xr[j].x;
            v[4 * j + 1] = xr[j].y;
            v[4 * j + 2] = xr[j].z;
            v[4 * j + 3] = xr[j].w;
        }
        fmb_build_group(v, qq, 4, &L.xq[0][g][0], &L.xsum[g], &L.xinv[g]);
        float unused_s, unused_i;
        fmb_build_group(v, qq, 2, &L.xq[1][g][0], &unused_s, &unused_i);
        fmb_arrive(&L.xready);
    }
    fmb_wait_lds(a, &L.xready, XW);
    const uint32_t ep = fm_epoch_tag(ep_ld);

    // ---- gate/up MMAs of the two units ----
    // the widths present in a tile (invalid rows take any: their sums are
    // never used); a tile of both widths runs both MMAs with the other
    // width's columns masked
    auto tile_bits = [&](const FmSlot *sl, const bool *ok, bool &w4, bool &w2) __attribute__((always_inline)) {
        w4 = w2 = false;
#pragma unroll
        for (int j = 0; j < SPT; j++) {
            w4 |= ok[j] && sl[j].bits == 4;
            w2 |= ok[j] && sl[j].bits == 2;
        }
    };
    auto unit_mma = [&](const FmbUnit &u, const FmSlot *sl, const bool *ok, int t) __attribute__((always_inline)) {
        bool w4, w2;
        tile_bits(sl, ok, w4, w2);
        fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
        const fm_h2 *x4 = &L.xq[0][NG * kq4][0], *x2 = &L.xq[1][NG * kq4][0];
        if (!(w4 && w2)) {
            if (!w2)
                fmb_mma<4, false, NG>(u.v, x4, L.zero, d0, d1, lane, true);
            else
                fmb_mma<2, false, NG>(u.v, x2, L.zero, d0, d1, lane, true);
        } else {
            int rb = 4;
#pragma unroll
            for (int j = 0; j < SPT; j++) rb = n / (2 * RI) == j ? sl[j].bits : rb;
            const bool col4 = rb == 4;
            fmb_mma<4, true, NG>(u.v, x4, L.zero, d0, d1, lane, col4);
            fmb_mma<2, true, NG>(u.v, x2, L.zero, d0, d1, lane, !col4);
        }
        const bool qok = 4 * q < NG;
        const int gq = NG * kq4 + 4 * (qok ? q : 0);
        float p = qok ? fmm_fold(d0 + d1, u.sc, u.bi, &L.xsum[gq], &L.xinv[gq]) : 0.f;
        p = fmm_q_sum(p);
        if (lane < 16) L.part[t][kq4][n] = p;
    };
    if (has0) unit_mma(u0, s0, ok0, t0);
    if (has1) unit_mma(u1, s1, ok1, t1);
    fmb_arrive(&L.pdone);
    if (RT && wv == FMB_GU - 1 && c == gridDim.x - 1) {
        // cpu_topk's slot order by serial replay, then cpu_normalize_weights
        // (sequential sum over the slots): bit-equal to fm_route_kernel.  This
        // wave holds no down tile (S <= 11), so the replay is off every chain.
        __builtin_amdgcn_s_setprio(3);
        const float pinv = L.rt.pconv ? 0.f : 1.0f / fm_serial_sum((const float *)L.rt.pb, a.route_E);
        fm_topk_serial(L.rt.pb, a.route_E, a.K, L.rt, pinv);
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

    // ---- wave 0: SwiGLU of the CU's RI S activations, publish, then wait for every CU ----
    // activation i of a slot is stored at (I / 16) (i % 16) + i / 16: a reader
    // lane l < I / 16 then holds elements 16 l .. 16 l + 15 with 16 coalesced loads
    float *actf = a.actf;
    if (wv == 0) {
        fmb_wait_lds(a, &L.pdone, FMB_GU);
        if (lane < 8 * NT) {
            const int t = lane >> 3, r8 = lane & 7, hs = r8 / RI, rr = r8 % RI, s = SPT * t + hs;
            const int ng = hs * 2 * RI + rr, nu = ng + RI;
            const float g = (L.part[t][0][ng] + L.part[t][1][ng]) + (L.part[t][2][ng] + L.part[t][3][ng]);
            const float u = (L.part[t][0][nu] + L.part[t][1][nu]) + (L.part[t][2][nu] + L.part[t][3][nu]);
            const uint32_t i = RI * c + rr;
            const size_t pos = (size_t)s * I + (I / 16) * (i & 15) + (i >> 4);
            if (s < S) {
                if (TAG)
                    fm_put_tagged(&a.act2[pos], fm_silu_mul(g, u), ep);
                else
                    __hip_atomic_store(&actf[pos], fm_silu_mul(g, u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (!TAG && wv == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the activations are at the coherence point
        if (lane == 0) fm_put_tagged(&a.flags[c], 0.f, ep);
        const uint32_t G = gridDim.x;
        uint64_t t[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            t[j] = 64 * j + lane < (int)G ? fm_get_tagged(&a.flags[64 * j + lane]) : ((uint64_t)ep << 32);
        uint32_t it = 0;
        do {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < 4; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
            if (__all(ready)) break;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(&a.flags[64 * j + lane]);
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        if (lane == 0) __hip_atomic_store(&L.go, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        // every CU's wave 0 has stored its flag, so every tag user of this
        // call has read the epoch: publish it for the next call
        if (c == 0 && lane == 0) fm_epoch_publish(a, ep);
    }

    // ---- down: the slot's activations -> operand rows, RD down rows from LDS ----
    if (down) {
        constexpr int AL = (int)I / 16;  // lanes holding activations
        const bool al = lane < AL;
        float v[16];
        if constexpr (TAG) {
            // the slot's I tagged activations (every CU stored RI of them)
            const uint64_t *src = a.act2 + (size_t)sd * I + (al ? lane : 0);
            uint64_t t[16];
#pragma unroll
            for (int i = 0; i < 16; i++) t[i] = fm_get_tagged(src + AL * i);
            uint32_t it = 0;
            do {
                bool ready = true;
#pragma unroll
                for (int i = 0; i < 16; i++) ready &= (uint32_t)(t[i] >> 32) == ep;
                if (__all(ready)) break;
#pragma unroll
                for (int i = 0; i < 16; i++)
                    if ((uint32_t)(t[i] >> 32) != ep) t[i] = fm_get_tagged(src + AL * i);
            } while (++it < FM_SPIN_MAX);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = __uint_as_float((uint32_t)t[i]);
            // slot sd's activations come from every CU, and every CU's wave 0
            // read the epoch before storing them: publish it for the next call
            if (sd == 0 && c == 0 && lane == 0) fm_epoch_publish(a, ep);
        } else {
            fmb_wait_lds(a, &L.go, 1);
#pragma unroll
            for (int i = 0; i < 16; i++)
                v[i] = __hip_atomic_load(&actf[(size_t)sd * I + AL * i + (al ? lane : 0)], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        }
        float y = 0.f;
        if (okD) {
            // lanes l < I / 16: group l / 4, elements 16 (l % 4) .. + 15
            const int g = al ? lane >> 2 : 0;
            fmb_build_group(v, lane & 3, sD.bits, &L.aq[sd][g][0], &L.asum[sd][g], &L.ainv[sd][g], al);
            fm_wave_lds_sync();
            fmb_wait_lds(a, &L.dn_ready, FMB_W - FMB_GU);
            fm_u4 dv[2][4];
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int h = 0; h < 4; h++) dv[p][h] = L.dn[sd][p][h][lane];
            fmm_f4 d0 = {0, 0, 0, 0}, d1 = d0;
            if (sD.bits == 4)
                fmb_mma<4, false, NG>(dv, &L.aq[sd][0][0], L.zero, d0, d1, lane, true);
            else
                fmb_mma<2, false, NG>(dv, &L.aq[sd][0][0], L.zero, d0, d1, lane, true);
            const bool qok = 4 * q < NG;
            const uint16_t *sbl = &L.dsb[sd][0][0];
            const int o = GI * (n % RD) + 4 * (qok ? q : 0);
            const fmm_u2 sc = *(const fmm_u2 *)&sbl[o];
            const fmm_u2 bi = *(const fmm_u2 *)&sbl[RD * GI + o];
            y = qok ? fmm_fold(d0 + d1, sc, bi, &L.asum[sd][4 * (qok ? q : 0)], &L.ainv[sd][4 * (qok ? q : 0)]) : 0.f;
            y = fmm_q_sum(y);
        }
        if (lane < RD) {
            if (a.mode == 1)
                a.expert_out[(size_t)sd * H + RD * c + n] = y;
            else
                L.y[sd][n] = y;
        }
        fmb_arrive(&L.ydone);
    }

    // ---- wave 0: the combine of the CU's RD rows over every slot, in slot order ----
    if (wv == 0 && a.mode == 0) {
        fmb_wait_lds(a, &L.ydone, (uint32_t)S);
        const uint32_t row = RD * c + (n % RD);
        float o = 0.f;
        if (lane < RD) {
            const uint32_t cv = L.cvalid;
            float moe = 0.f;
#pragma unroll
            for (int kk = 0; kk < FM_MAX_SLOTS; kk++)
                if (kk < a.K && ((cv >> kk) & 1u)) moe = __fadd_rn(moe, __fmul_rn(L.cw[kk], L.y[kk][lane]));
            o = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
            if (a.has_shared)
                o = __fadd_rn(o, __fmul_rn(L.sw, L.y[S - 1][lane]));
            else if (a.shared_y)
                o = __fadd_rn(o, __fmul_rn(L.sw, a.shared_y[row]));
            a.out[row] = o;
            if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(o);
        }
        if (a.norm_w) {
            // next layer's input RMS norm (cpu_kernels.h:235-246): every CU
            // publishes the sum of squares of its RD rows (tagged), then every
            // CU adds all of them in the same fixed order (all 64 lanes here)
            const float sq = fm_lane_sum<16>(lane < RD ? o * o : 0.f);
            const uint32_t G = gridDim.x;
            uint64_t *ssq = a.flags + G;
            if (lane == 0) fm_put_tagged(&ssq[c], sq, ep);
            uint64_t t[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                t[j] = 64 * j + lane < (int)G ? fm_get_tagged(&ssq[64 * j + lane]) : ((uint64_t)ep << 32);
            uint32_t it = 0;
            do {
                bool ready = true;
#pragma unroll
                for (int j = 0; j < 4; j++) ready &= (uint32_t)(t[j] >> 32) == ep;
                if (__all(ready)) break;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if ((uint32_t)(t[j] >> 32) != ep) t[j] = fm_get_tagged(&ssq[64 * j + lane]);
            } while (++it < FM_SPIN_MAX);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
            float part = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) part += 64 * j + lane < (int)G ? __uint_as_float((uint32_t)t[j]) : 0.f;
            const float tot = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fm_lane_sum<64>(part))));
            const float inv = 1.0f / sqrtf(tot / (float)H + a.norm_eps);
            if (lane < RD) a.normed[row] = o * inv * fm_bf16_to_f32(a.norm_w[row]);
        }
    }
    if (a.pool_mode && !RT && c == 0 && tid < a.K) {
        const int e = a.idx[tid];
        if (e < 0 || (uint32_t)e >= a.pool_n) atomicOr(a.err, FM_STATUS_BAD_EXPERT);  // skipped (invalid slot)
    }
}

// hidden 4096 / inter 1024 or hidden 2048 / inter 512, 1 .. 11 slots a token:
// one workgroup per CU for the 256 row blocks (every one must be resident:
// each waits for all the others' activations).  Several tokens (pool mode, the
// combine, no fused norm) run as one launch per token on the same workspace
// (each launch tags with its own epoch).
template <int NG>
static void (*fmb_kernel(bool rt, bool tagged))(FmDecodeArgs) {
    return rt ? (tagged ? fm_decode_bal_kernel<NG, true, true> : fm_decode_bal_kernel<NG, true, false>)
              : (tagged ? fm_decode_bal_kernel<NG, false, true> : fm_decode_bal_kernel<NG, false, false>);
}

int fm_launch_decode_bal(FmDecodeArgs &a, hipStream_t st) {
    // opt-in (FMOE_DECODE_BAL=1) until it has been measured on the GPU;
    // FMOE_DECODE_NO_BAL set: off
    const char *on = getenv("FMOE_DECODE_BAL"), *off = getenv("FMOE_DECODE_NO_BAL");
    if (!(on && *on == '1') || (off && *off)) return fm_fail(FM_ERR_UNSUPPORTED, "bal decode: disabled");
    const int ntok = a.ntok > 1 ? a.ntok : 1, spt = ntok > 1 ? a.spt : a.S;
    const int ng = a.hidden == 4096 && a.inter == 1024 ? 16 : (a.hidden == 2048 && a.inter == 512 ? 8 : 0);
    if (!ng || spt < 1 || spt > FMB_MAXS || (a.norm_w && a.mode != 0) || !a.actf || !a.flags)
        return fm_fail(FM_ERR_UNSUPPORTED, "bal decode: shape");
    if (ntok > 1 && (!a.pool_mode || a.mode != 0 || a.norm_w || a.route_logits || a.S != ntok * spt))
        return fm_fail(FM_ERR_UNSUPPORTED, "bal decode: several tokens need pool mode and the combine");
    if (a.route_logits && !(a.mode == 0 && a.pool_mode && a.K >= 1 && a.K <= 64 && a.route_E >= a.K &&
                            a.route_E <= FMC_THREADS))
        return fm_fail(FM_ERR_UNSUPPORTED, "bal decode: fused routing");
    const uint32_t grid = 256;  // hidden / (output rows of a workgroup)
    static int per_cu = -1;
    if (per_cu < 0 &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fm_decode_bal_kernel<16, false, false>, FMB_THREADS,
                                                     0) != hipSuccess)
        per_cu = 0;
    if (per_cu < 1 || (uint32_t)(per_cu * fm_num_cus()) < grid)
        return fm_fail(FM_ERR_UNSUPPORTED, "bal decode: %u workgroups not resident", grid);
    // FMOE_BAL_TAGGED=1: the tagged-activation hand-off (measured against the flag round)
    const char *tg = getenv("FMOE_BAL_TAGGED");
    const bool tagged = tg && *tg == '1';
    const size_t H = a.hidden;
    for (int t = 0; t < ntok; t++) {
        FmDecodeArgs b = a;
        if (ntok > 1) {
            b.ntok = 1;
            b.spt = b.S = spt;
            b.idx = a.idx + (size_t)t * a.K;
            b.wdev = a.wdev + (size_t)t * a.K;
            b.x = a.x + (size_t)t * H;
            b.out = a.out + (size_t)t * H;
            if (a.h_mid) b.h_mid = a.h_mid + (size_t)t * H;
            if (a.out_bf16) b.out_bf16 = a.out_bf16 + (size_t)t * H;
            if (a.shared_score) b.shared_score = a.shared_score + t;
        }
        void (*kern)(FmDecodeArgs) = ng == 16 ? fmb_kernel<16>(b.route_logits, tagged) : fmb_kernel<8>(b.route_logits, tagged);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(FMB_THREADS), 0, st, b);
        const int rc = fm_check_launch("fm_decode_bal_kernel");
        if (rc) return rc;
    }
    return FM_OK;
}
