// fm_route_cu.h -- routing of one token inside a one-workgroup-per-CU decode
// launch (768 threads): cpu_softmax / cpu_topk / cpu_normalize_weights
// (cpu_kernels.h:263-309) computed by every workgroup from the logits.
#pragma once
#include "fm_decode.h"
#include "fm_expf.h"
#include "fm_route_dev.h"

#ifndef FM_DX_MARK
#define FM_DX_MARK(n)
#endif

#define FMC_THREADS 768  // threads of the per-CU decode kernels (12 wavefronts)

// Routing fused into the step (FmDecodeArgs::route_logits): scratch of the
// prologue, and of the one wavefront that writes the slot-order outputs.
struct __attribute__((aligned(16))) FmcRoute {
    int pb[FMC_THREADS];              // exp(l - max) bits (probability bits once pconv), -2 past E
    int cv[FMC_THREADS + 4];          // top-K candidates: probability bits
    int ci[FMC_THREADS + 4];          // ... and element indices
    uint64_t ck[FMC_THREADS / 8];     // ... and their ranking keys (e bits, then 1023 - index), zero past the count
    float red[FMC_THREADS / 64];      // per-wave sums of exp(l - max)
    float inv;                        // 1 / softmax sum (per-wave sums: the kernel's own weights)
    int ncand, ek1, vk, pconv;        // candidates; e bits at places K - 1 and K; pb holds exact p
    float s_val[64];                  // cpu_topk slots (serial replay)
    int s_id[64];
};

// Whether the set chosen on e is cpu_topk's set whatever the softmax sum
// (see fmc_route); read after the prologue's second barrier.
FM_DEV bool fmc_set_exact(const FmcRoute &R) {
    const int ek1 = R.ek1, ekk = R.vk;
    return ekk < 0 || (ek1 >= 0x0d800000 /* 2^-100 */ && ek1 - ekk >= 4);
}

// Routing of one token in every workgroup of the one-workgroup-per-CU kernel
// (FmDecodeArgs::route_logits): cpu_softmax / cpu_topk / cpu_normalize_weights
// (cpu_kernels.h:263-309).  Every wave holds all E <= FMC_THREADS logits.
//  * softmax with the arithmetic of fm_route_kernel (same per-wave sums, added
//    in wave order; the waves past E add zeros), so the probabilities are
//    bit-equal to that kernel's;
//  * the top-K SET, chosen on e = exp(l - max) while the sum is still being
//    exchanged: any element of the K largest lies at or above the K-th largest
//    of its own 64-element chunk, so the chunk lower bounds of
//    fm_kth_lower_bound keep ~K candidates a chunk, and each candidate counts
//    the candidates ahead of it (larger e, or equal e and a lower index).
//    p = e * (1 / sum) is monotone in e, so unless p at the K-th place equals
//    p at the (K+1)-th, the K first are exactly cpu_topk's slots (a strictly
//    larger newcomer is needed to evict, and it can only evict an element with
//    K others at or above it); with equal p across that place wavefront 0
//    replays cpu_topk (fm_topk_serial), which settles which of them stay.
// L.rsel / L.rp receive the set in descending order (the kernel's slot order:
// only the order of the weighted sum differs from cpu_topk's slots, a
// rounding-level difference); returns 1 / sum of the selected probabilities,
// the renormalisation factor (computed by every wave alike).
template <class LT>
FM_DEV float fmc_route(const FmDecodeArgs &a, LT &L, const float *lgq, uint32_t etab) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int E = a.route_E, K = a.K, nch = (E + 63) >> 6;
    constexpr int NW = FMC_THREADS / 64;
    FmcRoute &R = L.rt;
    // every wave holds all E logits (lane l: elements l, 64 + l, ...): the
    // max needs no exchange between waves
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NW; q++) mx = fmaxf(mx, lgq[q]);
    mx = fm_wave_max(mx);
    FM_DX_MARK(8);
    float lg = lgq[0];
#pragma unroll
    for (int q = 1; q < NW; q++) lg = wv == q ? lgq[q] : lg;
    // the reference libm's exp, bit for bit (every lane active: fm_expf_lanes)
    const float ex = fm_expf_lanes(lg - mx, etab);
    const float ev = tid < E ? ex : 0.f;
    const float ws = fm_lane_sum<64>(ev);
    if (lane == 0) R.red[wv] = ws;
    // candidates on e = exp(l - max), before the sum is known: p = e * (1 /
    // sum) is monotone in e, so the K largest by e are cpu_topk's set unless
    // p rounds equal across the K-th place (checked below on p itself)
    const int eb = tid < E ? __float_as_int(ev) : -2;
    if (tid < nch * 64) R.pb[tid] = eb;
    if (wv < nch) {
        const int res = fm_kth_lower_bound(eb, K);
        const uint64_t m = __ballot(eb >= res);
        int base = 0;
        if (lane == 0) base = atomicAdd(&R.ncand, __builtin_popcountll(m));
        base = __builtin_amdgcn_readlane(base, 0);
        if ((m >> lane) & 1ull) {
            const int pos = base + fm_mbcnt(m);
            R.cv[pos] = eb;
            R.ci[pos] = tid;
            if (pos < FMC_THREADS / 8) R.ck[pos] = ((uint64_t)(uint32_t)eb << 32) | (uint32_t)(1023 - tid);
        }
    }
    __syncthreads();
    FM_DX_MARK(10);
    const int NC = R.ncand;
    // a candidate's place = the number of candidates ahead of it by the key
    // (e bits, then the lower index first): unique places, so place K - 1 is
    // the last selected and place K the first left out
    float inv = 0.f;
    if (NC <= FMC_THREADS / 8) {
        // eight lanes per candidate (lane r: keys 12 r .. 12 r + 11, zero past
        // the count, so no bound check), counts summed over the 8 lanes
        // (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror)
        const int c = tid >> 3, r = tid & 7;
        const bool act = c < NC;
        const uint64_t key = act ? R.ck[c] : 0;
        int cnt = 0;
        if (act) {
            uint64_t kk[12];
#pragma unroll
            for (int h = 0; h < 6; h++) {
                const fm_u4 v = *reinterpret_cast<const fm_u4 *>(&R.ck[12 * r + 2 * h]);
                kk[2 * h] = ((uint64_t)v.y << 32) | v.x;
                kk[2 * h + 1] = ((uint64_t)v.w << 32) | v.z;
            }
#pragma unroll
            for (int j = 0; j < 12; j++) cnt += kk[j] > key ? 1 : 0;
        }
        cnt += fm_dpp_i<0xB1>(cnt);
        cnt += fm_dpp_i<0x4E>(cnt);
        cnt += fm_dpp_i<0x141>(cnt);
        // the softmax sum with fm_route_kernel's arithmetic (the same per-wave
        // sums added in wave order; waves past E add zeros), so p is bit-equal
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) sum += R.red[w];
        inv = 1.0f / sum;
        if (act && r == 0) {
            const int pbits = __float_as_int(__int_as_float((int)(key >> 32)) * inv);
            if (cnt < K) {
                L.rsel[cnt] = (int)(1023 - (uint32_t)key);
                L.rp[cnt] = pbits;
            }
            if (cnt == K - 1) R.ek1 = (int)(key >> 32);
            if (cnt == K) R.vk = (int)(key >> 32);
        }
    } else {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) sum += R.red[w];
        inv = 1.0f / sum;
    }
    if (NC > FMC_THREADS / 8 && tid < NC) {
        const int v = R.cv[tid], me = R.ci[tid];
        int pos = 0;
        for (int j = 0; j < NC; j += 4) {
            const int4 c = *reinterpret_cast<const int4 *>(&R.cv[j]);
            const int4 d = *reinterpret_cast<const int4 *>(&R.ci[j]);
            const int cc[4] = {c.x, c.y, c.z, c.w}, dd[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
            for (int q = 0; q < 4; q++) pos += j + q < NC && (cc[q] > v || (cc[q] == v && dd[q] < me));
        }
        const int pbits = __float_as_int(__int_as_float(v) * inv);
        if (pos < K) {
            L.rsel[pos] = me;
            L.rp[pos] = pbits;
        }
        if (pos == K - 1) R.ek1 = v;
        if (pos == K) R.vk = v;
    }
    if (tid == 0) R.inv = inv;
    __syncthreads();
    FM_DX_MARK(11);
    // The set by e is cpu_topk's set when p = e * (1 / sum) cannot round equal
    // across the K-th place, whatever the sum: e at place K - 1 at least 4 ulps
    // above e at place K (p then differs by more than one rounding on each
    // side) and large enough that p stays a normal number (sum <= E, so
    // p >= e / 1024).  Otherwise (near-equal e there, a rare case) wavefront
    // 0 derives p exactly -- cpu_softmax's sum in index order -- and replays
    // cpu_topk on it.  Uniform (read after the barrier).
    if (!fmc_set_exact(R)) {
        if (wv == 0) {
            const float pinv = 1.0f / fm_serial_sum((const float *)R.pb, E);
            fm_wave_lds_sync();
            for (int i = lane; i < nch * 64; i += 64) {
                const int v = R.pb[i];
                R.pb[i] = v >= 0 ? __float_as_int(__int_as_float(v) * pinv) : v;
            }
            fm_wave_lds_sync();
            fm_topk_serial(R.pb, E, K, R);
            fm_wave_lds_sync();
            if (lane < K) {
                L.rsel[lane] = R.s_id[lane];
                L.rp[lane] = __float_as_int(R.s_val[lane]);
            }
            if (lane == 0) R.pconv = 1;
        }
        __syncthreads();
    }
    float s = 0.f;
    for (int k = 0; k < K; k++) s += __int_as_float(L.rp[k]);
    return s > 0.f ? 1.0f / s : 1.0f;
}

// The workgroup barriers of fmc_route, for the waves of a workgroup larger
// than FMC_THREADS that take no part in the routing (every wave of a
// workgroup must reach each barrier).
template <class LT>
FM_DEV void fmc_route_bystander(LT &L) {
    __syncthreads();
    __syncthreads();
    if (!fmc_set_exact(L.rt)) __syncthreads();
}
