// fm_route_dev.h -- device building blocks of the top-K routing's small path
// (E <= 1024), written for any number of wavefronts NW per workgroup
// (wavefront w handles chunks w, w + NW, ...); the routing kernel
// (fm_route.hip) runs them with 16.  The algorithm and its reference
// semantics (cpu_topk, cpu_kernels.h:280-299) are described at the top of
// fm_route.hip.
#pragma once
#include "fm_device.h"

#define FM_RT_SMALL_NCH 16  // chunks of 64 of the small path (E <= 1024)
#ifndef FM_RT_MARK
#define FM_RT_MARK(n)
#define FM_RT_DECL
#endif

// cpu_softmax's sum (cpu_kernels.h:269-273): v[0] + v[1] + ... in index
// order, one rounding per term, so the sum -- and 1 / sum -- are bit-equal to
// the reference's.  One wavefront, every lane active; v (LDS, 16-byte
// aligned) holds n >= 1 floats >= 0.  Blocks of 512: lane l holds terms
// 8l .. 8l + 7 in registers, and the running sum walks the lanes -- lane l
// adds its 8 terms to what lane l - 1 handed it (DPP wave_shr:1), so the
// chain is 9 VALU operations per 8 terms with no memory access in it.
// Terms past n are +0, which leave a sum >= +0 unchanged.  Returns the sum in
// every lane.
FM_DEV float fm_serial_sum(const float *v, int n) {
    const int lane = threadIdx.x & 63;
    float carry = 0.f;
    for (int b = 0; b < n; b += 512) {
        float r[8];
        const int i0 = b + 8 * lane;
        if (i0 + 8 <= n) {
            const fm_f4 lo = *(const fm_f4 *)(v + i0), hi = *(const fm_f4 *)(v + i0 + 4);
            r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
            r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) r[j] = i0 + j < n ? v[i0 + j] : 0.f;
        }
        float s = lane == 0 ? carry : 0.f;
        float t = s;
        for (int l = 0; l < 64; l++) {
            t = s;
#pragma unroll
            for (int j = 0; j < 8; j++) t = __fadd_rn(t, r[j]);
            // lane l + 1 continues from lane l's sum
            s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x138, 0xF, 0xF, false));
        }
        carry = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 63));
    }
    return carry;
}

FM_DEV float fm_wave_max(float v) {
    v = fmaxf(v, fm_dpp_f<0xB1>(v));
    v = fmaxf(v, fm_dpp_f<0x4E>(v));
    v = fmaxf(v, fm_dpp_f<0x124>(v));
    v = fmaxf(v, fm_dpp_f<0x128>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

FM_DEV int fm_wave_max_i(int v) {
    v = max(v, fm_dpp_i<0xB1>(v));
    v = max(v, fm_dpp_i<0x4E>(v));
    v = max(v, fm_dpp_i<0x124>(v));
    v = max(v, fm_dpp_i<0x128>(v));
    const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return max(max(r0, r1), max(r2, r3));
}

FM_DEV int fm_wave_sum_i(int v) {
    v += fm_dpp_i<0xB1>(v);
    v += fm_dpp_i<0x4E>(v);
    v += fm_dpp_i<0x124>(v);
    v += fm_dpp_i<0x128>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}

// Inclusive prefix sum across the wavefront.
FM_DEV int fm_wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
}

// Largest value with the low FM_RT_KTH_LOW bits clear that at least K lanes
// reach: a lower bound of the wave's K-th largest (bitwise radix select over
// the high bits; the low bits would only tighten the bound slightly).
#define FM_RT_KTH_LOW 16
FM_DEV int fm_kth_lower_bound(int x, int K) {
    int res = 0;
#pragma unroll
    for (int b = 30; b >= FM_RT_KTH_LOW; b--) {
        const int cand = res | (1 << b);
        if (__builtin_popcountll(__ballot(x >= cand)) >= K) res = cand;
    }
    return res;
}

// Row-local (16-lane) DPP shift right by N; lanes without a source get `fill`.
template <int N>
FM_DEV int fm_row_shr(int v, int fill) {
    return __builtin_amdgcn_update_dpp(fill, v, 0x110 + N, 0xF, 0xF, false);
}

FM_DEV int fm_mbcnt(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0));
}

FM_DEV void fm_wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Serial replay on one wavefront (fallback): exact for ties.  The K slot keys
// are kept sorted across lanes (lane 0 = the minimum, lowest slot first among
// equal values); an insertion shifts the smaller keys down one lane.
// pscale != 0: pb holds exp bits and the probabilities are exp * pscale
// (scaled on the fly, pb is not written).
template <class LDS>
__device__ void fm_topk_serial(const int *pb, int E, int K, LDS &L, float pscale = 0.f) {
    const int lane = threadIdx.x & 63;
    int kval = lane < K ? -1 : 0x7fffffff;
    int kslot = lane < K ? lane : 64;
    int kid = 0;
    int thr = -1;
    for (int base = 0; base < E; base += 64) {
        const int i = base + lane;
        int p = i < E ? pb[i] : -2;
        if (pscale != 0.f && p >= 0) p = __float_as_int(__int_as_float(p) * pscale);
        uint64_t cand = __ballot(p > thr);
        while (cand) {
            const int j = __builtin_ctzll(cand);
            cand &= cand - 1;
            const int pj = __builtin_amdgcn_readlane(p, j);
            if (pj <= thr) continue;
            const int vslot = __builtin_amdgcn_readfirstlane(kslot);
            const bool less = lane >= 1 && lane < K && (kval < pj || (kval == pj && kslot < vslot));
            const int pos = __builtin_popcountll(__ballot(less));
            // lane i <- lane i+1 (DPP wave_shl:1)
            const int nval = fm_dpp_i<0x130>(kval);
            const int nslot = fm_dpp_i<0x130>(kslot);
            const int nid = fm_dpp_i<0x130>(kid);
            if (lane < pos) {
                kval = nval;
                kslot = nslot;
                kid = nid;
            } else if (lane == pos) {
                kval = pj;
                kslot = vslot;
                kid = base + j;
            }
            thr = __builtin_amdgcn_readfirstlane(kval);
        }
    }
    if (lane < K) {
        L.s_val[kslot] = __int_as_float(kval);
        L.s_id[kslot] = kid;
    }
}

// Top-K slots for E <= 64 * FM_RT_SMALL_NCH, one element per thread
// (wavefront w holds chunk w in pv), called by the whole workgroup once pb,
// the per-chunk lower bounds kth[] and the lists big[] are in LDS.  The tests
// are lane-parallel VALU counts (one CU scalar unit serves all 16
// wavefronts, so per-element ballot chains would serialise there):
//  - chunk 0 has no bound: c_i = #{j < i : p_j >= p_i} is summed over all
//    wavefronts, wavefront w adding the four j in [4w, 4w+4);
//  - the survivors p_i > L_c of every chunk c >= 1 go into one flat list, and
//    thread (s, c') counts the elements of chunk c' at or above survivor s: an
//    earlier element p_j >= p_i > L_c >= kth[c'] is in big[c'], and an element
//    of the own chunk p_j >= p_i is itself a survivor, so every count runs over
//    a short list; the 16 counts of a survivor are summed across a DPP row.
// When U (initial elements plus insertions) fits one wavefront, wavefront 0
// then ranks U, inverts the ranks and pointer-jumps the eviction chains in
// registers.  Returns false (uniformly) when U is larger than a wavefront and
// the general path must finish the job.
template <int NW, class LDS>
__device__ bool fm_route_small(const int *pb, const int *pvq, int E, int K, int nch, LDS &L) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    // lane c of lb: L_c = max over c' < c of kth[c'] (-1 for chunk 0)
    int lb = lane < nch - 1 ? L.kth[lane] : -1;
    lb = max(lb, fm_row_shr<1>(lb, -1));
    lb = max(lb, fm_row_shr<2>(lb, -1));
    lb = max(lb, fm_row_shr<4>(lb, -1));
    lb = max(lb, fm_row_shr<8>(lb, -1));
    lb = fm_row_shr<1>(lb, -1);
    {
        // wavefront w adds the j in [JW w, JW w + JW)
        constexpr int JW = 64 / NW;
        const int q0 = pb[lane];
        int part = 0;
#pragma unroll
        for (int h = 0; h < JW; h += 4) {
            const int j0 = JW * wv + h;
            const int4 pj = *reinterpret_cast<const int4 *>(&pb[j0]);
            part += (lane > j0 && pj.x >= q0) + (lane > j0 + 1 && pj.y >= q0) + (lane > j0 + 2 && pj.z >= q0) +
                    (lane > j0 + 3 && pj.w >= q0);
        }
        if (part) atomicAdd(&L.c0cnt[lane], part);
    }
    FM_RT_MARK(11);
    constexpr int QW = FM_RT_SMALL_NCH / NW;  // chunks per wavefront: c = wv + NW q
#pragma unroll
    for (int qq = 0; qq < QW; qq++) {
        const int c = wv + NW * qq;
        const int pv = pvq[qq];
        const int lc = __builtin_amdgcn_readlane(lb, c & 15);
        if (c >= 1 && c < nch) {
            // survivors of chunk c (padding -2 never passes; every i >= 64 >= K): listed in
            // lane order per chunk, and in one flat list over all chunks
            const uint64_t own = __ballot(pv > lc);
            const int ns = __builtin_popcountll(own);
            const bool mine = (own >> lane) & 1ull;
            const int r = fm_mbcnt(own);
            int base = 0;
            if (lane == 0 && ns) base = atomicAdd(&L.nsurv, ns);
            base = __builtin_amdgcn_readlane(base, 0);
            if (mine) {
                L.sv[c][r] = pv;
                L.S_v[base + r] = pv;
                L.S_p[base + r] = (c * 64 + lane) * 64 + r;
            }
        }
    }
    FM_RT_MARK(12);
    __syncthreads();
    // c_i = #{j < i : p_j >= p_i} for every survivor, thread (s, c') counting the
    // elements of chunk c' at or above p_s: an earlier chunk's are in its big[] list
    // (p_j >= p_s > L_c >= kth[c']), the own chunk's are survivors listed before s.
    // The 16 threads of survivor s are one DPP row; their sum decides the insertion.
    {
        const int NS = L.nsurv;
        const int cp = tid & 15;
        for (int s0 = 0; s0 < NS; s0 += 4 * NW) {
            const int sidx = s0 + (tid >> 4);
            const bool act = sidx < NS;
            const int v = act ? L.S_v[sidx] : 0x7fffffff;
            const int sp = act ? L.S_p[sidx] : 0;
            const int i = sp >> 6, rs = sp & 63, cs = i >> 6;
            // the first 16 entries of either list in four loads issued together; entries
            // past a list's end are -2 (big[]) or masked by index (sv[])
            const bool own_chunk = act && cp == cs;
            const int *lst = own_chunk ? &L.sv[cs][0] : &L.big[cp][0];
            const int n = !act || cp > cs ? 0 : own_chunk ? rs : L.nbig[cp];
            int cnt = 0;
            if (n > 0) {
                int4 e[4];
#pragma unroll
                for (int h = 0; h < 4; h++) e[h] = *reinterpret_cast<const int4 *>(lst + 4 * h);
#pragma unroll
                for (int h = 0; h < 4; h++)
                    cnt += (4 * h < n && e[h].x >= v) + (4 * h + 1 < n && e[h].y >= v) +
                           (4 * h + 2 < n && e[h].z >= v) + (4 * h + 3 < n && e[h].w >= v);
                for (int k = 16; k < n; k++) cnt += lst[k] >= v;  // long lists (K > 12, ties at the bound)
            }
            cnt += fm_row_shr<1>(cnt, 0);
            cnt += fm_row_shr<2>(cnt, 0);
            cnt += fm_row_shr<4>(cnt, 0);
            cnt += fm_row_shr<8>(cnt, 0);
            if (act && cp == 15 && cnt < K) atomicOr(&L.ins[cs], 1ull << (i & 63));
        }
    }
    __syncthreads();
    FM_RT_MARK(7);
    const uint64_t ins0 = __ballot(lane >= K && lane < E && L.c0cnt[lane] < K);
    const uint64_t im = lane == 0 ? ins0 : lane < nch ? L.ins[lane] : 0ull;
    if (tid == 0) L.ins[0] = ins0;  // for the general path (read after its next barrier)
    const int cnt = __builtin_popcountll(im);
    int incl = cnt;
    incl += fm_row_shr<1>(incl, 0);
    incl += fm_row_shr<2>(incl, 0);
    incl += fm_row_shr<4>(incl, 0);
    incl += fm_row_shr<8>(incl, 0);
    const int M = __builtin_amdgcn_readlane(incl, 15);
    const int NU = K + M;
    if (NU > 64) return false;
    // U in LDS: position u < K holds initial element u, insertions follow in index order
    // (cross-lane reads stay outside lane-divergent code: an inactive lane's value is undefined there)
#pragma unroll
    for (int qq = 0; qq < QW; qq++) {
        const int c = wv + NW * qq;
        const int pre = __builtin_amdgcn_readlane(incl - cnt, c & 15);
        if (c < nch) {
            const uint64_t mc = ((uint64_t)(unsigned)__builtin_amdgcn_readlane((int)(im >> 32), c & 15) << 32) |
                                (unsigned)__builtin_amdgcn_readlane((int)im, c & 15);
            if ((mc >> lane) & 1ull) {
                const int pos = K + pre + fm_mbcnt(mc);
                L.U[pos] = c * 64 + lane;
                L.Uv[pos] = pvq[qq];
            }
        }
    }
    if (wv == 0) {
        if (lane < K) {
            L.U[lane] = lane;
            L.Uv[lane] = pvq[0];
        } else if (lane >= NU) {
            L.Uv[lane] = 0x7fffffff;
        }
    }
    __syncthreads();
    FM_RT_MARK(3);
    if (wv == 0) {
        const bool valid = lane < NU;
        const int vu = L.Uv[lane];
        const int uu = L.U[lane];
        // ascending rank; distinct values give a permutation of 0..NU-1
        int r = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int4 vw[8];
#pragma unroll
            for (int w = 0; w < 8; w++) vw[w] = *reinterpret_cast<const int4 *>(&L.Uv[32 * h + 4 * w]);
#pragma unroll
            for (int w = 0; w < 8; w++) r += (vw[w].x < vu) + (vw[w].y < vu) + (vw[w].z < vu) + (vw[w].w < vu);
        }
        FM_RT_MARK(9);
        if (fm_wave_sum_i(valid ? r : 0) != NU * (NU - 1) / 2) {
            fm_topk_serial(pb, E, K, L);  // equal probabilities inside U
        } else {
            if (valid) L.tor[r] = lane;
            fm_wave_lds_sync();
            // x_m (position K+m-1) evicts the slot of the element of rank m-1
            int ptr = lane < K ? lane : (valid ? L.tor[lane - K] : lane);
            // chains are shorter than 64: six doublings reach every root
            for (int round = 0; round < 6; round++) {
                const int nx = __builtin_amdgcn_ds_bpermute(ptr << 2, ptr);
                if (!__ballot(nx != ptr)) break;  // every chain at its root
                ptr = nx;
            }
            FM_RT_MARK(10);
            // the K largest (ranks M .. NU-1) are the final slots
            if (valid && r >= M) {
                L.s_id[ptr] = uu;
                L.s_val[ptr] = __int_as_float(vu);
            }
        }
    }
    return true;
}

// Per-chunk lower bound of the K-th largest and the chunk's values at or above
// it, for every chunk but the last (wavefront w handles chunks w + NW q, whose
// values it holds in pvq[q]).  The only elements a later survivor, being
// above the bound, can be compared unfavourably with are in these lists.
template <int NW, class LDS>
__device__ void fm_route_prep(const int *pvq, int K, int nch, LDS &L) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int qq = 0; qq < FM_RT_SMALL_NCH / NW; qq++) {
        const int c = wv + NW * qq;
        if (c < nch - 1) {
            const int pv = pvq[qq];
            const int res = fm_kth_lower_bound(pv, K);
            const uint64_t bm = __ballot(pv >= res);
            const int n = __builtin_popcountll(bm);
            const int below = fm_mbcnt(bm);  // members below this lane; the others pad from n on
            L.big[c][((bm >> lane) & 1ull) ? below : n + lane - below] = ((bm >> lane) & 1ull) ? pv : -2;
            if (lane < 4) L.big[c][64 + lane] = -2;
            if (lane == 0) {
                L.kth[c] = res;
                L.nbig[c] = n;
            }
        }
    }
}
