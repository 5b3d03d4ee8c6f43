// fm_route.hip -- softmax / top-K / renormalise on the device.
//
// Semantics of cpu_softmax, cpu_topk and cpu_normalize_weights
// (cpu_kernels.h:263-309) as called at layer_forward.h:3519-3523 and
// batched_prefill.h:256-261.  One 1024-thread workgroup per token.
//
// cpu_topk returns its K slots in SLOT order, which depends on the history of
// replacements: slots start at -1e30; element i evicts the first slot holding
// the minimum iff p_i > that minimum.  A serial replay of that history is a
// long dependent chain (~10 us for E = 512 on one wavefront), so the kernel
// derives the same answer in parallel from two facts:
//
//  (1) the slot values are always the top-K multiset of the prefix, so element
//      i (i >= K) is ever inserted iff  c_i = #{j < i : p_j >= p_i} < K;  the
//      first K elements fill slots 0..K-1 in order.  Let U = [0..K-1, x_1..x_M]
//      be the initial elements followed by the inserted ones in index order.
//  (2) every eviction removes the current minimum, evicted values never
//      decrease and every later insertion is larger than all of them, so the
//      m-th insertion x_m evicts exactly the m-th smallest element of U.
//
// Hence slot(x_m) = slot(m-th smallest of U): one rank sort of U plus pointer
// jumping.  (1) is evaluated for few elements only: with the array cut into
// 64-element chunks, the K-th largest value of any earlier chunk is a lower
// bound of the prefix's K-th largest, so element i of chunk c can only be
// inserted if p_i exceeds L_c = max over chunks c' < c of their K-th largest.
// The survivors of that filter get their exact c_i by a wave-wide count.
// Exact ties inside U (equal probabilities), more than FM_RT_UMAX entries or
// a filter too weak to pay off (K near 64) fall back to the serial replay on
// one wavefront.
// Probabilities are >= 0, so their IEEE bit patterns order like signed ints;
// -1e30 (the initial slot value) is represented by -1 and padding by -2.
#include "fm_device.h"
#include "fm_internal.h"
#include "fm_route_dev.h"

#define FM_RT_THREADS 1024
#define FM_RT_NW (FM_RT_THREADS / 64)
#define FM_RT_UMAX 256  // capacity of U (initial + inserted elements)
#define FM_RT_MAXE 4096
#ifndef FM_RT_MAX_PASSES
#define FM_RT_MAX_PASSES (24 * FM_RT_NW)  // above this the serial replay is cheaper
#endif
#define FM_RT_VPT (FM_RT_MAXE / FM_RT_THREADS)  // logits per thread

struct FmRouteLds {
    int U[FM_RT_UMAX];                                     // element index: [0,K) initial, then insertions
    int Uv[FM_RT_UMAX + 4] __attribute__((aligned(16)));  // value bits, padded with 0x7fffffff
    int rank[FM_RT_UMAX];                                  // ascending-value rank of U[u]
    int tor[FM_RT_UMAX];                                   // rank -> position in U
    int ptr[FM_RT_UMAX];                                   // pointer-jumping parents -> slots
    unsigned long long smask[FM_RT_MAXE / 64];             // per-chunk survivors of the filter
    unsigned long long ins[FM_RT_MAXE / 64];               // per-chunk insertions
    int kth[FM_RT_MAXE / 64];
    int cpre[FM_RT_MAXE / 64];
    float red[2][FM_RT_NW];
    int M, tie, nsurv;
    int s_id[64];
    float s_val[64];
    // E <= 64 * FM_RT_SMALL_NCH path
    int big[FM_RT_SMALL_NCH][68] __attribute__((aligned(16)));  // chunk values >= its kth bound, -2 padded
    int nbig[FM_RT_SMALL_NCH];
    int c0cnt[64];                                              // chunk 0: #{j < i : p_j >= p_i}
    int sv[FM_RT_SMALL_NCH][64] __attribute__((aligned(16)));  // chunk survivors' values in lane order
    int S_v[FM_RT_SMALL_NCH * 64];                              // all survivors: value bits
    int S_p[FM_RT_SMALL_NCH * 64];                              // element index * 64 + rank in its chunk's list
};

__global__ __launch_bounds__(FM_RT_THREADS) void fm_route_kernel(const float *__restrict__ logits, int T, int E,
                                                                 int K, int *__restrict__ idx,
                                                                 float *__restrict__ wout) {
    extern __shared__ __attribute__((aligned(16))) int pb[];  // probability bits, padded with -2 to whole chunks
    __shared__ FmRouteLds L;
    const int t = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (t >= T) return;
    FM_RT_DECL
    const float *l = logits + (size_t)t * E;
    const int nch = (E + 63) >> 6;
    FM_RT_MARK(0);

    // softmax: max, exp(x - max), sum, scale by 1/sum (cpu_kernels.h:263-277)
    const uint32_t etab = fm_expf_lanes_load();  // exp table in lanes, loaded with the logits
    float v[FM_RT_VPT];
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < FM_RT_VPT; q++) {
        const int i = tid + q * FM_RT_THREADS;
        v[q] = i < E ? l[i] : -INFINITY;
        mx = fmaxf(mx, v[q]);
    }
    mx = fm_wave_max(mx);
    if (lane == 0) L.red[0][wv] = mx;
    if (tid < FM_RT_MAXE / 64) L.ins[tid] = 0ull;
    if (tid < FM_RT_UMAX) L.rank[tid] = 0;
    if (tid < 64) L.c0cnt[tid] = 0;
    if (tid == 0) {
        L.tie = 0;
        L.nsurv = 0;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < FM_RT_NW; w++) mx = fmaxf(mx, L.red[0][w]);
    // exp with the reference libm's results, then the sum in index order
    // (wavefront 0, the exponentials staged in pb): bit-equal probabilities
#pragma unroll
    for (int q = 0; q < FM_RT_VPT; q++) {
        const int i = tid + q * FM_RT_THREADS;
        const float ex = fm_expf_lanes(v[q] - mx, etab);  // every lane active
        v[q] = i < E ? ex : 0.f;
        if (i < E) pb[i] = __float_as_int(v[q]);
    }
    __syncthreads();
    if (wv == 0) {
        const float s = fm_serial_sum((const float *)pb, E);
        if (lane == 0) L.red[1][0] = s;
    }
    __syncthreads();
    const float inv = 1.0f / L.red[1][0];
#pragma unroll
    for (int q = 0; q < FM_RT_VPT; q++) {
        const int i = tid + q * FM_RT_THREADS;
        if (i < E)
            pb[i] = __float_as_int(v[q] * inv);
        else if (i < nch * 64)
            pb[i] = -2;
    }
    FM_RT_MARK(1);
    bool done = false;
    if (nch <= FM_RT_SMALL_NCH) {
        // one element per thread: wavefront w holds chunk w in a register
        const int pv = tid < E ? __float_as_int(v[0] * inv) : -2;
        fm_route_prep<FM_RT_NW>(&pv, K, nch, L);
        __syncthreads();
        FM_RT_MARK(6);
        done = fm_route_small<FM_RT_NW>(pb, &pv, E, K, nch, L);
    } else {
        __syncthreads();
        // lower bound of the K-th largest of every full chunk but the last
        for (int c = wv; c < nch - 1; c += FM_RT_NW) {
            const int res = fm_kth_lower_bound(pb[c * 64 + lane], K);
            if (lane == 0) L.kth[c] = res;
        }
        __syncthreads();
        FM_RT_MARK(6);
        // survivors of chunk c: i >= K with p_i > L_c = max_{c' < c} kth[c'] (no bound in chunk 0)
        for (int c = wv; c < nch; c += FM_RT_NW) {
            const int lb = c == 0 ? -1 : fm_wave_max_i(lane < c ? L.kth[lane] : -1);
            const uint64_t m = __ballot(c * 64 + lane >= K && pb[c * 64 + lane] > lb);
            if (lane == 0) L.smask[c] = m;
        }
        __syncthreads();
        FM_RT_MARK(7);

        // exact test c_i = #{j < i : p_j >= p_i} < K for every survivor, in
        // batches of eight survivors of one chunk spread over all wavefronts; a
        // batch of chunk c takes c+1 ballots per survivor.
        {
            const uint64_t cm = lane < nch ? L.smask[lane] : 0ull;
            const int nb = (__builtin_popcountll(cm) + 7) >> 3;
            const int incl = fm_wave_incl_scan(nb);
            const int pre = incl - nb;
            const int NB = __builtin_amdgcn_readlane(incl, 63);
            // ballot passes the batches would take; a weak filter (K close to 64,
            // long ascending runs) makes the serial replay the cheaper choice
            const int passes = fm_wave_incl_scan(lane < nch ? nb * (lane + 1) : 0);
            const bool too_much = __builtin_amdgcn_readlane(passes, 63) > FM_RT_MAX_PASSES;
            if (too_much && tid == 0) L.tie = 1;
            for (int g = too_much ? NB : wv; g < NB; g += FM_RT_NW) {
                const int c = __builtin_ctzll(__ballot(lane < nch && g >= pre && g < incl));
                const int r8 = (g - __builtin_amdgcn_readlane(pre, c)) * 8;
                const uint64_t msk = ((uint64_t)(unsigned)__builtin_amdgcn_readlane((int)(cm >> 32), c) << 32) |
                                     (unsigned)__builtin_amdgcn_readlane((int)cm, c);
                const int p = pb[c * 64 + lane];
                const int rk = __builtin_popcountll(msk & lt_mask);
                const bool mine = ((msk >> lane) & 1ull) && rk >= r8 && rk < r8 + 8;
                int jb[8], pv[8], cnt[8];
    #pragma unroll
                for (int b = 0; b < 8; b++) {
                    const uint64_t bm = __ballot(mine && rk == r8 + b);
                    jb[b] = bm ? __builtin_ctzll(bm) : 64;
                    pv[b] = bm ? __builtin_amdgcn_readlane(p, jb[b]) : 0x7fffffff;
                    cnt[b] = 0;
                }
                for (int jc = 0; jc < c; jc++) {
                    const int q = pb[jc * 64 + lane];
    #pragma unroll
                    for (int b = 0; b < 8; b++) cnt[b] += __builtin_popcountll(__ballot(q >= pv[b]));
                }
                uint64_t insm = 0;
    #pragma unroll
                for (int b = 0; b < 8; b++) {
                    cnt[b] += __builtin_popcountll(__ballot(p >= pv[b] && lane < jb[b]));
                    if (jb[b] < 64 && cnt[b] < K) insm |= 1ull << jb[b];
                }
                if (lane == 0 && insm) atomicOr(&L.ins[c], insm);
            }
        }
        __syncthreads();
    }
    FM_RT_MARK(2);
    if (!done) {
        // U = [0..K-1, insertions in index order]
        if (wv == 0) {
            const int cnt = lane < nch ? __builtin_popcountll(L.ins[lane]) : 0;
            const int incl = fm_wave_incl_scan(cnt);
            if (lane < nch) L.cpre[lane] = incl - cnt;
            if (lane == 63) L.M = incl;
        }
        if (tid < K) {
            L.U[tid] = tid;
            L.Uv[tid] = pb[tid];
        }
        __syncthreads();
        const int M = L.M;
        const int NU = K + M;
        const bool par = NU <= FM_RT_UMAX;
        if (par) {
            for (int i = tid; i < nch * 64; i += FM_RT_THREADS) {
                const unsigned long long mk = L.ins[i >> 6];
                if ((mk >> (i & 63)) & 1ull) {
                    const int pos = K + L.cpre[i >> 6] + __builtin_popcountll(mk & ((1ull << (i & 63)) - 1ull));
                    L.U[pos] = i;
                    L.Uv[pos] = pb[i];
                }
            }
            if (tid < 4) L.Uv[NU + tid] = 0x7fffffff;
        }
        __syncthreads();
        bool serial = !par || L.tie != 0;
        if (!serial) {
            // rank sort of U (ascending value), four partial counts per element
            const int u = tid & (FM_RT_UMAX - 1);
            const int qtr = tid / FM_RT_UMAX;
            const int seg = ((NU + 15) >> 4) << 2;
            if (u < NU) {
                const int x = L.Uv[u];
                int r = 0, eq = 0;
                const int w1 = min(NU, (qtr + 1) * seg);
                for (int w = qtr * seg; w < w1; w += 4) {
                    const int4 vw = *reinterpret_cast<const int4 *>(&L.Uv[w]);
                    r += (vw.x < x) + (vw.y < x) + (vw.z < x) + (vw.w < x);
                    eq += (vw.x == x) + (vw.y == x) + (vw.z == x) + (vw.w == x);
                }
                if (u >= qtr * seg && u < w1) eq--;  // itself
                if (r) atomicAdd(&L.rank[u], r);
                if (eq) L.tie = 1;  // equal probabilities inside U: slot choice needs the replay
            }
            __syncthreads();
            serial = L.tie != 0;
            if (!serial) {
                if (tid < NU) L.tor[L.rank[tid]] = tid;
                __syncthreads();
                FM_RT_MARK(3);
                if (wv == 0) {
                    // parents: initial elements are roots; x_m (position K+m-1) -> rank m-1.
                    // Pointer jumping within one wavefront until every chain reaches its root.
                    for (int q = lane; q < NU; q += 64) L.ptr[q] = q < K ? q : L.tor[q - K];
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    for (int round = 0; round < 9; round++) {
                        int nx[FM_RT_UMAX / 64];
                        bool ch = false;
    #pragma unroll
                        for (int q = 0; q < FM_RT_UMAX / 64; q++) {
                            const int uu = lane + 64 * q;
                            const int pu = uu < NU ? L.ptr[uu] : 0;
                            nx[q] = uu < NU ? L.ptr[pu] : 0;
                            ch |= nx[q] != pu;
                        }
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        if (!__ballot(ch)) break;
    #pragma unroll
                        for (int q = 0; q < FM_RT_UMAX / 64; q++) {
                            const int uu = lane + 64 * q;
                            if (uu < NU) L.ptr[uu] = nx[q];
                        }
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    }
                    // survivors = the K largest (ranks M .. NU-1); slot = root of the chain
                    for (int r = M + lane; r < NU; r += 64) {
                        const int uu = L.tor[r];
                        const int slot = L.ptr[uu];
                        L.s_id[slot] = L.U[uu];
                        L.s_val[slot] = __int_as_float(L.Uv[uu]);
                    }
                }
            }
        }
        if (serial && wv == 0) fm_topk_serial(pb, E, K, L);
    }
    __syncthreads();
    FM_RT_MARK(4);
    // cpu_normalize_weights: sequential sum over slots, then scale by 1/sum
    if (tid < K) {
        float s = 0.f;
        for (int k = 0; k < K; k++) s += L.s_val[k];
        const float x = L.s_val[tid];
        idx[(size_t)t * K + tid] = L.s_id[tid];
        wout[(size_t)t * K + tid] = s > 0.f ? x * (1.0f / s) : x;
    }
    FM_RT_MARK(5);
}

extern "C" int fm_route_topk(const float *logits, int T, int E, int K, int *idx, float *weights,
                             void *stream) {
    fm_clear_error();
    FM_REQUIRE(logits && idx && weights, "fm_route_topk: NULL pointer argument");
    FM_REQUIRE(T >= 0, "fm_route_topk: T=%d < 0", T);
    FM_REQUIRE(E >= 1 && E <= FM_RT_MAXE, "fm_route_topk: E=%d outside 1..%d", E, FM_RT_MAXE);
    FM_REQUIRE(K >= 1 && K <= 64 && K <= E, "fm_route_topk: K=%d outside 1..min(64,E)", K);
    if (T == 0) return FM_OK;
    const size_t lds = (size_t)((E + 63) / 64) * 64 * sizeof(int);
    hipLaunchKernelGGL(fm_route_kernel, dim3(T), dim3(FM_RT_THREADS), lds, fm_stream(stream), logits, T, E, K, idx,
                       weights);
    return fm_check_launch("fm_route_kernel");
}
