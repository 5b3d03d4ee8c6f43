// fm_route.hip -- softmax / top-K / renormalise on the device.
//
// Semantics of cpu_softmax, cpu_topk and cpu_normalize_weights
// (cpu_kernels.h:263-309) as called at layer_forward.h:3519-3523 and
// batched_prefill.h:256-261.  One wavefront per token.
//
// cpu_topk returns its K slots in SLOT order, which depends on the history of
// replacements: slots start at -1e30; element i evicts the first slot holding
// the minimum iff p_i > that minimum.  Two facts make a fast exact replay
// possible:
//  * the slot values always form the top-K multiset of the prefix, so only
//    elements above the running minimum can ever be inserted -- the wave
//    ballots 64 elements at a time against it and replays just those;
//  * the evicted slot is the minimum of the keys (value, slot index).  The
//    wave keeps the K keys SORTED across lanes 0..K-1, so the victim is lane
//    0 and an insertion is one compare/ballot (rank of the new key), one
//    lane shift and two selects, all lane-parallel.
// A single wavefront issues roughly one instruction per four cycles, so the
// serial path is what matters: ~15 instructions per insertion, and about
// K*(1 + ln(E/K)) insertions for random scores.
// Probabilities are >= 0, so their IEEE bit patterns order like signed ints;
// the -1e30 initial value is represented by -1.
#include "fm_device.h"
#include "fm_internal.h"

__global__ __launch_bounds__(64) void fm_route_kernel(const float *__restrict__ logits, int T, int E,
                                                       int K, int *__restrict__ idx,
                                                       float *__restrict__ wout) {
    extern __shared__ float probs[];
    __shared__ int s_id[64];
    __shared__ float s_val[64];
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    if (t >= T) return;
    const float *l = logits + (size_t)t * E;

    float mx = -INFINITY;
    for (int i = lane; i < E; i += 64) mx = fmaxf(mx, l[i]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float sum = 0.f;
    for (int i = lane; i < E; i += 64) {
        float e = expf(l[i] - mx);
        probs[i] = e;
        sum += e;
    }
    sum = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fm_lane_sum<64>(sum))));
    const float inv = 1.0f / sum;

    int kval = lane < K ? -1 : 0x7fffffff;
    int kslot = lane < K ? lane : 64;
    int kid = 0;
    int thr = -1;
    for (int base = 0; base < E; base += 64) {
        const int i = base + lane;
        const int pb = i < E ? __float_as_int(probs[i] * inv) : -2;
        uint64_t cand = __ballot(pb > thr);
        while (cand) {
            const int j = __builtin_ctzll(cand);
            cand &= cand - 1;
            const int pj = __builtin_amdgcn_readlane(pb, j);
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
        s_val[kslot] = __int_as_float(kval);
        s_id[kslot] = kid;
    }
    __syncthreads();
    // cpu_normalize_weights: sequential sum over slots, then scale by 1/sum
    float s = 0.f;
    for (int k = 0; k < K; k++) s += s_val[k];
    const float iv = s > 0.f ? 1.0f / s : 1.0f;
    for (int k = lane; k < K; k += 64) {
        idx[(size_t)t * K + k] = s_id[k];
        wout[(size_t)t * K + k] = s > 0.f ? s_val[k] * iv : s_val[k];
    }
}

extern "C" int fm_route_topk(const float *logits, int T, int E, int K, int *idx, float *weights,
                             void *stream) {
    fm_clear_error();
    FM_REQUIRE(logits && idx && weights, "fm_route_topk: NULL pointer argument");
    FM_REQUIRE(T >= 0, "fm_route_topk: T=%d < 0", T);
    FM_REQUIRE(E >= 1 && E <= 4096, "fm_route_topk: E=%d outside 1..4096", E);
    FM_REQUIRE(K >= 1 && K <= 64 && K <= E, "fm_route_topk: K=%d outside 1..min(64,E)", K);
    if (T == 0) return FM_OK;
    hipLaunchKernelGGL(fm_route_kernel, dim3(T), dim3(64), (size_t)E * sizeof(float), fm_stream(stream),
                       logits, T, E, K, idx, weights);
    return fm_check_launch("fm_route_kernel");
}
