// fm_route.hip -- softmax / top-K / renormalise on the device.
//
// Semantics of cpu_softmax, cpu_topk and cpu_normalize_weights
// (cpu_kernels.h:263-309) as called at layer_forward.h:3519-3523 and
// batched_prefill.h:256-261.  One wavefront per token.
//
// cpu_topk's output is in SLOT order, which depends on the history of
// replacements: K slots start at -1e30; element i replaces the first slot
// holding the minimum iff p_i > that minimum.  The invariant "slot values =
// top-K multiset of the prefix" means element i can only be inserted if
// p_i > current minimum, so the wave scans 64 elements at a time, ballots the
// ones above the running minimum and replays only those, in index order, with
// the exact replacement rule.  Slots live in wave-uniform registers, so a
// replay step is a handful of scalar-path instructions.  Probabilities are
// >= 0, so their IEEE bit patterns order like signed integers; the -1e30
// initial value is represented by -1.
#include "fm_device.h"
#include "fm_internal.h"

template <int KMAX>
__global__ __launch_bounds__(64) void fm_route_kernel(const float *__restrict__ logits, int T, int E,
                                                      int K, int *__restrict__ idx,
                                                      float *__restrict__ wout) {
    extern __shared__ float probs[];
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    if (t >= T) return;
    const float *l = logits + (size_t)t * E;

    // softmax: max, exp(x - max), sum, scale by 1/sum
    float mx = -INFINITY;
    for (int i = lane; i < E; i += 64) mx = fmaxf(mx, l[i]);
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float sum = 0.f;
    for (int i = lane; i < E; i += 64) {
        float e = expf(l[i] - mx);
        probs[i] = e;
        sum += e;
    }
    sum = fm_lane_sum<64>(sum);
    const float inv = 1.0f / sum;
    for (int i = lane; i < E; i += 64) probs[i] *= inv;
    __syncthreads();

    int vals[KMAX], ids[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        vals[k] = k < K ? -1 : 0x7fffffff;  // unused slots never become the minimum
        ids[k] = 0;
    }
    int thr = -1, mslot = 0;
    for (int base = 0; base < E; base += 64) {
        const int i = base + lane;
        const int pb = i < E ? __float_as_int(probs[i]) : -2;
        uint64_t cand = __ballot(pb > thr);
        while (cand) {
            const int j = __builtin_ctzll(cand);
            cand &= cand - 1;
            const int pj = __builtin_amdgcn_readlane(pb, j);
            if (pj > thr) {
#pragma unroll
                for (int k = 0; k < KMAX; k++) {
                    if (k == mslot) {
                        vals[k] = pj;
                        ids[k] = base + j;
                    }
                }
                // first slot holding the minimum
                thr = vals[0];
                mslot = 0;
#pragma unroll
                for (int k = 1; k < KMAX; k++) {
                    if (vals[k] < thr) {
                        thr = vals[k];
                        mslot = k;
                    }
                }
            }
        }
    }
    // cpu_normalize_weights: sequential sum over slots, then scale by 1/sum
    if (lane == 0) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < KMAX; k++)
            if (k < K) s += __int_as_float(vals[k]);
        float iv = s > 0.f ? 1.0f / s : 1.0f;
#pragma unroll
        for (int k = 0; k < KMAX; k++) {
            if (k < K) {
                idx[(size_t)t * K + k] = ids[k];
                wout[(size_t)t * K + k] = s > 0.f ? __int_as_float(vals[k]) * iv : __int_as_float(vals[k]);
            }
        }
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
    hipStream_t st = fm_stream(stream);
    size_t lds = (size_t)E * sizeof(float);
    if (K <= 8)
        hipLaunchKernelGGL((fm_route_kernel<8>), dim3(T), dim3(64), lds, st, logits, T, E, K, idx, weights);
    else if (K <= 16)
        hipLaunchKernelGGL((fm_route_kernel<16>), dim3(T), dim3(64), lds, st, logits, T, E, K, idx, weights);
    else
        hipLaunchKernelGGL((fm_route_kernel<64>), dim3(T), dim3(64), lds, st, logits, T, E, K, idx, weights);
    return fm_check_launch("fm_route_kernel");
}
