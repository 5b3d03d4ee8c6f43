// fm_decode.hip -- fused decode step: K routed experts + shared expert.
//
// Replaces CMD3 of the reference decode (layer_forward.h:3895-3993):
// gpu_encode_experts_batched (gpu_dispatch.h:461-609: per expert a gate and an
// up matvec, SwiGLU, a down matvec -- four dispatches per expert), the shared
// expert's SwiGLU + down (layer_forward.h:3906-3937) and moe_combine_residual
// (shaders.metal:1865-1900).  Here the whole step is two launches:
//
//  A  fm_decode_gateup_kernel: every (slot, row-block) of every expert's gate
//     and up projection in one grid; SwiGLU in the epilogue; act[slot][inter]
//     (fp32) to the workspace.  Gate and up rows of the same index are done by
//     the same lanes so silu(g)*u needs no extra pass.
//  B  fm_decode_down_kernel: one block per run of output rows; one wavefront
//     per expert slot computes that slot's down-projection rows, the block
//     then combines the slots in the reference order
//       out = h_mid + sum_k w_k e_k + sigmoid(g) * shared
//     (layer_forward.h:1257, 1295-1305) with no atomics, so results are
//     deterministic and there is no K <= 8 limit.
//
// Slots are described either on the host (kernel arguments) or, in pool mode,
// resolved on the device from routing indices (no host round trip).
#include "fm_device.h"
#include "fm_internal.h"

#define FM_MAX_SLOTS (FM_MAX_K + 1)
#define FM_A_NP 2  // rows per wave in phase A
#define FM_B_NP 4  // row passes per wave in phase B

struct FmSlot {
    const uint32_t *gw, *uw, *dw;
    const uint16_t *gs, *gb, *us, *ub, *ds, *db;
    float weight;
    int bits;
    int valid;
    int pad;
};

struct FmDecodeArgs {
    FmSlot slot[FM_MAX_SLOTS];
    int S;          // slots in use (K routed + optional shared)
    int K;          // routed slots
    int has_shared; // slot K is the shared expert
    int pool_mode;  // routed slots resolved from pool + idx on the device
    int mode;       // 0: combine into out; 1: per-slot outputs (expert_out)
    int pad0;
    const void *const *pool_blobs;
    const uint8_t *pool_bits;
    const int *idx;
    const float *wdev;
    uint64_t off4[9], off2[9];
    uint32_t pool_n;
    uint32_t hidden, inter;
    float shared_w_host;       // used when shared_score == NULL and host mode
    const float *shared_score; // device scalar (pre-sigmoid) or NULL
    const float *x;
    float *act;
    const float *h_mid;
    float *out;
    uint16_t *out_bf16;
    float *expert_out;
};

__device__ __forceinline__ FmSlot fm_get_slot(const FmDecodeArgs &a, int k) {
    if (!a.pool_mode || k >= a.K) return a.slot[k];
    FmSlot s;
    int e = a.idx[k];
    if (e < 0 || (uint32_t)e >= a.pool_n) {
        s.valid = 0;
        s.bits = 4;
        s.weight = 0.f;
        return s;
    }
    const char *blob = (const char *)a.pool_blobs[e];
    int bits = a.pool_bits[e];
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
    s.weight = a.wdev[k];
    s.valid = blob != nullptr && (bits == 2 || bits == 4);
    return s;
}

// ---------------------------------------------------------------- phase A --
template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_gateup_body(const FmDecodeArgs &a, const FmSlot &s, int slot,
                                               uint32_t row0) {
    constexpr int RPP = 64 / LPR;
    constexpr int WPG = 2 * BITS;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, gl = lane % LPR;
    const uint32_t G = a.hidden / 64;
    const uint32_t wpr = a.hidden * BITS / 32;

    FmXGroup xg[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        uint32_t g = gl + j * LPR;
        if (g < G) fm_load_xgroup<BITS>(a.x + 64 * g, xg[j]);
    }
    FmWGroup wg[FM_A_NP][GPL], wu[FM_A_NP][GPL];
    float gs[FM_A_NP][GPL], gb[FM_A_NP][GPL], us[FM_A_NP][GPL], ub[FM_A_NP][GPL];
#pragma unroll
    for (int p = 0; p < FM_A_NP; p++) {
        uint32_t row = row0 + p * RPP + sub;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < a.inter && g < G) {
                size_t wo = (size_t)row * wpr + g * WPG, so = (size_t)row * G + g;
                fm_load_wgroup<BITS>(s.gw + wo, wg[p][j]);
                fm_load_wgroup<BITS>(s.uw + wo, wu[p][j]);
                gs[p][j] = fm_bf16_to_f32(s.gs[so]);
                gb[p][j] = fm_bf16_to_f32(s.gb[so]);
                us[p][j] = fm_bf16_to_f32(s.us[so]);
                ub[p][j] = fm_bf16_to_f32(s.ub[so]);
            }
        }
    }
#pragma unroll
    for (int p = 0; p < FM_A_NP; p++) {
        uint32_t row = row0 + p * RPP + sub;
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < a.inter && g < G) {
                pg += fm_group_dot<BITS>(wg[p][j], xg[j], gs[p][j], gb[p][j]);
                pu += fm_group_dot<BITS>(wu[p][j], xg[j], us[p][j], ub[p][j]);
            }
        }
        pg = fm_lane_sum<LPR>(pg);
        pu = fm_lane_sum<LPR>(pu);
        if (gl == 0 && row < a.inter) a.act[(size_t)slot * a.inter + row] = fm_silu_mul(pg, pu);
    }
}

template <int LPR, int GPL>
__global__ __launch_bounds__(256) void fm_decode_gateup_kernel(FmDecodeArgs a, uint32_t blocks_per_slot) {
    constexpr int RPP = 64 / LPR;
    constexpr int RB = 4 * FM_A_NP * RPP;
    const int slot = blockIdx.x / blocks_per_slot;
    const uint32_t rb = blockIdx.x % blocks_per_slot;
    if (slot >= a.S) return;
    const FmSlot s = fm_get_slot(a, slot);
    if (!s.valid) return;
    const uint32_t row0 = rb * RB + (threadIdx.x >> 6) * (FM_A_NP * RPP);
    if (s.bits == 4)
        fm_gateup_body<4, LPR, GPL>(a, s, slot, row0);
    else
        fm_gateup_body<2, LPR, GPL>(a, s, slot, row0);
}

// ---------------------------------------------------------------- phase B --
// Returns this lane's row partial sums for FM_B_NP passes of one slot (valid in
// lanes with gl == 0 after the reduction).
template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_down_body(const FmDecodeArgs &a, const FmSlot &s, int slot,
                                             uint32_t row0, float (&res)[FM_B_NP]) {
    constexpr int RPP = 64 / LPR;
    constexpr int WPG = 2 * BITS;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, gl = lane % LPR;
    const uint32_t G = a.inter / 64;
    const uint32_t wpr = a.inter * BITS / 32;

    FmWGroup wd[FM_B_NP][GPL];
    float ds[FM_B_NP][GPL], db[FM_B_NP][GPL];
#pragma unroll
    for (int p = 0; p < FM_B_NP; p++) {
        uint32_t row = row0 + p * RPP + sub;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < a.hidden && g < G) {
                fm_load_wgroup<BITS>(s.dw + (size_t)row * wpr + g * WPG, wd[p][j]);
                ds[p][j] = fm_bf16_to_f32(s.ds[(size_t)row * G + g]);
                db[p][j] = fm_bf16_to_f32(s.db[(size_t)row * G + g]);
            }
        }
    }
    FmXGroup xg[GPL];
    const float *act = a.act + (size_t)slot * a.inter;
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        uint32_t g = gl + j * LPR;
        if (g < G) fm_load_xgroup<BITS>(act + 64 * g, xg[j]);
    }
#pragma unroll
    for (int p = 0; p < FM_B_NP; p++) {
        uint32_t row = row0 + p * RPP + sub;
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < a.hidden && g < G) part += fm_group_dot<BITS>(wd[p][j], xg[j], ds[p][j], db[p][j]);
        }
        res[p] = fm_lane_sum<LPR>(part);
    }
}

template <int LPR, int GPL>
__global__ __launch_bounds__(1024) void fm_decode_down_kernel(FmDecodeArgs a) {
    constexpr int RPP = 64 / LPR;
    constexpr int RB = FM_B_NP * RPP;  // rows per block (every wave covers all of them)
    __shared__ float part[FM_MAX_SLOTS][RB];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, gl = lane % LPR;
    const uint32_t row0 = blockIdx.x * RB;

    for (int k = wave; k < a.S; k += nw) {
        const FmSlot s = fm_get_slot(a, k);
        float res[FM_B_NP];
        if (s.valid) {
            if (s.bits == 4)
                fm_down_body<4, LPR, GPL>(a, s, k, row0, res);
            else
                fm_down_body<2, LPR, GPL>(a, s, k, row0, res);
        } else {
#pragma unroll
            for (int p = 0; p < FM_B_NP; p++) res[p] = 0.f;
        }
        if (gl == 0) {
#pragma unroll
            for (int p = 0; p < FM_B_NP; p++) {
                uint32_t r = p * RPP + sub;
                if (a.mode == 1) {
                    uint32_t row = row0 + r;
                    if (s.valid && row < a.hidden) a.expert_out[(size_t)k * a.hidden + row] = res[p];
                } else {
                    part[k][r] = res[p];
                }
            }
        }
    }
    if (a.mode == 1) return;
    __syncthreads();
    if ((int)threadIdx.x < RB) {
        const uint32_t r = threadIdx.x, row = row0 + r;
        if (row < a.hidden) {
            // cpu_vec_madd order: moe += w_k * e_k over k (layer_forward.h:1257)
            float moe = 0.f;
            for (int k = 0; k < a.K; k++) {
                const FmSlot s = fm_get_slot(a, k);
                if (s.valid) moe = __fadd_rn(moe, __fmul_rn(s.weight, part[k][r]));
            }
            float v = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
            if (a.has_shared) {
                float sw = a.shared_score ? fm_sigmoid(*a.shared_score) : a.shared_w_host;
                v = __fadd_rn(v, __fmul_rn(sw, part[a.K][r]));
            }
            a.out[row] = v;
            if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(v);
        }
    }
}

// ---------------------------------------------------------------- combine --
__global__ __launch_bounds__(256) void fm_combine_kernel(const float *h_mid, const float *eo,
                                                         const float *w, const int *valid, int K,
                                                         const float *so, const float *score,
                                                         float *out, uint16_t *out_bf16,
                                                         uint32_t dim) {
    uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    float moe = 0.f;
    for (int k = 0; k < K; k++)
        if (!valid || valid[k]) moe = __fadd_rn(moe, __fmul_rn(w[k], eo[(size_t)k * dim + i]));
    float v = h_mid ? __fadd_rn(h_mid[i], moe) : moe;
    if (so) v = __fadd_rn(v, __fmul_rn(score ? fm_sigmoid(*score) : 1.0f, so[i]));
    out[i] = v;
    if (out_bf16) out_bf16[i] = fm_f32_to_bf16(v);
}

// ---------------------------------------------------------------- host -----
static void fm_fill_slot(FmSlot &d, const fm_expert_weights &e, int bits, float w, int valid) {
    d.gw = (const uint32_t *)e.gate_w;
    d.gs = (const uint16_t *)e.gate_s;
    d.gb = (const uint16_t *)e.gate_b;
    d.uw = (const uint32_t *)e.up_w;
    d.us = (const uint16_t *)e.up_s;
    d.ub = (const uint16_t *)e.up_b;
    d.dw = (const uint32_t *)e.down_w;
    d.ds = (const uint16_t *)e.down_s;
    d.db = (const uint16_t *)e.down_b;
    d.bits = bits;
    d.weight = w;
    d.valid = valid;
}

static int fm_check_expert(const char *who, int k, const fm_expert_weights &e, int bits) {
    if (bits != 2 && bits != 4) return fm_fail(FM_ERR_INVALID, "%s: slot %d bits must be 2 or 4 (got %d)", who, k, bits);
    const void *p[9] = {e.gate_w, e.gate_s, e.gate_b, e.up_w, e.up_s, e.up_b, e.down_w, e.down_s, e.down_b};
    for (int i = 0; i < 9; i++) {
        if (!p[i]) return fm_fail(FM_ERR_INVALID, "%s: slot %d tensor %d is NULL", who, k, i);
    }
    if (((uintptr_t)e.gate_w | (uintptr_t)e.up_w | (uintptr_t)e.down_w) & 15)
        return fm_fail(FM_ERR_INVALID, "%s: slot %d packed weights not 16-byte aligned", who, k);
    return FM_OK;
}

extern "C" size_t fm_moe_decode_workspace_size(int n_slots, uint32_t hidden, uint32_t inter) {
    (void)hidden;
    if (n_slots < 1) n_slots = 1;
    return fm_align_up((size_t)n_slots * inter * sizeof(float), 256);
}

static int fm_decode_launch(FmDecodeArgs &a, void *ws, size_t ws_bytes, hipStream_t st) {
    const char *who = "fm_moe_decode";
    FM_REQUIRE(a.hidden % 64 == 0 && a.inter % 64 == 0 && a.hidden && a.inter,
               "%s: hidden %u / inter %u must be positive multiples of 64", who, a.hidden, a.inter);
    int lh, gh, li, gi;
    if (!fm_pick_lanes(a.hidden / 64, &lh, &gh) || !fm_pick_lanes(a.inter / 64, &li, &gi))
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: hidden %u / inter %u exceed 16384", who, a.hidden, a.inter);
    size_t need = fm_moe_decode_workspace_size(a.S, a.hidden, a.inter);
    if (!ws || ws_bytes < need)
        return fm_fail(FM_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu required", who, ws_bytes, need);
    if ((uintptr_t)a.x & 15) return fm_fail(FM_ERR_INVALID, "%s: x not 16-byte aligned", who);
    a.act = (float *)ws;

    const uint32_t rba = 4u * FM_A_NP * (64u / lh);
    const uint32_t bps = (a.inter + rba - 1) / rba;
    dim3 ga((unsigned)(bps * a.S)), ba(256);
#define FM_A_CASE(L, G)                                                                   \
    if (lh == L && gh == G) {                                                             \
        hipLaunchKernelGGL((fm_decode_gateup_kernel<L, G>), ga, ba, 0, st, a, bps);      \
    } else
    FM_A_CASE(16, 1) FM_A_CASE(32, 1) FM_A_CASE(64, 1) FM_A_CASE(64, 2) FM_A_CASE(64, 4) {
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: no gate/up kernel", who);
    }
#undef FM_A_CASE
    int rc = fm_check_launch("fm_decode_gateup_kernel");
    if (rc) return rc;

    const uint32_t rbb = FM_B_NP * (64u / li);
    dim3 gb((a.hidden + rbb - 1) / rbb), bb(64 * (a.S < 16 ? a.S : 16));
#define FM_B_CASE(L, G)                                                        \
    if (li == L && gi == G) {                                                  \
        hipLaunchKernelGGL((fm_decode_down_kernel<L, G>), gb, bb, 0, st, a);  \
    } else
    FM_B_CASE(16, 1) FM_B_CASE(32, 1) FM_B_CASE(64, 1) FM_B_CASE(64, 2) FM_B_CASE(64, 4) {
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: no down kernel", who);
    }
#undef FM_B_CASE
    return fm_check_launch("fm_decode_down_kernel");
}

extern "C" int fm_moe_decode(int K, const fm_expert_weights *experts, const int *bits,
                             const float *weights, const int *valid,
                             const fm_expert_weights *shared, int shared_bits,
                             float shared_gate_score, uint32_t hidden, uint32_t inter,
                             uint32_t group_size, const float *x, const float *h_mid, float *out,
                             uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream) {
    const char *who = "fm_moe_decode";
    fm_clear_error();
    FM_REQUIRE(K >= 0 && K <= FM_MAX_K, "%s: K=%d outside 0..%d", who, K, FM_MAX_K);
    FM_REQUIRE(K == 0 || (experts && bits && weights), "%s: NULL experts/bits/weights", who);
    FM_REQUIRE(K > 0 || shared, "%s: no experts", who);
    FM_REQUIRE(x && out, "%s: NULL x or out", who);
    if (group_size != 64) return fm_fail(FM_ERR_UNSUPPORTED, "%s: group_size must be 64", who);
    FmDecodeArgs a = {};
    for (int k = 0; k < K; k++) {
        int v = valid ? (valid[k] != 0) : 1;
        if (v) {
            int rc = fm_check_expert(who, k, experts[k], bits[k]);
            if (rc) return rc;
        }
        fm_fill_slot(a.slot[k], experts[k], v ? bits[k] : 4, weights[k], v);
    }
    a.K = K;
    a.S = K;
    if (shared) {
        int rc = fm_check_expert(who, K, *shared, shared_bits);
        if (rc) return rc;
        fm_fill_slot(a.slot[K], *shared, shared_bits, 1.0f, 1);
        a.has_shared = 1;
        a.S = K + 1;
        a.shared_w_host = 1.0f / (1.0f + expf(-shared_gate_score));
    }
    a.hidden = hidden;
    a.inter = inter;
    a.x = x;
    a.h_mid = h_mid;
    a.out = out;
    a.out_bf16 = out_bf16;
    return fm_decode_launch(a, ws, ws_bytes, fm_stream(stream));
}

extern "C" int fm_moe_decode_pool(const fm_expert_pool *pool, int K, const int *idx,
                                  const float *weights, const fm_expert_weights *shared,
                                  int shared_bits, const float *shared_gate_score,
                                  const float *x, const float *h_mid, float *out,
                                  uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream) {
    const char *who = "fm_moe_decode_pool";
    fm_clear_error();
    FM_REQUIRE(pool && pool->blobs && pool->bits && pool->num_experts, "%s: invalid pool", who);
    FM_REQUIRE(K >= 0 && K <= FM_MAX_K, "%s: K=%d outside 0..%d", who, K, FM_MAX_K);
    FM_REQUIRE(K == 0 || (idx && weights), "%s: NULL idx/weights", who);
    FM_REQUIRE(K > 0 || shared, "%s: no experts", who);
    FM_REQUIRE(x && out, "%s: NULL x or out", who);
    if (pool->group_size != 64) return fm_fail(FM_ERR_UNSUPPORTED, "%s: group_size must be 64", who);
    FmDecodeArgs a = {};
    fm_expert_layout l4, l2;
    fm_expert_layout_compute(pool->hidden, pool->inter, 64, 4, &l4);
    fm_expert_layout_compute(pool->hidden, pool->inter, 64, 2, &l2);
    for (int i = 0; i < 9; i++) {
        a.off4[i] = l4.off[i];
        a.off2[i] = l2.off[i];
    }
    a.pool_mode = 1;
    a.pool_blobs = pool->blobs;
    a.pool_bits = pool->bits;
    a.pool_n = pool->num_experts;
    a.idx = idx;
    a.wdev = weights;
    a.K = K;
    a.S = K;
    if (shared) {
        int rc = fm_check_expert(who, K, *shared, shared_bits);
        if (rc) return rc;
        fm_fill_slot(a.slot[K], *shared, shared_bits, 1.0f, 1);
        a.has_shared = 1;
        a.S = K + 1;
        a.shared_score = shared_gate_score;
        a.shared_w_host = 1.0f;
    }
    a.hidden = pool->hidden;
    a.inter = pool->inter;
    a.x = x;
    a.h_mid = h_mid;
    a.out = out;
    a.out_bf16 = out_bf16;
    return fm_decode_launch(a, ws, ws_bytes, fm_stream(stream));
}

extern "C" int fm_encode_experts_batched(int K, const int *valid, const fm_expert_weights *experts,
                                         const int *bits, uint32_t hidden, uint32_t inter,
                                         uint32_t group_size, const float *x, float *expert_out,
                                         void *ws, size_t ws_bytes, void *stream) {
    const char *who = "fm_encode_experts_batched";
    fm_clear_error();
    FM_REQUIRE(K >= 1 && K <= FM_MAX_K, "%s: K=%d outside 1..%d", who, K, FM_MAX_K);
    FM_REQUIRE(experts && bits && x && expert_out, "%s: NULL argument", who);
    if (group_size != 64) return fm_fail(FM_ERR_UNSUPPORTED, "%s: group_size must be 64", who);
    FmDecodeArgs a = {};
    for (int k = 0; k < K; k++) {
        int v = valid ? (valid[k] != 0) : 1;
        if (v) {
            int rc = fm_check_expert(who, k, experts[k], bits[k]);
            if (rc) return rc;
        }
        fm_fill_slot(a.slot[k], experts[k], v ? bits[k] : 4, 1.0f, v);
    }
    a.K = K;
    a.S = K;
    a.mode = 1;
    a.hidden = hidden;
    a.inter = inter;
    a.x = x;
    a.expert_out = expert_out;
    return fm_decode_launch(a, ws, ws_bytes, fm_stream(stream));
}

extern "C" int fm_moe_combine(const float *h_mid, const float *expert_outs, const float *weights,
                              const int *valid, int K, const float *shared_out,
                              const float *shared_gate_score, float *out, uint16_t *out_bf16,
                              uint32_t dim, void *stream) {
    fm_clear_error();
    FM_REQUIRE(K >= 0, "fm_moe_combine: K=%d < 0", K);
    FM_REQUIRE(K == 0 || (expert_outs && weights), "fm_moe_combine: NULL expert_outs/weights");
    FM_REQUIRE(out && dim, "fm_moe_combine: NULL out or dim 0");
    hipLaunchKernelGGL(fm_combine_kernel, dim3((dim + 255) / 256), dim3(256), 0, fm_stream(stream), h_mid,
                       expert_outs, weights, valid, K, shared_out, shared_gate_score, out, out_bf16, dim);
    return fm_check_launch("fm_combine_kernel");
}
