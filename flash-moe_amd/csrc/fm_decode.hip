// fm_decode.hip -- fused decode step: K routed experts + shared expert.
//
// Replaces CMD3 of the reference decode (layer_forward.h:3895-3993):
// gpu_encode_experts_batched (gpu_dispatch.h:461-609: per expert a gate and an
// up matvec, SwiGLU, a down matvec -- four dispatches per expert), the shared
// expert's SwiGLU + down (layer_forward.h:3906-3937) and moe_combine_residual
// (shaders.metal:1865-1900).  Here the whole step is ONE kernel launch:
//
//  A  gate/up row passes of every slot (routed experts + shared), SwiGLU in
//     the epilogue -> activations;
//  B  down-projection row passes of every slot -> per-slot outputs y_k;
//  C  combine, in the slot order of cpu_vec_madd (layer_forward.h:1257,
//     1295-1305):  out = h_mid + sum_k w_k y_k + sigmoid(g) * y_shared.
//
// A persistent grid (sized to what stays resident) gives every wave an equal
// share of the slot-major A and B passes.  Values handed from one wave to
// another (activations, y_k) travel as 64-bit (value, epoch) words written
// and read with agent-coherent accesses; consumers poll exactly the words
// they need.  No atomics, no cache flushes, no K <= 8 limit, deterministic.
//
// Slots are described either on the host (kernel arguments) or, in pool mode,
// resolved on the device from routing indices (no host round trip).
#include "fm_decode.h"

#include <mutex>
#include <stdlib.h>
#include <string.h>

#define FM_DECODE_BLOCKS_PER_CU 4  // persistent 256-thread blocks per CU (cap)


// ---------------------------------------------------------------- phase A --
// Persistent stream over the (slot, row-pass) units of every expert's gate and
// up projections.  Each block stages x (fp32) and the slot descriptors in LDS
// once; each wavefront owns a contiguous run of units, keeps its slice of x in
// VGPRs as fp16 pairs, and issues the loads of unit u+1 before computing unit
// u, so every wave always has a row-pair of packed weights in flight.
template <int BITS, int LPR, int GPL>
struct FmGateUpBuf {
    FmWGroup g[GPL], u[GPL];
    float gs[GPL], gb[GPL], us[GPL], ub[GPL];
};

template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_gateup_load(const FmSlot &s, uint32_t row, uint32_t hidden, uint32_t inter,
                                               FmGateUpBuf<BITS, LPR, GPL> &b) {
    constexpr int WPG = 2 * BITS;
    const int gl = (threadIdx.x & 63) % LPR;
    const uint32_t G = hidden / 64;
    const uint32_t wpr = hidden * BITS / 32;
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        uint32_t g = gl + j * LPR;
        if (row < inter && g < G) {
            size_t wo = (size_t)row * wpr + g * WPG, so = (size_t)row * G + g;
            fm_load_wgroup<BITS>(s.gw + wo, b.g[j]);
            fm_load_wgroup<BITS>(s.uw + wo, b.u[j]);
            b.gs[j] = fm_bf16_to_f32(fm_ldg_u16(s.gs + so));
            b.gb[j] = fm_bf16_to_f32(fm_ldg_u16(s.gb + so));
            b.us[j] = fm_bf16_to_f32(fm_ldg_u16(s.us + so));
            b.ub[j] = fm_bf16_to_f32(fm_ldg_u16(s.ub + so));
        }
    }
}

template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_gateup_segment(const FmDecodeArgs &a, uint32_t ep, const FmSlot &s, int slot,
                                                  const float *xs, uint32_t ubeg, uint32_t uend) {
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, gl = lane % LPR;
    const uint32_t G = a.hidden / 64;
    FmXGroup xg[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        uint32_t g = gl + j * LPR;
        if (g < G) fm_load_xgroup<BITS>(xs + 64 * g, xg[j]);
    }
    FmGateUpBuf<BITS, LPR, GPL> cur, nxt;
    fm_gateup_load<BITS, LPR, GPL>(s, ubeg * RPP + sub, a.hidden, a.inter, cur);
    for (uint32_t u = ubeg; u < uend; u++) {
        const uint32_t row = u * RPP + sub;
        if (u + 1 < uend) fm_gateup_load<BITS, LPR, GPL>(s, row + RPP, a.hidden, a.inter, nxt);
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < a.inter && g < G) {
                pg += fm_group_dot<BITS>(cur.g[j], xg[j], cur.gs[j], cur.gb[j]);
                pu += fm_group_dot<BITS>(cur.u[j], xg[j], cur.us[j], cur.ub[j]);
            }
        }
        pg = fm_lane_sum<LPR>(pg);
        pu = fm_lane_sum<LPR>(pu);
        if (gl == 0 && row < a.inter) fm_put_tagged(&a.act2[(size_t)slot * a.inter + row], fm_silu_mul(pg, pu), ep);
        cur = nxt;
    }
}

// ---------------------------------------------------------------- phase B --
// Down projection, streamed like phase A: (slot, 4-row pass) units, slot-major.
// The lane's group of the slot's SwiGLU activation is read once per segment
// (fp32 from the workspace, converted to the slot's fp16 pair layout).
template <int BITS, int LPR, int GPL>
struct FmDownBuf {
    FmWGroup w[GPL];
    float s[GPL], b[GPL];
};

template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_down_load(const FmSlot &s, uint32_t row, uint32_t hidden, uint32_t inter,
                                             FmDownBuf<BITS, LPR, GPL> &b) {
    constexpr int WPG = 2 * BITS;
    const int gl = (threadIdx.x & 63) % LPR;
    const uint32_t G = inter / 64;
    const uint32_t wpr = inter * BITS / 32;
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        uint32_t g = gl + j * LPR;
        if (row < hidden && g < G) {
            size_t so = (size_t)row * G + g;
            fm_load_wgroup<BITS>(s.dw + (size_t)row * wpr + g * WPG, b.w[j]);
            b.s[j] = fm_bf16_to_f32(fm_ldg_u16(s.ds + so));
            b.b[j] = fm_bf16_to_f32(fm_ldg_u16(s.db + so));
        }
    }
}

// y[row] for rows of passes [pbeg, pend) of one slot; writes `dst` (fp32,
// indexed by row) from the first lane of each row segment.
template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_down_segment(const FmDecodeArgs &a, uint32_t ep, const FmSlot &s, int slot,
                                                uint32_t pbeg, uint32_t pend, float *dst, float *wbuf) {
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, gl = lane % LPR;
    const uint32_t G = a.inter / 64;
    FmDownBuf<BITS, LPR, GPL> cur, nxt;
    fm_down_load<BITS, LPR, GPL>(s, pbeg * RPP + sub, a.hidden, a.inter, cur);
    // The slot's activation: poll its tagged words (coalesced, agent-coherent)
    // until all carry this call's epoch, then stage the values in this wave's
    // LDS buffer so each lane can pick up its own groups.
    const uint64_t *act = a.act2 + (size_t)slot * a.inter;
    for (uint32_t i0 = 0; i0 < a.inter; i0 += 64) {
        const uint32_t i = i0 + lane;
        uint64_t v = i < a.inter ? fm_get_tagged(act + i) : ((uint64_t)ep << 32);
        uint32_t it = 0;
        while (!__all((uint32_t)(v >> 32) == ep) && ++it < FM_SPIN_MAX) {
            __builtin_amdgcn_s_sleep(1);
            if ((uint32_t)(v >> 32) != ep) v = fm_get_tagged(act + i);
        }
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        if (i < a.inter) wbuf[i] = __uint_as_float((uint32_t)v);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    FmXGroup xg[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        uint32_t g = gl + j * LPR;
        if (g < G) fm_load_xgroup<BITS>(wbuf + 64 * g, xg[j]);
    }
    __builtin_amdgcn_wave_barrier();
    for (uint32_t p = pbeg; p < pend; p++) {
        const uint32_t row = p * RPP + sub;
        if (p + 1 < pend) fm_down_load<BITS, LPR, GPL>(s, row + RPP, a.hidden, a.inter, nxt);
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < a.hidden && g < G) part += fm_group_dot<BITS>(cur.w[j], xg[j], cur.s[j], cur.b[j]);
        }
        part = fm_lane_sum<LPR>(part);
        if (gl == 0 && row < a.hidden) {
            if (a.mode == 1)
                dst[row] = part;
            else
                fm_put_tagged(&a.y2[(size_t)slot * a.hidden + row], part, ep);
        }
        cur = nxt;
    }
}

// ----------------------------------------------------------- fused kernel --
// One launch for the whole expert step.  The grid is sized to what the GPU
// keeps resident at once, so every wave a consumer waits on is running; each
// wait is bounded anyway (FM_SPIN_MAX polls) and a give-up raises *err.
//
// Wave w owns the same fraction of the slot-major A units (gate/up row passes)
// and B units (down row passes), so its B work belongs to the slot whose
// activations it just helped produce.  The wave that computes the LAST slot's
// down rows for a pass also combines those rows:
//   out = h_mid + sum_{k<K} w_k y_k + sigmoid(g) y_shared
// in the slot order of cpu_vec_madd (layer_forward.h:1257, 1295-1305), polling
// the other slots' tagged y words for the pass's rows first.
template <int RPP>
__device__ __forceinline__ void fm_combine_pass(const FmDecodeArgs &a, uint32_t ep, const FmSlot *sd, uint32_t row0, float sw,
                                                float *stage) {
    const int lane = threadIdx.x & 63;
    const int n = (a.S - 1) * RPP;  // values to collect from other slots
    for (int base = 0; base < n; base += 64) {
        const int q = base + lane;
        const int k = q / RPP, r = q % RPP;
        const bool need = q < n && sd[k].valid && row0 + r < a.hidden;
        uint64_t v = need ? fm_get_tagged(&a.y2[(size_t)k * a.hidden + row0 + r]) : ((uint64_t)ep << 32);
        uint32_t it = 0;
        while (!__all((uint32_t)(v >> 32) == ep) && ++it < FM_SPIN_MAX) {
            __builtin_amdgcn_s_sleep(1);
            if ((uint32_t)(v >> 32) != ep) v = fm_get_tagged(&a.y2[(size_t)k * a.hidden + row0 + r]);
        }
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
        if (q < n) stage[q] = need ? __uint_as_float((uint32_t)v) : 0.f;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    if (lane < RPP && row0 + lane < a.hidden) {
        const uint32_t row = row0 + lane;
        const float ylast = stage[(a.S - 1) * RPP + lane];
        float moe = 0.f;
        for (int k = 0; k < a.K; k++) {
            const float yk = k == a.S - 1 ? ylast : stage[k * RPP + lane];
            if (sd[k].valid) moe = __fadd_rn(moe, __fmul_rn(sd[k].weight, yk));
        }
        float v = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
        if (a.has_shared) v = __fadd_rn(v, __fmul_rn(sw, ylast));
        else if (a.shared_y) v = __fadd_rn(v, __fmul_rn(sw, a.shared_y[row]));
        a.out[row] = v;
        if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(v);
    }
    __builtin_amdgcn_wave_barrier();
}

template <int LH, int GH, int LI, int GI>
__global__ __launch_bounds__(256) void fm_decode_fused_kernel(FmDecodeArgs a, uint32_t nwaves) {
    constexpr int RPPA = 64 / LH, RPPB = 64 / LI;
    // LDS: x (hidden floats), then one inter-float buffer per wave
    extern __shared__ float xs[];
    __shared__ FmSlot sd[FM_MAX_SLOTS];
    const uint32_t ep_ld = fm_epoch_load(a);
    if ((int)threadIdx.x < a.S) sd[threadIdx.x] = fm_get_slot(a, threadIdx.x);
    for (uint32_t i = threadIdx.x * 4; i < a.hidden; i += 1024) *(fm_f4 *)(xs + i) = *(const fm_f4 *)(a.x + i);
    __syncthreads();
    const uint32_t ep = fm_epoch_tag(ep_ld);
    const int lane = threadIdx.x & 63;
    const uint32_t w = blockIdx.x * 4 + (threadIdx.x >> 6);
    float *wbuf = xs + a.hidden + (threadIdx.x >> 6) * a.inter;

    // ---- A: gate/up + SwiGLU -> tagged act ----
    const uint32_t upsA = (a.inter + RPPA - 1) / RPPA;
    const uint64_t NA = (uint64_t)a.S * upsA;
    uint32_t u = (uint32_t)(NA * w / nwaves);
    const uint32_t u1 = (uint32_t)(NA * (w + 1) / nwaves);
    while (u < u1) {
        const int k = u / upsA;
        const uint32_t seg_end = min(u1, (uint32_t)(k + 1) * upsA);
        const FmSlot s = sd[k];
        if (s.valid) {
            const uint32_t b = u - k * upsA, e = seg_end - k * upsA;
            if (s.bits == 4)
                fm_gateup_segment<4, LH, GH>(a, ep, s, k, xs, b, e);
            else
                fm_gateup_segment<2, LH, GH>(a, ep, s, k, xs, b, e);
        }
        u = seg_end;
    }

    // ---- B: down projection -> tagged y; the last slot's waves combine ----
    const float sw =
        (a.has_shared || a.shared_y) ? (a.shared_score ? fm_sigmoid(*a.shared_score) : a.shared_w_host) : 0.f;
    const uint32_t upsB = (a.hidden + RPPB - 1) / RPPB;
    const uint64_t NB = (uint64_t)a.S * upsB;
    uint32_t v = (uint32_t)(NB * w / nwaves);
    const uint32_t v1 = (uint32_t)(NB * (w + 1) / nwaves);
    while (v < v1) {
        const int k = v / upsB;
        const uint32_t seg_end = min(v1, (uint32_t)(k + 1) * upsB);
        const uint32_t pb = v - k * upsB, pe = seg_end - k * upsB;
        const FmSlot s = sd[k];
        if (s.valid) {
            float *dst = a.mode == 1 ? a.expert_out + (size_t)k * a.hidden : nullptr;
            if (s.bits == 4)
                fm_down_segment<4, LI, GI>(a, ep, s, k, pb, pe, dst, wbuf);
            else
                fm_down_segment<2, LI, GI>(a, ep, s, k, pb, pe, dst, wbuf);
        }
        if (a.mode == 0 && k == a.S - 1) {
            for (uint32_t p = pb; p < pe; p++) {
                // the last slot's own y for this pass (if valid) is read back tagged too
                if (s.valid) {
                    const uint32_t row = p * RPPB + (lane < RPPB ? lane : 0);
                    uint64_t t = lane < RPPB && row < a.hidden ? fm_get_tagged(&a.y2[(size_t)k * a.hidden + row])
                                                               : ((uint64_t)ep << 32);
                    uint32_t it = 0;
                    while (!__all((uint32_t)(t >> 32) == ep) && ++it < FM_SPIN_MAX) {
                        __builtin_amdgcn_s_sleep(1);
                        if ((uint32_t)(t >> 32) != ep) t = fm_get_tagged(&a.y2[(size_t)k * a.hidden + row]);
                    }
                    if (lane < RPPB) wbuf[(a.S - 1) * RPPB + lane] = __uint_as_float((uint32_t)t);
                } else if (lane < RPPB) {
                    wbuf[(a.S - 1) * RPPB + lane] = 0.f;
                }
                fm_combine_pass<RPPB>(a, ep, sd, p * RPPB, sw, wbuf);
            }
        }
        v = seg_end;
    }
    __syncthreads();
    if (threadIdx.x == 0) fm_epoch_finish(a, ep, gridDim.x);
}

// ------------------------------------------------- fused kernel, eager loads --
// Fast path for rows of one group per lane (hidden, inter <= 4096).  Each wave
// owns <= UMAX gate/up units and <= UMAX down units and issues ALL of their
// weight loads before any compute -- weights never depend on activations, so
// the whole 78 MB stream is in flight from the first microsecond and the
// memory system, not a chain of per-wave round trips, sets the pace.  Compute
// then follows the data in issue order.  Between the phases the block stages
// the activations of its (at most two) down-projection slots once in LDS.
#define FM_UMAX 6
#ifndef FM_DX_MARK
#define FM_DX_MARK(n)
#endif

struct FmUnitW {
    FmWGroup w;
    float s, b;
};

__device__ __forceinline__ void fm_unit_load(const uint32_t *W, const uint16_t *S, const uint16_t *B, int bits,
                                             uint32_t row, uint32_t in_dim, uint32_t g, bool ok, FmUnitW &u) {
    if (!ok) return;
    const uint32_t G = in_dim / 64;
    const uint32_t wpr = in_dim * bits / 32;
    const uint32_t *wp = W + (size_t)row * wpr + g * 2 * bits;
    u.w.a = fm_ldg_u4_nt(wp);
    if (bits == 4) u.w.b = fm_ldg_u4_nt(wp + 4);
    u.s = fm_bf16_to_f32(fm_ldg_u16(S + (size_t)row * G + g));
    u.b = fm_bf16_to_f32(fm_ldg_u16(B + (size_t)row * G + g));
}

__device__ __forceinline__ float fm_unit_dot(const FmUnitW &u, const FmXGroup &x, int bits) {
    return bits == 4 ? fm_group_dot<4>(u.w, x, u.s, u.b) : fm_group_dot<2>(u.w, x, u.s, u.b);
}

__device__ __forceinline__ void fm_xgroup_bits(const float *src, int bits, FmXGroup &x) {
    if (bits == 4)
        fm_load_xgroup<4>(src, x);
    else
        fm_load_xgroup<2>(src, x);
}

// gate and up group dots with four independent accumulator chains
template <int BITS>
__device__ __forceinline__ void fm_dot_gu(const FmUnitW &g, const FmUnitW &u, const FmXGroup &x, float &pg,
                                          float &pu) {
    float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
    if constexpr (BITS == 4) {
        const uint32_t gw[8] = {g.w.a.x, g.w.a.y, g.w.a.z, g.w.a.w, g.w.b.x, g.w.b.y, g.w.b.z, g.w.b.w};
        const uint32_t uw[8] = {u.w.a.x, u.w.a.y, u.w.a.z, u.w.a.w, u.w.b.x, u.w.b.y, u.w.b.z, u.w.b.w};
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const uint32_t a = gw[p], b = uw[p], ta = a >> 8, tb = b >> 8;
            const fm_h2 *q = &x.q[4 * p];
            g0 = fm_dot2(fm_as_h2(a & 0x000F000Fu), q[0], g0);
            u0 = fm_dot2(fm_as_h2(b & 0x000F000Fu), q[0], u0);
            g1 = fm_dot2(fm_as_h2(a & 0x00F000F0u), q[1], g1);
            u1 = fm_dot2(fm_as_h2(b & 0x00F000F0u), q[1], u1);
            g0 = fm_dot2(fm_as_h2(ta & 0x000F000Fu), q[2], g0);
            u0 = fm_dot2(fm_as_h2(tb & 0x000F000Fu), q[2], u0);
            g1 = fm_dot2(fm_as_h2(ta & 0x00F000F0u), q[3], g1);
            u1 = fm_dot2(fm_as_h2(tb & 0x00F000F0u), q[3], u1);
        }
    } else {
        const uint32_t gw[4] = {g.w.a.x, g.w.a.y, g.w.a.z, g.w.a.w};
        const uint32_t uw[4] = {u.w.a.x, u.w.a.y, u.w.a.z, u.w.a.w};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const fm_h2 *q = &x.q[8 * p];
            g0 = fm_dot_word2(gw[p], q, g0);
            u0 = fm_dot_word2(uw[p], q, u0);
        }
    }
    pg = __builtin_fmaf(g.s * x.inv, g0 + g1, g.b * x.sum);
    pu = __builtin_fmaf(u.s * x.inv, u0 + u1, u.b * x.sum);
}

// one group dot with four accumulator chains
template <int BITS>
__device__ __forceinline__ float fm_dot_one(const FmUnitW &g, const FmXGroup &x) {
    float c0 = 0.f, c1 = 0.f, c2 = 0.f, c3 = 0.f;
    if constexpr (BITS == 4) {
        const uint32_t gw[8] = {g.w.a.x, g.w.a.y, g.w.a.z, g.w.a.w, g.w.b.x, g.w.b.y, g.w.b.z, g.w.b.w};
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const uint32_t a = gw[p], ta = a >> 8;
            const fm_h2 *q = &x.q[4 * p];
            c0 = fm_dot2(fm_as_h2(a & 0x000F000Fu), q[0], c0);
            c1 = fm_dot2(fm_as_h2(a & 0x00F000F0u), q[1], c1);
            c2 = fm_dot2(fm_as_h2(ta & 0x000F000Fu), q[2], c2);
            c3 = fm_dot2(fm_as_h2(ta & 0x00F000F0u), q[3], c3);
        }
    } else {
        const uint32_t gw[4] = {g.w.a.x, g.w.a.y, g.w.a.z, g.w.a.w};
        c0 = fm_dot_word2(gw[0], &x.q[0], c0);
        c1 = fm_dot_word2(gw[1], &x.q[8], c1);
        c2 = fm_dot_word2(gw[2], &x.q[16], c2);
        c3 = fm_dot_word2(gw[3], &x.q[24], c3);
    }
    return __builtin_fmaf(g.s * x.inv, (c0 + c1) + (c2 + c3), g.b * x.sum);
}

template <int LH, int LI>
__global__ __launch_bounds__(256, 2) void fm_decode_eager_kernel(FmDecodeArgs a, uint32_t nwaves) {
    constexpr int RPPA = 64 / LH, RPPB = 64 / LI;
    extern __shared__ float xs[];  // x [hidden] | act [2][inter] | combine stage [4][S*RPPB]
    __shared__ FmSlot sd[FM_MAX_SLOTS];
    float *acts = xs + a.hidden;
    float *stage_all = acts + 2 * a.inter;
    const uint32_t ep_ld = fm_epoch_load(a);
    if ((int)threadIdx.x < a.S) sd[threadIdx.x] = fm_get_slot(a, threadIdx.x);
    for (uint32_t i = threadIdx.x * 4; i < a.hidden; i += 1024) *(fm_f4 *)(xs + i) = *(const fm_f4 *)(a.x + i);
    __syncthreads();
    const uint32_t ep = fm_epoch_tag(ep_ld);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t w = blockIdx.x * 4 + wv;
    const int subA = lane / LH, glA = lane % LH;
    const int subB = lane / LI, glB = lane % LI;

    const uint32_t upsA = (a.inter + RPPA - 1) / RPPA;
    const uint64_t NA = (uint64_t)a.S * upsA;
    const uint32_t u0 = (uint32_t)(NA * w / nwaves), u1 = (uint32_t)(NA * (w + 1) / nwaves);
    const uint32_t upsB = (a.hidden + RPPB - 1) / RPPB;
    const uint64_t NB = (uint64_t)a.S * upsB;
    const uint32_t v0 = (uint32_t)(NB * w / nwaves), v1 = (uint32_t)(NB * (w + 1) / nwaves);

    FM_DX_MARK(0);
    // ---- issue every weight load of this wave ----
    FmUnitW ga[FM_UMAX], ua[FM_UMAX];
#pragma unroll
    for (int i = 0; i < FM_UMAX; i++) {
        const uint32_t u = u0 + i;
        if (u < u1) {
            const int k = u / upsA;
            const FmSlot &s = sd[k];
            const uint32_t row = (u - k * upsA) * RPPA + subA;
            const bool ok = s.valid && row < a.inter && (uint32_t)glA < a.hidden / 64;
            fm_unit_load(s.gw, s.gs, s.gb, s.bits, row, a.hidden, glA, ok, ga[i]);
            fm_unit_load(s.uw, s.us, s.ub, s.bits, row, a.hidden, glA, ok, ua[i]);
        }
    }
    FmUnitW db[FM_UMAX];
    FM_DX_MARK(1);
    // ---- A: gate/up + SwiGLU -> tagged act ----
    FmXGroup xg;
    int xbits = 0;
#pragma unroll
    for (int i = 0; i < FM_UMAX; i++) {
        const uint32_t u = u0 + i;
        if (u < u1) {
            const int k = u / upsA;
            const FmSlot &s = sd[k];
            if (s.valid) {
                if (s.bits != xbits) {
                    xbits = s.bits;
                    if ((uint32_t)glA < a.hidden / 64) fm_xgroup_bits(xs + 64 * glA, xbits, xg);
                }
                const uint32_t row = (u - k * upsA) * RPPA + subA;
                const bool ok = row < a.inter && (uint32_t)glA < a.hidden / 64;
                float pg = 0.f, pu = 0.f;
                if (ok) {
                    if (s.bits == 4) {
                        fm_dot_gu<4>(ga[i], ua[i], xg, pg, pu);
                    } else {
                        fm_dot_gu<2>(ga[i], ua[i], xg, pg, pu);
                    }
                }
                pg = fm_lane_sum<LH>(pg);
                pu = fm_lane_sum<LH>(pu);
                if (glA == 0 && row < a.inter) fm_put_tagged(&a.act2[(size_t)k * a.inter + row], fm_silu_mul(pg, pu), ep);
            }
        }
        // issue down-projection unit i's loads (independent of act) between
        // gate/up computations, so the memory queue stays full while computing
        const uint32_t v = v0 + i;
        if (v < v1) {
            const int k = v / upsB;
            const FmSlot &s = sd[k];
            const uint32_t row = (v - k * upsB) * RPPB + subB;
            const bool ok = s.valid && row < a.hidden && (uint32_t)glB < a.inter / 64;
            fm_unit_load(s.dw, s.ds, s.db, s.bits, row, a.inter, glB, ok, db[i]);
        }
    }

    FM_DX_MARK(2);
    FM_DX_MARK(3);
    // ---- stage the block's down-projection slots' activations ----
    const uint32_t bv0 = (uint32_t)(NB * (blockIdx.x * 4) / nwaves);
    const uint32_t bv1 = (uint32_t)(NB * (blockIdx.x * 4 + 4) / nwaves);
    const int kb0 = bv0 / upsB;
    const int kb1 = bv1 > bv0 ? (bv1 - 1) / upsB : kb0;
    {
        // every thread issues all of its coherent loads for both slots at once,
        // then re-polls only what was not yet tagged with this call's epoch
        constexpr int MAXQ = 16;  // (2 slots x inter) / 256 threads, inter <= 2048
        uint64_t t[MAXQ];
        const int nslot = (kb1 < a.S ? kb1 : a.S - 1) - kb0 + 1;
        const uint32_t total = (uint32_t)nslot * a.inter;
#pragma unroll
        for (int q = 0; q < MAXQ; q++) {
            const uint32_t i = q * 256 + threadIdx.x;
            const int kk = kb0 + (int)(i / a.inter);
            const bool need = i < total && sd[kk].valid;
            t[q] = need ? fm_get_tagged(a.act2 + (size_t)kb0 * a.inter + i) : ((uint64_t)ep << 32);
        }
        uint32_t it = 0;
        bool ready;
        do {
            ready = true;
#pragma unroll
            for (int q = 0; q < MAXQ; q++) ready &= (uint32_t)(t[q] >> 32) == ep;
            if (__all(ready)) break;
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int q = 0; q < MAXQ; q++) {
                const uint32_t i = q * 256 + threadIdx.x;
                if ((uint32_t)(t[q] >> 32) != ep) t[q] = fm_get_tagged(a.act2 + (size_t)kb0 * a.inter + i);
            }
        } while (++it < FM_SPIN_MAX);
        if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
#pragma unroll
        for (int q = 0; q < MAXQ; q++) {
            const uint32_t i = q * 256 + threadIdx.x;
            if (i < total) acts[i] = __uint_as_float((uint32_t)t[q]);
        }
    }
    __syncthreads();

    FM_DX_MARK(4);
    // ---- B: down projection -> tagged y (or per-slot outputs) ----
    const float sw =
        (a.has_shared || a.shared_y) ? (a.shared_score ? fm_sigmoid(*a.shared_score) : a.shared_w_host) : 0.f;
    float *stage = stage_all + wv * (FM_UMAX * a.S * RPPB);
    xbits = 0;
    int xslot = -1;
#pragma unroll
    for (int i = 0; i < FM_UMAX; i++) {
        const uint32_t v = v0 + i;
        if (v < v1) {
            const int k = v / upsB;
            const FmSlot &s = sd[k];
            const uint32_t p = v - k * upsB;
            const uint32_t row = p * RPPB + subB;
            float y = 0.f;
            if (s.valid) {
                if (k != xslot || s.bits != xbits) {
                    xslot = k;
                    xbits = s.bits;
                    if ((uint32_t)glB < a.inter / 64) fm_xgroup_bits(acts + (k - kb0) * a.inter + 64 * glB, xbits, xg);
                }
                const bool ok = row < a.hidden && (uint32_t)glB < a.inter / 64;
                y = fm_lane_sum<LI>(ok ? (s.bits == 4 ? fm_dot_one<4>(db[i], xg) : fm_dot_one<2>(db[i], xg)) : 0.f);
                if (glB == 0 && row < a.hidden) {
                    if (a.mode == 1)
                        a.expert_out[(size_t)k * a.hidden + row] = y;
                    else if (k != a.S - 1)
                        fm_put_tagged(&a.y2[(size_t)k * a.hidden + row], y, ep);
                }
            }
            if (a.mode == 0 && k == a.S - 1 && glB == 0) stage[i * a.S * RPPB + (a.S - 1) * RPPB + subB] = y;
        }
    }

    FM_DX_MARK(5);
    // ---- combine the passes whose last slot this wave computed ----
    if (a.mode == 0) {
        // units [v0, v1) of the last slot -> passes; gather other slots' y for
        // all of them with one batch of coherent loads, re-poll stragglers
        const int kl = a.S - 1;
        const uint32_t lb = max(v0, (uint32_t)kl * upsB), le = min(v1, (uint32_t)(kl + 1) * upsB);
        if (lb < le) {
            const int nu = le - lb;
            const int per = kl * RPPB;          // values per pass from other slots
            const int n = nu * per;             // <= FM_UMAX * 16 * 4
            constexpr int MAXQ = (FM_UMAX * FM_MAX_SLOTS * 4 + 63) / 64;
            uint64_t t[MAXQ];
#pragma unroll
            for (int q = 0; q < MAXQ; q++) {
                const int e = q * 64 + lane;
                const int ui = e / (per > 0 ? per : 1), rem = e % (per > 0 ? per : 1);
                const int k = rem / RPPB, r = rem % RPPB;
                const uint32_t row = (lb + ui - kl * upsB) * RPPB + r;
                const bool need = e < n && sd[k].valid && row < a.hidden;
                t[q] = need ? fm_get_tagged(&a.y2[(size_t)k * a.hidden + row]) : ((uint64_t)ep << 32);
            }
            uint32_t it = 0;
            do {
                bool ready = true;
#pragma unroll
                for (int q = 0; q < MAXQ; q++) ready &= (uint32_t)(t[q] >> 32) == ep;
                if (__all(ready)) break;
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int q = 0; q < MAXQ; q++) {
                    if ((uint32_t)(t[q] >> 32) != ep) {
                        const int e = q * 64 + lane;
                        const int ui = e / per, rem = e % per;
                        const int k = rem / RPPB, r = rem % RPPB;
                        const uint32_t row = (lb + ui - kl * upsB) * RPPB + r;
                        t[q] = fm_get_tagged(&a.y2[(size_t)k * a.hidden + row]);
                    }
                }
            } while (++it < FM_SPIN_MAX);
            if (it >= FM_SPIN_MAX && lane == 0) atomicOr(a.err, FM_STATUS_WAIT_TIMEOUT);
            // stage[ui][k][r] holds every slot's y for unit ui (slot kl written above)
            const int i_of_lb = lb - v0;
#pragma unroll
            for (int q = 0; q < MAXQ; q++) {
                const int e = q * 64 + lane;
                if (e < n) {
                    const int ui = e / per, rem = e % per;
                    const int k = rem / RPPB, r = rem % RPPB;
                    stage[(i_of_lb + ui) * a.S * RPPB + k * RPPB + r] =
                        sd[k].valid ? __uint_as_float((uint32_t)t[q]) : 0.f;
                }
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            if (lane < nu * RPPB) {
                const int ui = lane / RPPB, r = lane % RPPB;
                const uint32_t row = (lb + ui - kl * upsB) * RPPB + r;
                const float *st = stage + (i_of_lb + ui) * a.S * RPPB;
                if (row < a.hidden) {
                    float moe = 0.f;
                    for (int k = 0; k < a.K; k++)
                        if (sd[k].valid) moe = __fadd_rn(moe, __fmul_rn(sd[k].weight, st[k * RPPB + r]));
                    float o = a.h_mid ? __fadd_rn(a.h_mid[row], moe) : moe;
                    if (a.has_shared) o = __fadd_rn(o, __fmul_rn(sw, st[kl * RPPB + r]));
                    else if (a.shared_y) o = __fadd_rn(o, __fmul_rn(sw, a.shared_y[row]));
                    a.out[row] = o;
                    if (a.out_bf16) a.out_bf16[row] = fm_f32_to_bf16(o);
                }
            }
        }
    }
    FM_DX_MARK(6);
    __syncthreads();
    if (threadIdx.x == 0) fm_epoch_finish(a, ep, gridDim.x);
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

// Zero fill of a workspace (a kernel, not hipMemsetAsync, so a caller may
// record it into a graph).
__global__ __launch_bounds__(256) void fm_ws_zero_kernel(fm_u4 *p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
        p[i] = (fm_u4){0u, 0u, 0u, 0u};
}

extern "C" int fm_workspace_init(void *ws, size_t ws_bytes, void *stream) {
    fm_clear_error();
    FM_REQUIRE(ws, "fm_workspace_init: NULL workspace");
    if ((uintptr_t)ws & 255) return fm_fail(FM_ERR_INVALID, "fm_workspace_init: workspace not 256-byte aligned");
    const size_t n16 = ws_bytes / 16;
    if (n16 == 0) return FM_OK;
    size_t blocks = (n16 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fm_ws_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, fm_stream(stream), (fm_u4 *)ws, n16);
    return fm_check_launch("fm_ws_zero_kernel");
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

// Workspace: [header, 256 B: status word, epoch, finished-unit count]
// [act2: S x inter x 8 B] [y2: S x hidden x 8 B]
// [ss2: hidden/64 x 8 B tagged partial sums of squares for the fused RMS norm]
// It starts zeroed (fm_workspace_init); tags make stale contents harmless after that.
// [p2: up to 4 slots x inter/16 tiles x 4 quarters x 32 tagged partial sums (the few-slot kernel)]
// [actf: S x inter x 4 B activations] [flags: 2 x hidden/16 x 8 B tagged: activation
//  flags, then norm partial sums] (the row-split kernel)
extern "C" size_t fm_moe_decode_workspace_size(int n_slots, uint32_t hidden, uint32_t inter) {
    if (n_slots < 1) n_slots = 1;
    const size_t few = n_slots < 4 ? n_slots : 4;
    return 256 + fm_align_up((size_t)n_slots * inter * 8, 256) + fm_align_up((size_t)n_slots * hidden * 8, 256) +
           fm_align_up((size_t)(hidden + 63) / 64 * 8, 256) + fm_align_up(few * (inter / 16) * 4 * 32 * 8, 256) +
           fm_align_up((size_t)n_slots * inter * 4, 256) + fm_align_up((size_t)(hidden + 15) / 16 * 16, 256);
}

template <int LH, int GH, int LI, int GI>
static int fm_launch_fused(FmDecodeArgs &a, hipStream_t st) {
    auto kern = fm_decode_fused_kernel<LH, GH, LI, GI>;
    const size_t lds = ((size_t)a.hidden + 4 * (size_t)a.inter) * sizeof(float);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds) != hipSuccess || per_cu < 1)
        return fm_fail(FM_ERR_HIP, "fm_moe_decode: occupancy query failed");
    if (per_cu > FM_DECODE_BLOCKS_PER_CU) per_cu = FM_DECODE_BLOCKS_PER_CU;
    uint32_t blocks = (uint32_t)(fm_num_cus() * per_cu);
    uint32_t nwaves = blocks * 4;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, st, a, nwaves);
    return fm_check_launch("fm_decode_fused_kernel");
}

template <int LH, int LI>
static int fm_launch_eager_t(FmDecodeArgs &a, hipStream_t st) {
    auto kern = fm_decode_eager_kernel<LH, LI>;
    const size_t lds = ((size_t)a.hidden + 2 * (size_t)a.inter + 4 * FM_UMAX * (size_t)a.S * (64 / LI)) * sizeof(float);
    if (a.inter > 2048) return fm_fail(FM_ERR_UNSUPPORTED, "eager decode: inter");
    if (lds > 65536) return fm_fail(FM_ERR_UNSUPPORTED, "eager decode: LDS");
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds) != hipSuccess || per_cu < 1)
        return fm_fail(FM_ERR_HIP, "fm_moe_decode: occupancy query failed");
    if (per_cu > FM_DECODE_BLOCKS_PER_CU) per_cu = FM_DECODE_BLOCKS_PER_CU;
    const uint32_t blocks = (uint32_t)(fm_num_cus() * per_cu);
    const uint32_t nwaves = blocks * 4;
    const uint64_t NA = (uint64_t)a.S * ((a.inter + 64 / LH - 1) / (64 / LH));
    const uint64_t NB = (uint64_t)a.S * ((a.hidden + 64 / LI - 1) / (64 / LI));
    // units per wave must fit the register-resident buffers, and one block's
    // down units may span at most two slots
    if ((NA + nwaves - 1) / nwaves > FM_UMAX || (NB + nwaves - 1) / nwaves > FM_UMAX)
        return fm_fail(FM_ERR_UNSUPPORTED, "eager decode: too many units per wave");
    const uint64_t upsB = (a.hidden + 64 / LI - 1) / (64 / LI);
    if (4 * ((NB + nwaves - 1) / nwaves) > upsB) return fm_fail(FM_ERR_UNSUPPORTED, "eager decode: slot span");
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, st, a, nwaves);
    return fm_check_launch("fm_decode_eager_kernel");
}

static int fm_launch_eager(FmDecodeArgs &a, int lh, int li, hipStream_t st) {
#define FM_E(A, B) \
    if (lh == A && li == B) return fm_launch_eager_t<A, B>(a, st);
    FM_E(64, 16) FM_E(64, 32) FM_E(64, 64) FM_E(32, 16) FM_E(32, 32) FM_E(32, 64) FM_E(16, 16) FM_E(16, 32) FM_E(16, 64)
#undef FM_E
    return fm_fail(FM_ERR_UNSUPPORTED, "eager decode: lanes");
}

// FMOE_DECODE_KERNEL=mfma|eager|fused restricts the decode step to
// one kernel family (tests and benchmarks compare them); unset = fastest that fits.
static bool fm_decode_allowed(const char *name) {
    static const char *only = getenv("FMOE_DECODE_KERNEL");
    return !only || !*only || !strcmp(only, name);
}

// hdr: the workspace header (status, epoch, finished-unit count) when the
// step's buffers are a sub-region of a larger workspace (the shared expert of
// its own size): every launch on a workspace then tags from the one epoch and
// reports into the one status word; NULL = ws itself.
static int fm_decode_launch(FmDecodeArgs &a, void *ws, size_t ws_bytes, hipStream_t st, void *hdr = nullptr) {
    const char *who = "fm_moe_decode";
    if (a.ntok <= 1) {
        a.ntok = 1;
        a.spt = a.S;
    }
    FM_REQUIRE(a.hidden % 64 == 0 && a.inter % 64 == 0 && a.hidden && a.inter,
               "%s: hidden %u / inter %u must be positive multiples of 64", who, a.hidden, a.inter);
    size_t need = fm_moe_decode_workspace_size(a.S, a.hidden, a.inter);
    if (!ws || ws_bytes < need)
        return fm_fail(FM_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu required", who, ws_bytes, need);
    if ((uintptr_t)a.x & 15) return fm_fail(FM_ERR_INVALID, "%s: x not 16-byte aligned", who);
    if ((uintptr_t)ws & 255) return fm_fail(FM_ERR_INVALID, "%s: workspace not 256-byte aligned", who);
    FM_REQUIRE(a.S * 4 <= (int)a.inter, "%s: inter %u too small for %d slots", who, a.inter, a.S);
    char *p = (char *)ws;
    char *h = hdr ? (char *)hdr : p;
    a.err = (uint32_t *)h;
    p += 256;
    a.act2 = (uint64_t *)p;
    p += fm_align_up((size_t)a.S * a.inter * 8, 256);
    a.y2 = (uint64_t *)p;
    p += fm_align_up((size_t)a.S * a.hidden * 8, 256);
    a.ss2 = (uint64_t *)p;
    p += fm_align_up((size_t)(a.hidden + 63) / 64 * 8, 256);
    a.p2 = (uint64_t *)p;
    p += fm_align_up((size_t)(a.S < 4 ? a.S : 4) * (a.inter / 16) * 4 * 32 * 8, 256);
    a.actf = (float *)p;
    p += fm_align_up((size_t)a.S * a.inter * 4, 256);
    a.flags = (uint64_t *)p;
    a.ws_epoch = (uint32_t *)(h + FM_WS_EPOCH_OFF);
    a.ws_done = (uint32_t *)(h + FM_WS_DONE_OFF);
    if (a.route_logits) {
        // routing fused into the step where the per-CU kernel runs it;
        // otherwise the routing kernel first, then the step on its outputs
        int rc = fm_decode_allowed("mfma") ? fm_launch_decode_mfma(a, st) : FM_ERR_UNSUPPORTED;
        if (rc != FM_ERR_UNSUPPORTED) return rc;
        fm_clear_error();
        rc = fm_route_topk(a.route_logits, 1, a.route_E, a.K, a.route_idx, a.route_w, st);
        if (rc) return rc;
        a.route_logits = nullptr;
        a.idx = a.route_idx;
        a.wdev = a.route_w;
    }
    if (a.ntok > 1)  // several tokens in one launch: only the mfma kernel implements it
        return fm_decode_allowed("mfma") ? fm_launch_decode_mfma(a, st)
                                         : fm_fail(FM_ERR_UNSUPPORTED, "%s: several tokens need the mfma kernel", who);
    if (a.norm_w) {
        // the fused kernels normalise in their combine; every other path runs
        // the standalone norm after the step
        int rc = fm_decode_allowed("mfma") ? fm_launch_decode_mfma(a, st) : FM_ERR_UNSUPPORTED;
        if (rc != FM_ERR_UNSUPPORTED) return rc;
        fm_clear_error();
        FmDecodeArgs b = a;
        b.norm_w = nullptr;
        rc = fm_decode_launch(b, ws, ws_bytes, st, hdr);
        if (rc) return rc;
        return fm_launch_rms_norm(a.out, a.norm_w, a.hidden, a.norm_eps, a.normed, nullptr, st);
    }
    if (((size_t)a.hidden + 4 * (size_t)a.inter) * sizeof(float) > 65536)
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: hidden + 4*inter must be <= 16384 floats", who);
    int lh, gh, li, gi;
    if (!fm_pick_lanes(a.hidden / 64, &lh, &gh) || !fm_pick_lanes(a.inter / 64, &li, &gi) || gh > 2 || gi > 2)
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: hidden %u / inter %u must be <= 8192", who, a.hidden, a.inter);
    {
        int rc = fm_decode_allowed("mfma") ? fm_launch_decode_mfma(a, st) : FM_ERR_UNSUPPORTED;
        if (rc != FM_ERR_UNSUPPORTED) return rc;
        fm_clear_error();
    }
    if (gh == 1 && gi == 1 && fm_decode_allowed("eager")) {
        int rc = fm_launch_eager(a, lh, li, st);
        if (rc != FM_ERR_UNSUPPORTED) return rc;
        fm_clear_error();
    }
    const int ch = lh * 10 + gh, ci = li * 10 + gi;
#define FM_F(A, B, C, D) \
    if (ch == A * 10 + B && ci == C * 10 + D) return fm_launch_fused<A, B, C, D>(a, st);
#define FM_FI(A, B) FM_F(A, B, 16, 1) FM_F(A, B, 32, 1) FM_F(A, B, 64, 1) FM_F(A, B, 64, 2)
    FM_FI(16, 1) FM_FI(32, 1) FM_FI(64, 1) FM_FI(64, 2)
#undef FM_FI
#undef FM_F
    return fm_fail(FM_ERR_UNSUPPORTED, "%s: no kernel instance for hidden %u / inter %u", who, a.hidden, a.inter);
}

// A shared expert whose intermediate size differs from the routed experts'
// (config.h:23 shared_intermediate) runs as its own one-slot launch (per-slot
// output mode) into the workspace tail; the routed step then adds
// sigmoid(g) * that output in its combine, in the same place of the sum.
// Workspace: [routed step: K slots][shared launch: 1 slot of shared_inter][shared y]
static bool fm_shared_apart(int K, int has_shared, uint32_t inter, uint32_t shared_inter) {
    return has_shared && K > 0 && shared_inter != 0 && shared_inter != inter;
}

extern "C" size_t fm_moe_decode_workspace_size_ex(int K, int has_shared, uint32_t hidden, uint32_t inter,
                                                  uint32_t shared_inter) {
    has_shared = has_shared ? 1 : 0;
    if (has_shared && K == 0 && shared_inter) return fm_moe_decode_workspace_size(1, hidden, shared_inter);
    if (!fm_shared_apart(K, has_shared, inter, shared_inter))
        return fm_moe_decode_workspace_size(K + has_shared, hidden, inter);
    return fm_moe_decode_workspace_size(K, hidden, inter) + fm_moe_decode_workspace_size(1, hidden, shared_inter) +
           fm_align_up((size_t)hidden * 4, 256);
}

// Launches a built step (slot K = the shared expert when has_shared), the
// shared expert apart when its intermediate size differs (one token only).
static int fm_decode_launch_shared(FmDecodeArgs &a, uint32_t shared_inter, void *ws, size_t ws_bytes,
                                   hipStream_t st) {
    if (a.has_shared && a.K == 0 && shared_inter) a.inter = shared_inter;
    if (!fm_shared_apart(a.K, a.has_shared, a.inter, shared_inter)) return fm_decode_launch(a, ws, ws_bytes, st);
    const size_t need = fm_moe_decode_workspace_size_ex(a.K, 1, a.hidden, a.inter, shared_inter);
    if (!ws || ws_bytes < need)
        return fm_fail(FM_ERR_WORKSPACE, "fm_moe_decode: workspace %zu bytes < %zu required (shared_inter %u)",
                       ws_bytes, need, shared_inter);
    const size_t main = fm_moe_decode_workspace_size(a.K, a.hidden, a.inter);
    const size_t sub = fm_moe_decode_workspace_size(1, a.hidden, shared_inter);
    float *shared_y = (float *)((char *)ws + main + sub);
    FmDecodeArgs b = {};
    b.slot[0] = a.slot[a.K];
    b.K = b.S = 1;
    b.mode = 1;
    b.hidden = a.hidden;
    b.inter = shared_inter;
    b.x = a.x;
    b.expert_out = shared_y;
    // the sub-launch's buffers lie in the tail, its header is the workspace's
    // own: its tags come from the same epoch (so they only ever grow in every
    // word of the workspace, whatever shapes alternate on it) and its status
    // bits reach fm_workspace_status
    int rc = fm_decode_launch(b, (char *)ws + main, sub, st, ws);
    if (rc) return rc;
    a.has_shared = 0;
    a.S = a.K;
    a.shared_y = shared_y;
    return fm_decode_launch(a, ws, main, st);
}

extern "C" int fm_moe_decode(int K, const fm_expert_weights *experts, const int *bits,
                             const float *weights, const int *valid,
                             const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
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
    return fm_decode_launch_shared(a, shared_inter, ws, ws_bytes, fm_stream(stream));
}

// T tokens (rows of idx/weights/x/h_mid/out/out_bf16, entries of
// shared_gate_score) in one launch; T > 1 only through fm_moe_decode_pool_tokens.
static int fm_decode_pool_impl(const char *who, const fm_expert_pool *pool, int K, const int *idx,
                               const float *weights, const fm_expert_weights *shared, int shared_bits,
                               uint32_t shared_inter, const float *shared_gate_score, const float *x, const float *h_mid, float *out,
                               uint16_t *out_bf16, const uint16_t *norm_w, float norm_eps, float *normed, void *ws,
                               size_t ws_bytes, void *stream, int T = 1, const float *route_logits = nullptr,
                               int route_E = 0) {
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
    a.norm_w = norm_w;
    a.norm_eps = norm_eps;
    a.normed = normed;
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
    if (route_logits) {
        a.route_logits = route_logits;
        a.route_E = route_E;
        a.route_idx = const_cast<int *>(idx);
        a.route_w = const_cast<float *>(weights);
    }
    if (T > 1) {
        if (fm_shared_apart(K, a.has_shared, a.inter, shared_inter))
            return fm_fail(FM_ERR_UNSUPPORTED, "%s: several tokens with a shared expert of its own size", who);
        a.ntok = T;
        a.spt = a.S;
        a.S = T * a.spt;
    }
    return fm_decode_launch_shared(a, shared_inter, ws, ws_bytes, fm_stream(stream));
}

size_t fm_moe_decode_tokens_workspace_size(int T, int K, int has_shared, uint32_t hidden, uint32_t inter) {
    return fm_moe_decode_workspace_size(T * (K + has_shared), hidden, inter);
}

int fm_moe_decode_pool_tokens(const fm_expert_pool *pool, int T, int K, const int *idx, const float *weights,
                              const fm_expert_weights *shared, int shared_bits, const float *shared_gate_scores,
                              const float *X, const float *h_mid, float *out, uint16_t *out_bf16, void *ws,
                              size_t ws_bytes, void *stream) {
    return fm_decode_pool_impl("fm_prefill_moe", pool, K, idx, weights, shared, shared_bits, 0, shared_gate_scores, X,
                               h_mid, out, out_bf16, nullptr, 0.f, nullptr, ws, ws_bytes, stream, T);
}

extern "C" int fm_moe_decode_pool(const fm_expert_pool *pool, int K, const int *idx, const float *weights,
                                  const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                                  const float *shared_gate_score, const float *x, const float *h_mid, float *out,
                                  uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream) {
    fm_clear_error();
    return fm_decode_pool_impl("fm_moe_decode_pool", pool, K, idx, weights, shared, shared_bits, shared_inter,
                               shared_gate_score, x,
                               h_mid, out, out_bf16, nullptr, 0.f, nullptr, ws, ws_bytes, stream);
}

extern "C" int fm_moe_route_decode_pool(const fm_expert_pool *pool, const float *logits, int E, int K, int *idx,
                                        float *weights, const fm_expert_weights *shared, int shared_bits,
                                        uint32_t shared_inter, const float *shared_gate_score, const float *x,
                                        const float *h_mid, float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes,
                                        void *stream) {
    const char *who = "fm_moe_route_decode_pool";
    fm_clear_error();
    FM_REQUIRE(logits && idx && weights, "%s: NULL logits/idx/weights", who);
    FM_REQUIRE(pool && pool->blobs && pool->bits && pool->num_experts, "%s: invalid pool", who);
    FM_REQUIRE(K >= 1 && K <= FM_MAX_K, "%s: K=%d outside 1..%d", who, K, FM_MAX_K);
    FM_REQUIRE(E >= K && E <= 4096 && (uint32_t)E <= pool->num_experts,
               "%s: E=%d outside K..min(4096, pool experts %u)", who, E, pool->num_experts);
    return fm_decode_pool_impl(who, pool, K, idx, weights, shared, shared_bits, shared_inter, shared_gate_score, x,
                               h_mid, out, out_bf16, nullptr, 0.f, nullptr, ws, ws_bytes, stream, 1, logits, E);
}

// ------------------------------------------------------- step by step --
// fm_moe_decode_pool_stepwise: the decode step as a chain of launches that
// never wait on one another (batched gate/up matvecs, SwiGLU, per-slot down
// matvecs, the combine): no workgroup depends on another being resident, so
// it completes whatever else occupies the GPU.  The recovery path of the layer
// driver after FM_STATUS_WAIT_TIMEOUT (fm_moe_forward_checked); it reads the
// routing on the host, so it synchronises `stream`.  The workspace is the
// step's own (fm_moe_decode_workspace_size_ex), used as plain scratch and
// re-initialised (fm_workspace_init) at the end.
extern "C" int fm_moe_decode_pool_stepwise(const fm_expert_pool *pool, int K, const int *idx, const float *weights,
                                           const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                                           const float *shared_gate_score, const float *x, const float *h_mid,
                                           float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream) {
    const char *who = "fm_moe_decode_pool_stepwise";
    fm_clear_error();
    FM_REQUIRE(pool && pool->blobs && pool->bits && pool->num_experts, "%s: invalid pool", who);
    FM_REQUIRE(K >= 0 && K <= FM_MAX_K, "%s: K=%d outside 0..%d", who, K, FM_MAX_K);
    FM_REQUIRE(K == 0 || (idx && weights), "%s: NULL idx/weights", who);
    FM_REQUIRE(K > 0 || shared, "%s: no experts", who);
    FM_REQUIRE(x && out && ws, "%s: NULL x, out or workspace", who);
    if (pool->group_size != 64) return fm_fail(FM_ERR_UNSUPPORTED, "%s: group_size must be 64", who);
    const uint32_t H = pool->hidden, I = pool->inter, Is = shared_inter ? shared_inter : I;
    const int S = K + (shared ? 1 : 0);
    const size_t need = fm_moe_decode_workspace_size_ex(K, shared ? 1 : 0, H, I, shared ? shared_inter : 0);
    const size_t scratch_bytes = 256 + fm_align_up(((size_t)K * 3 * I + (shared ? 3 * (size_t)Is : 0) +
                                                    (size_t)S * H + (size_t)K) * 4, 256);
    if (ws_bytes < need || ws_bytes < scratch_bytes)
        return fm_fail(FM_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu required", who, ws_bytes,
                       need > scratch_bytes ? need : scratch_bytes);
    if ((uintptr_t)ws & 255) return fm_fail(FM_ERR_INVALID, "%s: workspace not 256-byte aligned", who);
    hipStream_t st = fm_stream(stream);
    // the routing and the selected experts' table entries, on the host
    int hidx[FM_MAX_K] = {0}, hvalid[FM_MAX_K] = {0};
    fm_expert_weights ew[FM_MAX_SLOTS];
    int ebits[FM_MAX_SLOTS];
    hipError_t e = K ? hipMemcpyAsync(hidx, idx, sizeof(int) * K, hipMemcpyDeviceToHost, st) : hipSuccess;
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    fm_expert_layout l4, l2;
    fm_expert_layout_compute(H, I, 64, 4, &l4);
    fm_expert_layout_compute(H, I, 64, 2, &l2);
    for (int k = 0; k < K && e == hipSuccess; k++) {
        if (hidx[k] < 0 || (uint32_t)hidx[k] >= pool->num_experts) continue;  // skipped, as in the one-launch step
        const void *blob = nullptr;
        uint8_t b = 0;
        e = hipMemcpy(&blob, pool->blobs + hidx[k], sizeof blob, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(&b, pool->bits + hidx[k], 1, hipMemcpyDeviceToHost);
        if (e == hipSuccess && blob && (b == 2 || b == 4)) {
            fm_expert_from_blob(blob, b == 2 ? &l2 : &l4, &ew[k]);
            ebits[k] = b;
            hvalid[k] = 1;
        }
    }
    if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    if (shared) {
        int rc = fm_check_expert(who, K, *shared, shared_bits);
        if (rc) return rc;
        ew[K] = *shared;
        ebits[K] = shared_bits;
    }
    // scratch after the header: gate / up / act per slot, then y [S][H], then valid [K]
    float *g = (float *)((char *)ws + 256);
    float *gs[FM_MAX_SLOTS], *us[FM_MAX_SLOTS], *as[FM_MAX_SLOTS];
    {
        float *q = g;
        for (int k = 0; k < S; k++) {
            const uint32_t ik = k < K ? I : Is;
            gs[k] = q;
            us[k] = q + ik;
            as[k] = q + 2 * ik;
            q += 3 * ik;
        }
        g = q;
    }
    float *y = g;
    int *dvalid = (int *)(y + (size_t)S * H);
    fm_batch_matvec_spec specs[2 * FM_MAX_SLOTS];
    int ns = 0;
    for (int k = 0; k < S; k++) {
        if (k < K && !hvalid[k]) continue;
        const uint32_t ik = k < K ? I : Is;
        specs[ns++] = {ew[k].gate_w, ew[k].gate_s, ew[k].gate_b, gs[k], ik, H, 64, ebits[k]};
        specs[ns++] = {ew[k].up_w, ew[k].up_s, ew[k].up_b, us[k], ik, H, 64, ebits[k]};
    }
    int rc = ns ? fm_batch_matvec(x, H, specs, ns, stream) : FM_OK;
    for (int k = 0; k < S && !rc; k++) {
        if (k < K && !hvalid[k]) continue;
        const uint32_t ik = k < K ? I : Is;
        rc = fm_swiglu(gs[k], us[k], as[k], ik, stream);
        if (!rc)
            rc = fm_dequant_matvec(ew[k].down_w, ew[k].down_s, ew[k].down_b, as[k], y + (size_t)k * H, H, ik, 64,
                                   ebits[k], stream);
    }
    if (rc) return rc;
    if (K) {
        e = hipMemcpyAsync(dvalid, hvalid, sizeof(int) * K, hipMemcpyHostToDevice, st);
        if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    }
    rc = fm_moe_combine(h_mid, y, weights, K ? dvalid : nullptr, K, shared ? y + (size_t)K * H : nullptr,
                        shared ? shared_gate_score : nullptr, out, out_bf16, H, stream);
    if (rc) return rc;
    // hvalid is read by the copy above: wait for it before returning
    e = hipStreamSynchronize(st);
    if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    return fm_workspace_init(ws, ws_bytes, stream);
}

// ------------------------------------------------- no-allocation variant --
// fm_moe_decode_pool_noalloc: the same step with its workspace in a file-scope
// device array (`scratch`, FM_NOALLOC_WS_BYTES per GPU, held until the process
// ends) instead of a caller buffer.  The host only ever uses the array's device
// address from hipGetSymbolAddress, looked up once per device (the array's
// name in host code is a host-side stand-in, not a device address).  The
// first call on a device zeroes the array with a kernel; after that the
// epoch protocol needs no clearing between calls.  Every call on one GPU
// shares that GPU's array: calls that overlap on one GPU race.
static __device__ __align__(256) uint8_t scratch[FM_NOALLOC_WS_BYTES];

#define FM_NOALLOC_MAX_DEV 64
static std::mutex fm_noalloc_mu;
static void *fm_noalloc_ptr[FM_NOALLOC_MAX_DEV];

// Device address of this device's scratch array (set up on first use: symbol
// lookup, then a zero fill on `st`, ordered before the caller's step).
static int fm_noalloc_scratch(hipStream_t st, void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= FM_NOALLOC_MAX_DEV)
        return fm_fail(FM_ERR_HIP, "fm_moe_decode_pool_noalloc: no current device (or device id >= %d)",
                       FM_NOALLOC_MAX_DEV);
    std::lock_guard<std::mutex> lock(fm_noalloc_mu);
    if (!fm_noalloc_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fm_fail(FM_ERR_HIP, "fm_moe_decode_pool_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
        const int rc = fm_workspace_init(p, FM_NOALLOC_WS_BYTES, st);
        if (rc) return rc;
        fm_noalloc_ptr[dev] = p;
    }
    *out = fm_noalloc_ptr[dev];
    return FM_OK;
}

extern "C" size_t fm_noalloc_workspace_bytes(void) { return FM_NOALLOC_WS_BYTES; }

// fm_workspace_status of this device's static array: the status bits of the
// no-allocation calls since the last read (bounded-wait timeouts, skipped
// out-of-range experts, epoch wrap), then cleared.
extern "C" int fm_noalloc_status(uint32_t *status, void *stream) {
    fm_clear_error();
    FM_REQUIRE(status, "fm_noalloc_status: NULL status");
    void *ws = nullptr;
    const int rc = fm_noalloc_scratch(fm_stream(stream), &ws);
    if (rc) return rc;
    return fm_workspace_status(ws, status, stream);
}

extern "C" int fm_moe_decode_pool_noalloc(const fm_expert_pool *pool, int K, const int *idx, const float *weights,
                                          const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                                          const float *shared_gate_score, const float *x, const float *h_mid,
                                          float *out, uint16_t *out_bf16, void *stream) {
    const char *who = "fm_moe_decode_pool_noalloc";
    fm_clear_error();
    FM_REQUIRE(pool, "%s: NULL pool", who);
    FM_REQUIRE(K >= 0 && K <= FM_MAX_K, "%s: K=%d outside 0..%d", who, K, FM_MAX_K);
    const size_t need =
        fm_moe_decode_workspace_size_ex(K, shared ? 1 : 0, pool->hidden, pool->inter, shared ? shared_inter : 0);
    if (need > FM_NOALLOC_WS_BYTES)
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: K=%d, hidden %u, inter %u need a %zu-byte workspace; the static one "
                       "holds %zu bytes (use fm_moe_decode_pool with a caller workspace)", who, K, pool->hidden,
                       pool->inter, need, (size_t)FM_NOALLOC_WS_BYTES);
    void *ws = nullptr;
    const int rc = fm_noalloc_scratch(fm_stream(stream), &ws);
    if (rc) return rc;
    return fm_decode_pool_impl(who, pool, K, idx, weights, shared, shared_bits, shared_inter, shared_gate_score, x,
                               h_mid, out, out_bf16, nullptr, 0.f, nullptr, ws, FM_NOALLOC_WS_BYTES, stream);
}

extern "C" int fm_moe_decode_pool_norm(const fm_expert_pool *pool, int K, const int *idx, const float *weights,
                                       const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                                       const float *shared_gate_score, const float *x, const float *h_mid,
                                       float *out, uint16_t *out_bf16, const uint16_t *norm_w, float eps,
                                       float *normed, void *ws, size_t ws_bytes, void *stream) {
    fm_clear_error();
    FM_REQUIRE(norm_w && normed, "fm_moe_decode_pool_norm: NULL norm weights or output");
    FM_REQUIRE(eps >= 0.f, "fm_moe_decode_pool_norm: eps < 0");
    return fm_decode_pool_impl("fm_moe_decode_pool_norm", pool, K, idx, weights, shared, shared_bits, shared_inter,
                               shared_gate_score, x, h_mid, out, out_bf16, norm_w, eps, normed, ws, ws_bytes, stream);
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
