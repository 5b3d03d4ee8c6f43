// fm_decode.h -- definitions shared by the decode-step kernels: slot
// descriptors, launch arguments and the epoch-tagged cross-wave hand-off.
#pragma once
#include "fm_device.h"
#include "fm_internal.h"

#define FM_MAX_SLOTS (FM_MAX_K + 1)

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
    int S;          // slots in use: ntok x spt
    int K;          // routed slots per token
    int ntok;       // tokens of the launch (mfma kernel, pool mode); others: 1
    int spt;        // slots per token (K + has_shared)
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
    const float *shared_y;     // shared expert's output computed by its own launch (own intermediate size), or NULL
    const float *x;
    const float *h_mid;
    float *out;
    uint16_t *out_bf16;
    float *expert_out;
    uint64_t *act2;  // [S][inter]  (value bits | epoch << 32) SwiGLU activations
    uint64_t *y2;    // [S][hidden] (value bits | epoch << 32) per-slot down outputs
    uint32_t *err;      // workspace status word (FM_STATUS_* bits)
    uint32_t *ws_epoch; // workspace header: tag of the last completed call
    uint32_t *ws_done;  // workspace header: counted units of the running call that finished
    // optional next-layer input RMS norm of out (cpu_kernels.h:235-246)
    const uint16_t *norm_w;  // bf16 [hidden] or NULL
    float norm_eps;
    float *normed;           // fp32 [hidden]
    uint64_t *ss2;           // [hidden/64] tagged partial sums of squares
    uint64_t *p2;            // few-slot kernel: [S][64 tiles][4 quarters][16 rows][gate, up] tagged partials
    float *actf;             // row-split kernel: [S][inter] activations (untagged; guarded by flags)
    uint64_t *flags;         // row-split kernel: [hidden / 16] tagged "activations stored" words, then [hidden / 16] norm partials
    // routing fused into the step (one token, pool mode, one-workgroup-per-CU
    // kernel): softmax / top-K / renormalise of route_logits in every
    // workgroup; idx / wdev are then unused, and the slot-order indices and
    // weights of cpu_topk / cpu_normalize_weights go to route_idx / route_w
    const float *route_logits;  // [route_E] or NULL (routing done by the caller)
    int route_E;
    int *route_idx;             // [K] out
    float *route_w;             // [K] out
};

// Slot k of token tok (routed slots of token tok read idx/wdev row tok).
__device__ __forceinline__ FmSlot fm_get_slot(const FmDecodeArgs &a, int k, int tok = 0) {
    if (!a.pool_mode || k >= a.K) return a.slot[k];
    FmSlot s;
    int e = a.idx[tok * a.K + k];
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
    s.weight = a.wdev[tok * a.K + k];
    s.valid = blob != nullptr && (bits == 2 || bits == 4);
    return s;
}

// Cross-wave hand-off without atomics read-modify-writes or cache
// maintenance.  Every handed-off value is stored together with this call's
// epoch as ONE 64-bit agent-coherent store (global_store_dwordx2 sc1); a
// consumer polls the 64-bit words it needs with agent-coherent loads until
// every tag equals the epoch.  No counters (which would serialise thousands of
// device-scope atomics on one cache line), no L2 write-back/invalidate, and no
// reset between calls.
//
// The epoch lives in the workspace header, on the device, so a call recorded
// into a graph tags each replay differently:
//   +0   status word (FM_STATUS_* bits, fm_workspace_status)
//   +64  epoch of the last completed call (0 after fm_workspace_init)
//   +128 count of the running call's finished units
// Every wave loads the header epoch at its start and tags with epoch + 1; the workgroups (or work items) that end the hand-off
// chains -- the combining ones -- bump the count after their last tagged
// access, and the last one stores the new epoch and clears the count.  Tags
// only grow, and the tagged region is written only with tags, so after
// fm_workspace_init (all zero) a stale word never carries the running call's
// tag.  (After 2^32 - 1 calls the tag wraps: the status word then reports
// FM_STATUS_EPOCH_WRAP and the workspace needs fm_workspace_init again.)
__device__ __forceinline__ void fm_put_tagged(uint64_t *p, float v, uint32_t epoch) {
    __hip_atomic_store(p, ((uint64_t)epoch << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t fm_get_tagged(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
#define FM_SPIN_MAX (1u << 16)
#define FM_WS_EPOCH_OFF 64
#define FM_WS_DONE_OFF 128

// The header epoch, loaded by every wave at its start (uniform address: one
// request per wave) and turned into the call's tag by fm_epoch_tag only where
// first needed, so no wave stalls on this load before issuing its other loads.
__device__ __forceinline__ uint32_t fm_epoch_load(const FmDecodeArgs &a) {
    return __hip_atomic_load(a.ws_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fm_epoch_tag(uint32_t loaded) {
    const uint32_t e = __builtin_amdgcn_readfirstlane(loaded) + 1u;
    return e ? e : 1u;
}

// One thread per counted unit of work, after its last tagged access: the last
// of `total` units publishes the epoch for the next call.  Counted units must
// be the ends of every hand-off chain (every wave that tags or polls a word
// feeds, directly or not, one of them), so when the last one arrives every tag
// user of this call has read the epoch (a wave's load completes before its
// first tagged access).
__device__ __forceinline__ void fm_epoch_finish(const FmDecodeArgs &a, uint32_t ep, uint32_t total) {
    if (atomicAdd(a.ws_done, 1u) == total - 1) {
        __hip_atomic_store(a.ws_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.ws_epoch, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ep == 0xFFFFFFFFu) atomicOr(a.err, FM_STATUS_EPOCH_WRAP);
    }
}

// Publishes the epoch for the next call from one unit that has, through its
// own waits, observed a tagged word of every tag user of this call (so each
// of them has already read the epoch).
__device__ __forceinline__ void fm_epoch_publish(const FmDecodeArgs &a, uint32_t ep) {
    __hip_atomic_store(a.ws_epoch, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (ep == 0xFFFFFFFFu) atomicOr(a.err, FM_STATUS_EPOCH_WRAP);
}

// Alternative launchers tried by fm_decode_launch before the eager kernel;
// each returns FM_ERR_UNSUPPORTED (message cleared by the caller) when the
// shape or slot mix is outside what it implements.
int fm_launch_decode_mfma(FmDecodeArgs &a, hipStream_t st);
int fm_launch_decode_bal(FmDecodeArgs &a, hipStream_t st);

// Standalone RMS norm launch (fm_rms_norm's kernel) for paths without the fused one.
int fm_launch_rms_norm(const float *x, const uint16_t *w, uint32_t dim, float eps, float *out, uint16_t *out_bf16,
                       hipStream_t st);
