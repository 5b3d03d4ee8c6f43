/*
 * fm_layer_forward.h -- host-side MoE layer driver over the gfx950 backend.
 *
 * C counterpart of the MoE half of the reference's layer forward: the
 * routing-gate + shared-expert-gate matvecs, softmax/top-K, K routed experts
 * + the shared expert, and the combine into the residual stream.  Everything
 * stays on the device; the calls only enqueue work on `stream`.
 */
#ifndef FM_LAYER_FORWARD_H
#define FM_LAYER_FORWARD_H

#include "fm_gpu_dispatch.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One MoE layer's device-resident weights (model.layers.N.mlp.*). */
typedef struct {
    const void *router_w, *router_s, *router_b; /* mlp.gate [num_experts, hidden]       */
    int router_bits;
    const void *seg_w, *seg_s, *seg_b;          /* mlp.shared_expert_gate [1, hidden]   */
    int seg_bits;
    fm_expert_weights shared;                   /* mlp.shared_expert.{gate,up,down}_proj */
    int shared_bits;
    int has_shared;
    fm_expert_pool pool;                        /* routed experts (packed blobs)         */
    uint32_t shared_inter;                      /* shared_expert_intermediate_size (config.h:23,200);
                                                   0 = the routed experts' pool.inter       */
} fm_moe_layer;

size_t fm_moe_forward_workspace_size(const fm_moe_layer *L, int K);

/* Decode step for one token: moe_forward (layer_forward.h:1071-1322) with the
 * GPU dispatch of fused_layer_forward (layer_forward.h:3506-3993):
 *   logits = router(h_post); g = seg(h_post)                  (3506-3512)
 *   idx, w = topK(softmax(logits)), renormalised               (3519-3523)
 *   out = h_mid + sum_k w_k E_idx[k](h_post) + sigmoid(g) S(h_post)
 * h_post, h_mid, out: device [hidden] fp32; out_bf16 optional.  Routing and
 * the expert step run as one launch (fm_moe_route_decode_pool). */
int fm_moe_forward(const fm_moe_layer *L, int K, const float *h_post, const float *h_mid,
                   float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream);

/* fm_moe_forward plus the next layer's input RMS norm of `out`, as CMD3 Enc
 * C2/C3 do (layer_forward.h:3995-4029, cpu_rms_norm cpu_kernels.h:235-246):
 *   normed[i] = out[i] / sqrt(mean(out^2) + eps) * next_norm_w[i]
 * next_norm_w: device bf16 [hidden]; normed: device fp32 [hidden].  Same
 * workspace as fm_moe_forward. */
int fm_moe_forward_norm(const fm_moe_layer *L, int K, const float *h_post, const float *h_mid, float *out,
                        uint16_t *out_bf16, const uint16_t *next_norm_w, float eps, float *normed, void *ws,
                        size_t ws_bytes, void *stream);

/* fm_moe_forward, then a check of the step: *status receives the step's
 * FM_STATUS_* bits (this call synchronises `stream`).  The one-launch step
 * needs all of its workgroups resident at once; work from other streams or
 * processes holding CUs for long can make a bounded wait give up
 * (FM_STATUS_WAIT_TIMEOUT), leaving `out` invalid.  Then the step is
 * recomputed with fm_moe_decode_pool_stepwise (independent launches, no
 * residency needed) on the routing the first launch wrote, FM_STATUS_RECOVERED
 * is added and the result is valid (an error code only if a call fails).
 * FMOE_FORCE_STEP_RECOVERY=1 in the environment takes the recovery path on
 * every call (to exercise it).  Same workspace as fm_moe_forward. */
int fm_moe_forward_checked(const fm_moe_layer *L, int K, const float *h_post, const float *h_mid,
                           float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream,
                           uint32_t *status);

size_t fm_moe_prefill_workspace_size(const fm_moe_layer *L, int K, int T);

/* Prefill of T tokens: the MoE part of batched_prefill (batched_prefill.h:
 * 122-308) -- router and shared-expert-gate GEMMs over all tokens, per-token
 * routing, then the grouped expert GEMM (routed + shared) and the combine.
 * h_post, h_mid, out: device [T, hidden] fp32. */
int fm_moe_prefill_forward(const fm_moe_layer *L, int K, int T, const float *h_post,
                           const float *h_mid, float *out, uint16_t *out_bf16, void *ws,
                           size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FM_LAYER_FORWARD_H */
