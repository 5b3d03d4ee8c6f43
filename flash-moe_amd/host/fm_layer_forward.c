/*
 * fm_layer_forward.c -- MoE layer driver (host C) over the C-ABI launchers.
 *
 * Decode mirrors moe_forward (layer_forward.h:1071-1322) and the GPU CMD2/CMD3
 * sequence of fused_layer_forward (layer_forward.h:3506-3993); prefill mirrors
 * pfb_batched_shared_expert + the per-token routed loop (batched_prefill.h:
 * 122-308), with routed experts run as one grouped GEMM instead of per token.
 * No host synchronisation: routing results stay on the device.
 */
#include "fm_layer_forward.h"

#include <stdint.h>
#include <stdlib.h>

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

/* sets fm_last_error() (fm_abi.cpp) and returns code */
int fm_host_fail(int code, const char *msg);

static int layer_ok(const fm_moe_layer *L, int K) {
    return L && L->router_w && L->router_s && L->router_b && L->pool.num_experts > 0 && K >= 1 &&
           K <= FM_MAX_K && (!L->has_shared || (L->seg_w && L->seg_s && L->seg_b));
}

size_t fm_moe_forward_workspace_size(const fm_moe_layer *L, int K) {
    if (!L) return 0;
    size_t n = align256((size_t)L->pool.num_experts * sizeof(float)); /* logits */
    n += align256(sizeof(float));                                      /* seg score */
    n += align256((size_t)K * sizeof(int));                            /* idx */
    n += align256((size_t)K * sizeof(float));                          /* weights */
    n += fm_moe_decode_workspace_size_ex(K, L->has_shared, L->pool.hidden, L->pool.inter, L->shared_inter);
    return n;
}

static int moe_forward_impl(const char *who, const fm_moe_layer *L, int K, const float *h_post, const float *h_mid,
                            float *out, uint16_t *out_bf16, const uint16_t *norm_w, float eps, float *normed,
                            void *ws, size_t ws_bytes, void *stream) {
    (void)who;
    if (!layer_ok(L, K)) return fm_host_fail(FM_ERR_INVALID, "fm_moe_forward: incomplete layer or K outside 1..FM_MAX_K");
    if (!h_post || !out) return fm_host_fail(FM_ERR_INVALID, "fm_moe_forward: NULL h_post or out");
    size_t need = fm_moe_forward_workspace_size(L, K);
    if (!ws || ws_bytes < need) return fm_host_fail(FM_ERR_WORKSPACE, "fm_moe_forward: workspace too small");
    /* [decode step's workspace: status word first][logits][seg][idx][w] */
    const size_t step =
        fm_moe_decode_workspace_size_ex(K, L->has_shared, L->pool.hidden, L->pool.inter, L->shared_inter);
    char *p = (char *)ws + step;
    float *logits = (float *)p;
    p += align256((size_t)L->pool.num_experts * sizeof(float));
    float *seg = (float *)p;
    p += align256(sizeof(float));
    int *idx = (int *)p;
    p += align256((size_t)K * sizeof(int));
    float *w = (float *)p;
    p = (char *)ws;
    size_t rest = step;

    /* CMD2: routing gate (+ shared_expert_gate) share h_post (3506-3512) */
    fm_batch_matvec_spec specs[2] = {
        {L->router_w, L->router_s, L->router_b, logits, L->pool.num_experts, L->pool.hidden,
         L->pool.group_size, L->router_bits},
        {L->seg_w, L->seg_s, L->seg_b, seg, 1, L->pool.hidden, L->pool.group_size, L->seg_bits},
    };
    int rc = fm_batch_matvec(h_post, L->pool.hidden, specs, L->has_shared ? 2 : 1, stream);
    if (rc) return rc;
    /* softmax -> top-K -> renormalise (3519-3523), then CMD3: experts + shared
     * expert + combine (3895-3993) -- one launch where the routing fuses into
     * the step */
    if (!norm_w && L->pool.num_experts <= 4096)
        return fm_moe_route_decode_pool(&L->pool, logits, (int)L->pool.num_experts, K, idx, w,
                                        L->has_shared ? &L->shared : NULL, L->shared_bits, L->shared_inter,
                                        L->has_shared ? seg : NULL, h_post, h_mid, out, out_bf16, p, rest, stream);
    rc = fm_route_topk(logits, 1, (int)L->pool.num_experts, K, idx, w, stream);
    if (rc) return rc;
    /* ... with the next layer's input RMS norm (3995-4029) */
    if (norm_w)
        return fm_moe_decode_pool_norm(&L->pool, K, idx, w, L->has_shared ? &L->shared : NULL, L->shared_bits,
                                       L->shared_inter, L->has_shared ? seg : NULL, h_post, h_mid, out, out_bf16, norm_w, eps,
                                       normed, p, rest, stream);
    return fm_moe_decode_pool(&L->pool, K, idx, w, L->has_shared ? &L->shared : NULL,
                              L->shared_bits, L->shared_inter, L->has_shared ? seg : NULL, h_post, h_mid, out,
                              out_bf16, p, rest, stream);
}

int fm_moe_forward(const fm_moe_layer *L, int K, const float *h_post, const float *h_mid,
                   float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream) {
    return moe_forward_impl("fm_moe_forward", L, K, h_post, h_mid, out, out_bf16, NULL, 0.f, NULL, ws, ws_bytes,
                            stream);
}

int fm_moe_forward_norm(const fm_moe_layer *L, int K, const float *h_post, const float *h_mid, float *out,
                        uint16_t *out_bf16, const uint16_t *next_norm_w, float eps, float *normed, void *ws,
                        size_t ws_bytes, void *stream) {
    if (!next_norm_w || !normed) return fm_host_fail(FM_ERR_INVALID, "fm_moe_forward_norm: NULL norm weights or output");
    return moe_forward_impl("fm_moe_forward_norm", L, K, h_post, h_mid, out, out_bf16, next_norm_w, eps, normed, ws,
                            ws_bytes, stream);
}

int fm_moe_forward_checked(const fm_moe_layer *L, int K, const float *h_post, const float *h_mid,
                           float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream,
                           uint32_t *status) {
    if (!status) return fm_host_fail(FM_ERR_INVALID, "fm_moe_forward_checked: NULL status");
    int rc = moe_forward_impl("fm_moe_forward_checked", L, K, h_post, h_mid, out, out_bf16, NULL, 0.f, NULL, ws,
                              ws_bytes, stream);
    if (rc) return rc;
    uint32_t st = 0;
    rc = fm_workspace_status(ws, &st, stream); /* the step's region starts the workspace */
    if (rc) return rc;
    const char *force = getenv("FMOE_FORCE_STEP_RECOVERY");
    if (force && force[0] == '1') st |= FM_STATUS_WAIT_TIMEOUT;
    if (st & FM_STATUS_WAIT_TIMEOUT) {
        /* the routing the step wrote (it needs no other workgroup) and the
         * router outputs, in the workspace layout of moe_forward_impl */
        const size_t step =
            fm_moe_decode_workspace_size_ex(K, L->has_shared, L->pool.hidden, L->pool.inter, L->shared_inter);
        char *p = (char *)ws + step;
        p += align256((size_t)L->pool.num_experts * sizeof(float));
        const float *seg = (const float *)p;
        p += align256(sizeof(float));
        const int *idx = (const int *)p;
        p += align256((size_t)K * sizeof(int));
        const float *w = (const float *)p;
        rc = fm_moe_decode_pool_stepwise(&L->pool, K, idx, w, L->has_shared ? &L->shared : NULL, L->shared_bits,
                                         L->shared_inter, L->has_shared ? seg : NULL, h_post, h_mid, out, out_bf16,
                                         ws, step, stream);
        if (rc) return rc;
        st |= FM_STATUS_RECOVERED;
    }
    *status = st;
    return FM_OK;
}

size_t fm_moe_prefill_workspace_size(const fm_moe_layer *L, int K, int T) {
    if (!L || T <= 0) return 0;
    size_t n = align256((size_t)T * L->pool.num_experts * sizeof(float)); /* logits */
    n += align256((size_t)T * sizeof(float));                             /* seg scores */
    n += align256((size_t)T * K * sizeof(int));
    n += align256((size_t)T * K * sizeof(float));
    /* the expert step's region (its header and decode-tagged words first) and
     * the router GEMM's region are disjoint: the GEMM never overwrites tags */
    n += align256(fm_pfb_gemm_workspace_size((uint32_t)T, L->pool.hidden));
    return n + align256(fm_prefill_moe_workspace_size(T, K, &L->pool, L->shared_inter));
}

int fm_moe_prefill_forward(const fm_moe_layer *L, int K, int T, const float *h_post,
                           const float *h_mid, float *out, uint16_t *out_bf16, void *ws,
                           size_t ws_bytes, void *stream) {
    if (!layer_ok(L, K)) return fm_host_fail(FM_ERR_INVALID, "fm_moe_prefill_forward: incomplete layer or bad K");
    if (T <= 0 || !h_post || !out) return fm_host_fail(FM_ERR_INVALID, "fm_moe_prefill_forward: T <= 0 or NULL buffer");
    size_t need = fm_moe_prefill_workspace_size(L, K, T);
    if (!ws || ws_bytes < need) return fm_host_fail(FM_ERR_WORKSPACE, "fm_moe_prefill_forward: workspace too small");
    /* [expert step region: header first][router GEMM region][logits][seg][idx][w] */
    const size_t step = align256(fm_prefill_moe_workspace_size(T, K, &L->pool, L->shared_inter));
    const size_t gemm = align256(fm_pfb_gemm_workspace_size((uint32_t)T, L->pool.hidden));
    char *g = (char *)ws + step;
    char *p = g + gemm;
    float *logits = (float *)p;
    p += align256((size_t)T * L->pool.num_experts * sizeof(float));
    float *seg = (float *)p;
    p += align256((size_t)T * sizeof(float));
    int *idx = (int *)p;
    p += align256((size_t)T * K * sizeof(int));
    float *w = (float *)p;
    p = (char *)ws;
    size_t rest = step;

    /* routing gate and shared_expert_gate over all tokens (batched_prefill.h:164-182) */
    int rc = fm_pfb_gemm(L->router_w, L->router_s, L->router_b, h_post, logits, (uint32_t)T,
                         L->pool.num_experts, L->pool.hidden, L->pool.group_size, L->router_bits,
                         g, gemm, stream);
    if (rc) return rc;
    if (L->has_shared) {
        rc = fm_pfb_gemm(L->seg_w, L->seg_s, L->seg_b, h_post, seg, (uint32_t)T, 1, L->pool.hidden,
                         L->pool.group_size, L->seg_bits, g, gemm, stream);
        if (rc) return rc;
    }
    /* per-token softmax / top-K / renormalise (batched_prefill.h:256-261) */
    rc = fm_route_topk(logits, T, (int)L->pool.num_experts, K, idx, w, stream);
    if (rc) return rc;
    return fm_prefill_moe(&L->pool, T, K, idx, w, L->has_shared ? &L->shared : NULL,
                          L->shared_bits, L->shared_inter, L->has_shared ? seg : NULL, h_post, h_mid, out,
                          out_bf16, p, rest, stream);
}
