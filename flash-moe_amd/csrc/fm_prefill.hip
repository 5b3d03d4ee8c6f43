// fm_prefill.hip -- batched-prefill grouped dequant-GEMM (MFMA).  Placeholder
// until the grouped GEMM lands: the entry points report FM_ERR_UNSUPPORTED.
#include "fm_device.h"
#include "fm_internal.h"

extern "C" size_t fm_prefill_moe_workspace_size(int T, int K, const fm_expert_pool *pool) {
    (void)T; (void)K; (void)pool;
    return 0;
}

extern "C" int fm_prefill_moe(const fm_expert_pool *pool, int T, int K, const int *idx,
                              const float *weights, const fm_expert_weights *shared, int shared_bits,
                              const float *shared_gate_scores, const float *X, const float *h_mid,
                              float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream) {
    (void)pool; (void)T; (void)K; (void)idx; (void)weights; (void)shared; (void)shared_bits;
    (void)shared_gate_scores; (void)X; (void)h_mid; (void)out; (void)out_bf16; (void)ws;
    (void)ws_bytes; (void)stream;
    return fm_fail(FM_ERR_UNSUPPORTED, "fm_prefill_moe: not built yet");
}

extern "C" size_t fm_pfb_gemm_workspace_size(uint32_t N, uint32_t in_dim) {
    (void)N; (void)in_dim;
    return 0;
}

extern "C" int fm_pfb_gemm(const void *W, const void *scales, const void *biases, const float *X,
                           float *Y, uint32_t N, uint32_t out_dim, uint32_t in_dim,
                           uint32_t group_size, int bits, void *ws, size_t ws_bytes, void *stream) {
    (void)W; (void)scales; (void)biases; (void)X; (void)Y; (void)N; (void)out_dim; (void)in_dim;
    (void)group_size; (void)bits; (void)ws; (void)ws_bytes; (void)stream;
    return fm_fail(FM_ERR_UNSUPPORTED, "fm_pfb_gemm: not built yet");
}
