/*
 * fm_gpu_dispatch.h -- C ABI of the MI355X (gfx950) quantized-expert backend.
 *
 * This is the drop-in boundary for Flash-MoE's quantized-expert hot path: the
 * launchers below replace the Metal encode/dispatch functions of
 * metal_infer/gpu_dispatch.h and metal_infer/metal_ctx.h (cited per entry
 * point) with plain extern "C" calls on a HIP stream.
 *
 * Conventions (all entry points):
 *   - Pointers named W/scales/biases/x/out/... are DEVICE pointers; arrays
 *     documented as "host" are read on the host during the call only.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     Launches are asynchronous; nothing is synchronised unless stated.
 *   - Return 0 on success or a negative FM_ERR_* code; fm_last_error() then
 *     holds a message (thread-local).  The reference's void functions only
 *     print; these report instead.
 *   - Quantisation format (shaders.metal:13-25): W is uint32 [out, in*bits/32],
 *     codes LSB-first ((w >> bits*n) & mask is element (32/bits)*col + n);
 *     scales/biases are bf16 [out, in/group_size]; w = code*scale + bias.
 *     bits in {2, 4}; group_size 64 (the only size Flash-MoE models use).
 *   - Nothing allocates device memory on the hot path: the decode/prefill
 *     launchers take a caller workspace sized by the *_workspace_size query.
 *   - Calls are thread-compatible: concurrent callers use distinct streams
 *     and distinct workspaces.
 */
#ifndef FM_GPU_DISPATCH_H
#define FM_GPU_DISPATCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FM_OK 0
#define FM_ERR_INVALID (-1)     /* bad argument: null pointer, dims, bits, K */
#define FM_ERR_WORKSPACE (-2)   /* caller workspace smaller than required    */
#define FM_ERR_HIP (-3)         /* a HIP runtime call or launch failed        */
#define FM_ERR_UNSUPPORTED (-4) /* shape outside what the kernels implement   */

#define FM_MAX_K 16 /* routed experts per token (metal_ctx.h:76 MAX_K) */

/* Message for the last failing call on this thread ("" if none). */
const char *fm_last_error(void);

/* Library version string. */
const char *fm_version(void);

/* ------------------------------------------------------------------------ */
/* Expert blob layout: config.h:94-137 compute_expert_offsets().             */
/* ------------------------------------------------------------------------ */

/* Byte offsets of the 9 tensors of one packed expert (layer_XX.bin entry):
 * off[0..8] = gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s,
 * down_b; size = bytes per expert (7,077,888 for 4-bit 4096/1024/64,
 * 3,932,160 for 2-bit). */
typedef struct {
    size_t off[9];
    size_t size;
} fm_expert_layout;

int fm_expert_layout_compute(uint32_t hidden, uint32_t inter, uint32_t group_size,
                             int bits, fm_expert_layout *out);

/* Device pointers to one expert's nine tensors.  Routed experts come from a
 * blob (fm_expert_from_blob); the shared expert's tensors live separately in
 * the weight file (layer_forward.h:3506-3512, 3906-3937). */
typedef struct {
    const void *gate_w, *gate_s, *gate_b;
    const void *up_w, *up_s, *up_b;
    const void *down_w, *down_s, *down_b;
} fm_expert_weights;

int fm_expert_from_blob(const void *blob, const fm_expert_layout *layout,
                        fm_expert_weights *out);

/* A device-resident pool of experts (one MoE layer): blobs[e] is the device
 * address of expert e's packed blob, bits[e] its width (2 or 4) -- the HBM
 * counterpart of TieredExpertInfo (config.h:81-92) and expert_offset_size()
 * (timing.h:138-148).  Both arrays live in device memory. */
typedef struct {
    const void *const *blobs; /* device [num_experts] */
    const uint8_t *bits;      /* device [num_experts] */
    uint32_t num_experts;
    uint32_t hidden, inter, group_size;
} fm_expert_pool;

/* ------------------------------------------------------------------------ */
/* Dequant matvec                                                            */
/* ------------------------------------------------------------------------ */

/* out[out_dim] = dequant(W) x.  Replaces fast_dequant_matvec (metal_ctx.h:
 * 907-929) and gpu_encode_dequant_matvec_with_io_bufs (gpu_dispatch.h:
 * 162-206); `bits` selects dequant_matvec_4bit_v3 (shaders.metal:266-359) or
 * dequant_matvec_2bit (shaders.metal:447-537) semantics.  in_dim must be a
 * multiple of group_size and at most 16384. */
int fm_dequant_matvec(const void *W, const void *scales, const void *biases,
                      const float *x, float *out, uint32_t out_dim, uint32_t in_dim,
                      uint32_t group_size, int bits, void *stream);

/* gpu_dispatch.h:10-19 BatchMatvecSpec, with a device output pointer in place
 * of out_cpu/batch_slot and a per-spec bit width. */
typedef struct {
    const void *W, *scales, *biases;
    float *out;
    uint32_t out_dim, in_dim, group_size;
    int bits;
} fm_batch_matvec_spec;

/* N matvecs sharing one input x, in ONE kernel launch.  Replaces
 * gpu_batch_matvec / gpu_encode_batch_matvec / fast_batch_matvec
 * (gpu_dispatch.h:23-147, 729-742).  specs is a host array, num_specs <= 64;
 * every spec's in_dim must equal x_dim. */
int fm_batch_matvec(const float *x, uint32_t x_dim, const fm_batch_matvec_spec *specs,
                    int num_specs, void *stream);

/* ------------------------------------------------------------------------ */
/* Decode: K routed experts + shared expert, SwiGLU, weighted combine        */
/* ------------------------------------------------------------------------ */

/* Workspace bytes for fm_moe_decode / fm_moe_decode_pool(_norm) /
 * fm_encode_experts_batched with n_slots = K (+1 if a shared expert).
 * The workspace must be 256-byte aligned and start zeroed (fm_workspace_init
 * once after allocation).  Values handed between workgroups carry a per-call
 * tag that the kernels keep in the workspace header, on the device, so stale
 * contents are ignored and a call recorded into a HIP graph may be replayed.
 * Between calls nothing else may write the workspace (or re-initialise it).
 * Calls that share one workspace must be ordered (same stream); concurrent
 * calls need their own. */
size_t fm_moe_decode_workspace_size(int n_slots, uint32_t hidden, uint32_t inter);

/* Workspace bytes for a decode step of K routed experts (+ the shared expert
 * when has_shared) whose shared expert has its own intermediate size
 * shared_inter (config.h:23 shared_intermediate; 0 = inter).  Equal sizes give
 * fm_moe_decode_workspace_size(K + has_shared, ...). */
size_t fm_moe_decode_workspace_size_ex(int K, int has_shared, uint32_t hidden, uint32_t inter,
                                       uint32_t shared_inter);

/* Zero a decode / prefill / layer workspace (ws_bytes rounded down to 16 B)
 * with a kernel on `stream` (no hipMemsetAsync: recordable into a graph). */
int fm_workspace_init(void *ws, size_t ws_bytes, void *stream);

/* Status word kept in the first 4 bytes of a decode or prefill workspace
 * (fm_moe_decode*, fm_prefill_moe, fm_moe_forward*, fm_moe_prefill_forward):
 * the kernels OR in FM_STATUS_* bits and never clear them.  This call waits for
 * the work queued on `stream`, returns the accumulated bits in *status and
 * clears them.  A freshly allocated workspace holds arbitrary bits: clear it
 * once with this call (or fm_workspace_init) before relying on it.  The reference only printed
 * (e.g. "WARNING: expert %d pread" in expert_io.h:314); here the caller can ask. */
#define FM_STATUS_WAIT_TIMEOUT 1u  /* a bounded wait between workgroups gave up: output invalid */
#define FM_STATUS_BAD_EXPERT 2u    /* a routed expert index outside the pool was skipped */
#define FM_STATUS_CHUNKS 4u        /* prefill: more expert chunks than the workspace holds */
#define FM_STATUS_EPOCH_WRAP 8u    /* the per-call tag wrapped after 2^32 - 1 calls: fm_workspace_init needed */
#define FM_STATUS_RECOVERED 16u    /* fm_moe_forward_checked: the step timed out and was recomputed (output valid) */
int fm_workspace_status(void *ws, uint32_t *status, void *stream);

/* K expert FFNs sharing input x, one output per expert:
 *   expert_out[k] = down(silu(gate x) * up x)            [K][hidden] fp32
 * Replaces gpu_encode_experts_batched (gpu_dispatch.h:461-609): experts/bits
 * (and valid, may be NULL) are host arrays [K]; an expert with valid[k]==0 is
 * skipped and its output row left untouched, as in gpu_dispatch.h:485. */
int fm_encode_experts_batched(int K, const int *valid, const fm_expert_weights *experts,
                              const int *bits, uint32_t hidden, uint32_t inter,
                              uint32_t group_size, const float *x, float *expert_out,
                              void *ws, size_t ws_bytes, void *stream);

/* Weighted combine (moe_combine_residual, shaders.metal:1865-1900, with the
 * CPU semantics of layer_forward.h:1257,1295-1305 and no K<=8 limit):
 *   out[i] = h_mid[i] + sum_k w[k]*expert_outs[k][i] + sigmoid(g)*shared_out[i]
 * weights: device [K]; valid: device [K] or NULL; h_mid, shared_out,
 * shared_gate_score (device scalar g) may be NULL (terms dropped); out_bf16
 * (device, may be NULL) receives the round-to-nearest-even bf16 of out. */
int fm_moe_combine(const float *h_mid, const float *expert_outs, const float *weights,
                   const int *valid, int K, const float *shared_out,
                   const float *shared_gate_score, float *out, uint16_t *out_bf16,
                   uint32_t dim, void *stream);

/* The fused decode step (CMD3 of layer_forward.h:3895-3993): K routed experts
 * and the shared expert, gate/up/SwiGLU/down, weighted accumulation and the
 * residual, in one kernel launch.  shared_inter is the shared expert's own
 * intermediate size (config.h:23 shared_intermediate, layer_forward.h:
 * 1099-1137; 0 = inter); when it differs from inter the shared expert runs
 * as a second, one-slot launch before the step (workspace:
 * fm_moe_decode_workspace_size_ex).
 *   out = h_mid + sum_k weights[k]*E_k(x) + sigmoid(shared_gate_score)*S(x)
 * experts/bits/weights/valid are HOST arrays [K] (K <= FM_MAX_K, routing done
 * on the CPU as in layer_forward.h:3519-3523); valid may be NULL.  shared may
 * be NULL (no shared term).  h_mid and out_bf16 may be NULL. */
int fm_moe_decode(int K, const fm_expert_weights *experts, const int *bits,
                  const float *weights, const int *valid,
                  const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                  float shared_gate_score, uint32_t hidden, uint32_t inter,
                  uint32_t group_size, const float *x, const float *h_mid,
                  float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes,
                  void *stream);

/* Same step with routing on the device: idx/weights are DEVICE arrays [K]
 * (e.g. from fm_route_topk), experts come from `pool`, shared_gate_score is a
 * device scalar; NULL means the shared expert enters with weight 1.0f (no
 * sigmoid).  shared_inter as for fm_moe_decode.  No host synchronisation. */
int fm_moe_decode_pool(const fm_expert_pool *pool, int K, const int *idx,
                       const float *weights, const fm_expert_weights *shared,
                       int shared_bits, uint32_t shared_inter, const float *shared_gate_score,
                       const float *x, const float *h_mid, float *out,
                       uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream);

/* Routing and the decode step in ONE launch: cpu_softmax / cpu_topk /
 * cpu_normalize_weights of the E router logits (cpu_kernels.h:263-309, as
 * called at layer_forward.h:3519-3523) followed by CMD3 (layer_forward.h:
 * 3895-3993) on the selected pool experts -- fm_route_topk + fm_moe_decode_pool
 * without the boundary between them.  logits: device fp32 [E]; idx / weights:
 * device [K] OUTPUTS, written in cpu_topk's slot order (bit-equal to
 * fm_route_topk).  K <= FM_MAX_K, E <= min(4096, pool experts).  The weighted
 * sum of the step runs over the experts in descending probability (the output
 * differs from fm_moe_decode_pool's only by rounding).  Where the fused kernel
 * does not apply (E > 768, other shapes, no free wave group) it runs the two
 * launches.  Workspace: fm_moe_decode_workspace_size_ex, as for
 * fm_moe_decode_pool. */
int fm_moe_route_decode_pool(const fm_expert_pool *pool, const float *logits, int E, int K, int *idx,
                             float *weights, const fm_expert_weights *shared, int shared_bits,
                             uint32_t shared_inter, const float *shared_gate_score, const float *x,
                             const float *h_mid, float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes,
                             void *stream);

/* fm_moe_decode_pool as a chain of independent launches -- one batched
 * gate/up matvec launch, per slot SwiGLU and down matvec, the weighted
 * combine -- the way the reference's non-fused path runs an expert step
 * (gpu_encode_experts_batched + moe_combine_residual, gpu_dispatch.h:461-609,
 * shaders.metal:1865-1900).  No workgroup waits on another, so it completes
 * even when the one-launch step could not have all its workgroups resident
 * (FM_STATUS_WAIT_TIMEOUT); the layer driver's recovery path
 * (fm_moe_forward_checked).  Reads the routing on the host: synchronises
 * `stream`.  Same workspace as fm_moe_decode_pool (used as scratch, then
 * re-initialised with fm_workspace_init). */
int fm_moe_decode_pool_stepwise(const fm_expert_pool *pool, int K, const int *idx, const float *weights,
                                const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                                const float *shared_gate_score, const float *x, const float *h_mid,
                                float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes, void *stream);

/* act[i] = silu(gate[i]) * up[i], n elements (cpu_swiglu, cpu_kernels.h:
 * 249-255; swiglu_fused, shaders.metal:714-727).  Device fp32 arrays. */
int fm_swiglu(const float *gate, const float *up, float *act, uint32_t n, void *stream);

/* No counterpart in the reference: fm_moe_decode_pool for callers that cannot
 * allocate device memory (code recorded into a HIP graph, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and result, minus the
 * workspace: the step uses a file-scope device array of FM_NOALLOC_WS_BYTES per
 * GPU (held until the process ends; enough for K <= 16 + shared at hidden
 * 8192 / inter 2048), set up on the first call on each device -- make that
 * first call outside graph capture.  Calls nothing that allocates.  Shapes
 * whose workspace exceeds the array return FM_ERR_UNSUPPORTED.  All calls on
 * one GPU share the array: calls that overlap on one GPU (different streams,
 * host threads) race and must be serialised by the caller. */
#define FM_NOALLOC_WS_BYTES (2u << 20)
size_t fm_noalloc_workspace_bytes(void);
/* No counterpart in the reference either: the status word of this device's
 * static array (FM_STATUS_* bits of the no-allocation calls since the last
 * read, e.g. FM_STATUS_WAIT_TIMEOUT, whose step output is then invalid, or
 * FM_STATUS_BAD_EXPERT), read and cleared like fm_workspace_status (it
 * synchronises `stream`).  Poll it after a step, outside graph capture. */
int fm_noalloc_status(uint32_t *status, void *stream);
int fm_moe_decode_pool_noalloc(const fm_expert_pool *pool, int K, const int *idx,
                               const float *weights, const fm_expert_weights *shared,
                               int shared_bits, uint32_t shared_inter, const float *shared_gate_score,
                               const float *x, const float *h_mid, float *out,
                               uint16_t *out_bf16, void *stream);

/* fm_moe_decode_pool plus the next layer's input RMS norm of `out` (CMD3 Enc
 * C2/C3, layer_forward.h:3995-4029; rms_norm_sum_sq / rms_norm_apply_bf16,
 * shaders.metal:792-870; CPU semantics cpu_rms_norm, cpu_kernels.h:235-246):
 *   normed[i] = out[i] / sqrt(mean(out^2) + eps) * norm_w[i]
 * norm_w: device bf16 [hidden]; normed: device fp32 [hidden].  Fused into the
 * combine where the fused kernel runs, otherwise one extra launch. */
int fm_moe_decode_pool_norm(const fm_expert_pool *pool, int K, const int *idx,
                            const float *weights, const fm_expert_weights *shared,
                            int shared_bits, uint32_t shared_inter, const float *shared_gate_score,
                            const float *x, const float *h_mid, float *out,
                            uint16_t *out_bf16, const uint16_t *norm_w, float eps,
                            float *normed, void *ws, size_t ws_bytes, void *stream);

/* RMS norm with bf16 weights (cpu_rms_norm, cpu_kernels.h:235-246):
 *   out[i] = x[i] / sqrt(sum(x^2) / dim + eps) * w[i]
 * x, out: device fp32 [dim]; w: device bf16 [dim]; out_bf16 optional (RNE). */
int fm_rms_norm(const float *x, const uint16_t *w, uint32_t dim, float eps, float *out,
                uint16_t *out_bf16, void *stream);

/* ------------------------------------------------------------------------ */
/* Routing                                                                   */
/* ------------------------------------------------------------------------ */

/* For each of T tokens: softmax over E logits, top-K in the slot order of
 * cpu_topk, renormalised weights -- cpu_softmax / cpu_topk /
 * cpu_normalize_weights (cpu_kernels.h:263-309) as called at
 * layer_forward.h:3519-3523 and batched_prefill.h:256-261.
 * logits [T,E], idx [T,K] int32, weights [T,K] fp32; E <= 4096, K <= 64. */
int fm_route_topk(const float *logits, int T, int E, int K, int *idx, float *weights,
                  void *stream);

/* ------------------------------------------------------------------------ */
/* Prefill                                                                   */
/* ------------------------------------------------------------------------ */

/* Workspace bytes for fm_prefill_moe with T tokens, K routed per token and a
 * shared expert of intermediate size shared_inter (0 = pool->inter). */
size_t fm_prefill_moe_workspace_size(int T, int K, const fm_expert_pool *pool, uint32_t shared_inter);

/* Batched-prefill MoE layer as a per-expert grouped dequant-GEMM on MFMA.
 * Same result as the per-token loop of batched_prefill.h:241-308 plus the
 * shared expert of pfb_batched_shared_expert (batched_prefill.h:122-226):
 *   out[t] = h_mid[t] + sum_k w[t,k] E_{idx[t,k]}(X[t]) + sigmoid(g[t]) S(X[t])
 * idx/weights: device [T,K]; X, h_mid, out: device [T,hidden] fp32 (X enters
 * the matrix cores as fp16 scaled by a power of two per token, so any finite
 * magnitude keeps ~11 bits relative to the token's largest |x|); shared,
 * shared_gate_scores (device [T]), h_mid and out_bf16 may be NULL.
 * Up to 8 tokens (K <= 16, hidden 4096 / inter 1024) run as ONE launch of
 * the decode kernel over all T x (K + shared) slots (batched decode: few
 * experts are shared, so grouping buys nothing); bit-equal to
 * fm_moe_decode_pool per token.  A shared expert whose shared_inter differs
 * from pool->inter (0 = same) runs apart as three plain dequant GEMMs over all
 * tokens, as pfb_batched_shared_expert does (batched_prefill.h:122-226). */
int fm_prefill_moe(const fm_expert_pool *pool, int T, int K, const int *idx,
                   const float *weights, const fm_expert_weights *shared, int shared_bits,
                   uint32_t shared_inter, const float *shared_gate_scores, const float *X, const float *h_mid,
                   float *out, uint16_t *out_bf16, void *ws, size_t ws_bytes,
                   void *stream);

/* Workspace bytes for fm_pfb_gemm. */
size_t fm_pfb_gemm_workspace_size(uint32_t N, uint32_t in_dim);

/* Y[N,out_dim] = X[N,in_dim] dequant(W)^T on MFMA.  Replaces pfb_encode_gemm
 * (batched_prefill.h:30-67) / dequant_gemm_4bit_batch (shaders.metal:
 * 2140-2216) without the N <= 32 limit.  X is fp32 of any value (split into
 * two bf16 terms internally). */
int fm_pfb_gemm(const void *W, const void *scales, const void *biases, const float *X,
                float *Y, uint32_t N, uint32_t out_dim, uint32_t in_dim,
                uint32_t group_size, int bits, void *ws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FM_GPU_DISPATCH_H */
