/*
 * fm_oracle.h -- CPU restatement of Flash-MoE's quantized-expert arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library (libfmoe.so) never links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the Alexintosh/flash-moe tree, metal_infer/).  Accumulation order follows
 * the reference CPU code exactly, so results are bit-identical to the
 * reference's own cpu_kernels.h compiled with the same compiler flags.
 */
#ifndef FM_ORACLE_H
#define FM_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weights.h:9-14 */
float fmo_bf16_to_f32(uint16_t v);
/* weights.h:17-21 (truncating, as the reference's offline tools do) */
uint16_t fmo_f32_to_bf16_trunc(float f);
/* round-to-nearest-even bf16; the build's output rounding (not in the reference) */
uint16_t fmo_f32_to_bf16_rne(float f);

/* cpu_kernels.h:199-232 -- 4-bit group-wise affine dequant matvec */
void fmo_dequant_matvec_4bit(const uint32_t *W, const uint16_t *scales,
                             const uint16_t *biases, const float *x, float *out,
                             int out_dim, int in_dim, int group_size);
/* shaders.metal:447-537 semantics (16 LSB-first 2-bit codes per u32), in the
 * sequential order of cpu_kernels.h:199-232; the reference has no CPU 2-bit
 * kernel */
void fmo_dequant_matvec_2bit(const uint32_t *W, const uint16_t *scales,
                             const uint16_t *biases, const float *x, float *out,
                             int out_dim, int in_dim, int group_size);
/* bits in {2,4} */
void fmo_dequant_matvec(int bits, const uint32_t *W, const uint16_t *scales,
                        const uint16_t *biases, const float *x, float *out,
                        int out_dim, int in_dim, int group_size);

/* repack_experts_2bit.py:149-161 / 170-182 -- LSB-first unpack of a u32 row */
void fmo_unpack_codes(int bits, const uint32_t *packed, size_t n_words, uint8_t *codes);
/* repack_experts_2bit.py:191-206 (and its 4-bit analogue) */
void fmo_pack_codes(int bits, const uint8_t *codes, size_t n_codes, uint32_t *packed);

void fmo_swiglu(const float *gate, const float *up, float *out, int dim);   /* cpu_kernels.h:249-255 */
float fmo_sigmoid(float x);                                                /* cpu_kernels.h:258-260 */
void fmo_softmax(float *x, int dim);
/* cpu_kernels.h:235-246 -- RMS norm with bf16 weights: sequential sum of
 * squares, rms = sqrtf(sum/dim + eps), out = x * (1/rms) * w */
void fmo_rms_norm(const float *x, const uint16_t *w_bf16, float *out, int dim, float eps);                                       /* cpu_kernels.h:263-277 */
void fmo_topk(const float *scores, int dim, int K, int *indices, float *values); /* cpu_kernels.h:280-299 */
void fmo_normalize_weights(float *w, int K);                               /* cpu_kernels.h:302-309 */
void fmo_vec_madd(float *dst, const float *src, float scale, int dim);     /* cpu_kernels.h:318-321 */

/* layer_forward.h:3519-3523: softmax over a copy of logits, top-K, renormalise.
 * probs (may be NULL) receives the full softmax. */
void fmo_route(const float *logits, int E, int K, int *idx, float *w, float *probs);

/* config.h:94-137 -- byte offsets of the 9 tensors of one expert blob.
 * off[0..8] = gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b;
 * returns the blob size. */
size_t fmo_expert_offsets(int hidden, int inter, int group_size, int bits, size_t off[9]);

/* main.m:1431-1477 / layer_forward.h:1183-1202: gate, up, SwiGLU, down. */
void fmo_expert_forward(const uint8_t *blob, int bits, int hidden, int inter,
                        int group_size, const float *x, float *out);

/* layer_forward.h:1143-1305 routed + shared combine (CPU path):
 *   moe = sum_k w_k * expert_k(x)        (cpu_vec_madd, slot order, skipped if !valid)
 *   out = h_mid + moe + sigmoid(shared_gate_score) * shared(x)
 * blobs[k] / bits[k] for the K routed experts; shared_blob may be NULL.  The
 * shared expert has its own intermediate size shared_inter (config.h:23,
 * layer_forward.h:1099-1137; 0 = inter). */
void fmo_moe_decode(int K, const uint8_t *const *blobs, const int *bits,
                    const float *w, const int *valid,
                    const uint8_t *shared_blob, int shared_bits, int shared_inter, float shared_gate_score,
                    int hidden, int inter, int group_size,
                    const float *x, const float *h_mid, float *out);

/* batched_prefill.h:241-308: per-token routed experts + shared combine.
 * idx/w are [T,K]; blob_table[e] / bits_table[e] the expert pool. */
void fmo_prefill_moe(int T, int K, const int *idx, const float *w,
                     const uint8_t *const *blob_table, const int *bits_table,
                     const uint8_t *shared_blob, int shared_bits, int shared_inter,
                     const float *shared_gate_scores,
                     int hidden, int inter, int group_size,
                     const float *X, const float *h_mid, float *out);

/* shaders.metal:2140-2216 / batched_prefill.h:30-67: Y[N,out] = X[N,in] W^T,
 * each token column exactly the 4-bit matvec above. */
void fmo_dequant_gemm(int bits, const uint32_t *W, const uint16_t *scales,
                      const uint16_t *biases, const float *X, float *Y,
                      int N, int out_dim, int in_dim, int group_size);

#ifdef __cplusplus
}
#endif
#endif
