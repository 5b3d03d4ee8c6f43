/*
 * fm_oracle.c -- CPU restatement of Flash-MoE's quantized-expert arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or
 * shipped).  See fm_oracle.h for the contract; each function cites the
 * reference file:line (metal_infer/...) whose semantics it restates.
 * Compiled with gcc -O2 -fno-fast-math so fp32 accumulation order matches
 * the reference's scalar loops.
 */
#include "fm_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* weights.h:9-14: bf16 bits are the top half of an f32 */
float fmo_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* weights.h:17-21: truncation (drops the low 16 bits) */
uint16_t fmo_f32_to_bf16_trunc(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return (uint16_t)(u >> 16);
}

/* IEEE round-to-nearest-even onto bf16; NaN stays a quiet NaN */
uint16_t fmo_f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
        return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/*
 * cpu_kernels.h:199-232.  For each row: acc over groups g, packed words p,
 * nibbles n (LSB first): acc += ((float)code * scale + bias) * x[8p+n],
 * one fp32 accumulator per row, this exact order.
 */
void fmo_dequant_matvec_4bit(const uint32_t *W, const uint16_t *scales,
                             const uint16_t *biases, const float *x, float *out,
                             int out_dim, int in_dim, int group_size) {
    int num_groups = in_dim / group_size;
    int words_per_group = group_size / 8;
    int words_per_row = in_dim / 8;
    for (int r = 0; r < out_dim; r++) {
        const uint32_t *wr = W + (size_t)r * words_per_row;
        const uint16_t *sr = scales + (size_t)r * num_groups;
        const uint16_t *br = biases + (size_t)r * num_groups;
        float acc = 0.0f;
        for (int g = 0; g < num_groups; g++) {
            float s = fmo_bf16_to_f32(sr[g]);
            float b = fmo_bf16_to_f32(br[g]);
            for (int p = 0; p < words_per_group; p++) {
                uint32_t word = wr[g * words_per_group + p];
                const float *xp = x + g * group_size + p * 8;
                for (int n = 0; n < 8; n++) {
                    uint32_t c = (word >> (4 * n)) & 0xFu;
                    acc += ((float)c * s + b) * xp[n];
                }
            }
        }
        out[r] = acc;
    }
}

/*
 * 2-bit analogue.  Code order from shaders.metal:515-530 and
 * repack_experts_2bit.py:170-182 (element 16p+n is (word >> 2n) & 3);
 * affine dequant c*s+b per 64-element group as in shaders.metal:447-537;
 * accumulation order is that of the 4-bit CPU loop above.
 */
void fmo_dequant_matvec_2bit(const uint32_t *W, const uint16_t *scales,
                             const uint16_t *biases, const float *x, float *out,
                             int out_dim, int in_dim, int group_size) {
    int num_groups = in_dim / group_size;
    int words_per_group = group_size / 16;
    int words_per_row = in_dim / 16;
    for (int r = 0; r < out_dim; r++) {
        const uint32_t *wr = W + (size_t)r * words_per_row;
        const uint16_t *sr = scales + (size_t)r * num_groups;
        const uint16_t *br = biases + (size_t)r * num_groups;
        float acc = 0.0f;
        for (int g = 0; g < num_groups; g++) {
            float s = fmo_bf16_to_f32(sr[g]);
            float b = fmo_bf16_to_f32(br[g]);
            for (int p = 0; p < words_per_group; p++) {
                uint32_t word = wr[g * words_per_group + p];
                const float *xp = x + g * group_size + p * 16;
                for (int n = 0; n < 16; n++) {
                    uint32_t c = (word >> (2 * n)) & 0x3u;
                    acc += ((float)c * s + b) * xp[n];
                }
            }
        }
        out[r] = acc;
    }
}

void fmo_dequant_matvec(int bits, const uint32_t *W, const uint16_t *scales,
                        const uint16_t *biases, const float *x, float *out,
                        int out_dim, int in_dim, int group_size) {
    if (bits == 2)
        fmo_dequant_matvec_2bit(W, scales, biases, x, out, out_dim, in_dim, group_size);
    else
        fmo_dequant_matvec_4bit(W, scales, biases, x, out, out_dim, in_dim, group_size);
}

/* repack_experts_2bit.py:149-161 (4-bit) and 170-182 (2-bit): codes[i*per+n] = (w>>bits*n)&mask */
void fmo_unpack_codes(int bits, const uint32_t *packed, size_t n_words, uint8_t *codes) {
    int per = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    for (size_t i = 0; i < n_words; i++)
        for (int n = 0; n < per; n++)
            codes[i * per + n] = (uint8_t)((packed[i] >> (bits * n)) & mask);
}

/* repack_experts_2bit.py:191-206 and its 4-bit analogue: LSB-first OR of shifted codes */
void fmo_pack_codes(int bits, const uint8_t *codes, size_t n_codes, uint32_t *packed) {
    int per = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    size_t n_words = n_codes / per;
    for (size_t i = 0; i < n_words; i++) {
        uint32_t w = 0;
        for (int n = 0; n < per; n++)
            w |= ((uint32_t)codes[i * per + n] & mask) << (bits * n);
        packed[i] = w;
    }
}

/* cpu_kernels.h:249-255: silu(g) = g / (1 + exp(-g)); out = silu(g) * u */
void fmo_swiglu(const float *gate, const float *up, float *out, int dim) {
    for (int i = 0; i < dim; i++) {
        float g = gate[i];
        float sg = g / (1.0f + expf(-g));
        out[i] = sg * up[i];
    }
}

/* cpu_kernels.h:258-260 */
float fmo_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* cpu_kernels.h:263-277: max, exp(x-max) with a sequential sum, times 1/sum */
/* cpu_kernels.h:235-246 */
void fmo_rms_norm(const float *x, const uint16_t *w_bf16, float *out, int dim, float eps) {
    float sum_sq = 0.0f;
    for (int i = 0; i < dim; i++) sum_sq += x[i] * x[i];
    const float rms = sqrtf(sum_sq / dim + eps);
    const float inv_rms = 1.0f / rms;
    for (int i = 0; i < dim; i++) out[i] = x[i] * inv_rms * fmo_bf16_to_f32(w_bf16[i]);
}

void fmo_softmax(float *x, int dim) {
    float mx = x[0];
    for (int i = 1; i < dim; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < dim; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < dim; i++) x[i] *= inv;
}

/*
 * cpu_kernels.h:280-299: K slots start at (-1e30, 0).  Scan i = 0..dim-1;
 * the victim is the first slot holding the smallest value; replace it when
 * scores[i] is strictly greater.  Output is in slot order (not sorted).
 */
void fmo_topk(const float *scores, int dim, int K, int *indices, float *values) {
    for (int k = 0; k < K; k++) {
        values[k] = -1e30f;
        indices[k] = 0;
    }
    for (int i = 0; i < dim; i++) {
        int mk = 0;
        for (int k = 1; k < K; k++)
            if (values[k] < values[mk]) mk = k;
        if (scores[i] > values[mk]) {
            values[mk] = scores[i];
            indices[mk] = i;
        }
    }
}

/* cpu_kernels.h:302-309 */
void fmo_normalize_weights(float *w, int K) {
    float sum = 0.0f;
    for (int k = 0; k < K; k++) sum += w[k];
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int k = 0; k < K; k++) w[k] *= inv;
    }
}

/* cpu_kernels.h:318-321 */
void fmo_vec_madd(float *dst, const float *src, float scale, int dim) {
    for (int i = 0; i < dim; i++) dst[i] += scale * src[i];
}

/* layer_forward.h:3519-3523 (and 1144-1150): softmax, top-K, renormalise */
void fmo_route(const float *logits, int E, int K, int *idx, float *w, float *probs) {
    float *p = (float *)malloc(sizeof(float) * (size_t)E);
    memcpy(p, logits, sizeof(float) * (size_t)E);
    fmo_softmax(p, E);
    fmo_topk(p, E, K, idx, w);
    fmo_normalize_weights(w, K);
    if (probs) memcpy(probs, p, sizeof(float) * (size_t)E);
    free(p);
}

/* config.h:94-137: gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b */
size_t fmo_expert_offsets(int hidden, int inter, int group_size, int bits, size_t off[9]) {
    int per = 32 / bits;
    size_t gw = (size_t)inter * ((hidden + per - 1) / per) * 4;
    size_t gsz = (size_t)inter * ((hidden + group_size - 1) / group_size) * 2;
    size_t dw = (size_t)hidden * ((inter + per - 1) / per) * 4;
    size_t dsz = (size_t)hidden * ((inter + group_size - 1) / group_size) * 2;
    size_t sizes[9] = {gw, gsz, gsz, gw, gsz, gsz, dw, dsz, dsz};
    size_t o = 0;
    for (int i = 0; i < 9; i++) {
        off[i] = o;
        o += sizes[i];
    }
    return o;
}

/* main.m:1431-1477 / layer_forward.h:1183-1202 */
void fmo_expert_forward(const uint8_t *blob, int bits, int hidden, int inter,
                        int group_size, const float *x, float *out) {
    size_t off[9];
    fmo_expert_offsets(hidden, inter, group_size, bits, off);
    float *g = (float *)malloc(sizeof(float) * (size_t)inter);
    float *u = (float *)malloc(sizeof(float) * (size_t)inter);
    float *a = (float *)malloc(sizeof(float) * (size_t)inter);
#define T32(i) ((const uint32_t *)(blob + off[i]))
#define T16(i) ((const uint16_t *)(blob + off[i]))
    fmo_dequant_matvec(bits, T32(0), T16(1), T16(2), x, g, inter, hidden, group_size);
    fmo_dequant_matvec(bits, T32(3), T16(4), T16(5), x, u, inter, hidden, group_size);
    fmo_swiglu(g, u, a, inter);
    fmo_dequant_matvec(bits, T32(6), T16(7), T16(8), a, out, hidden, inter, group_size);
#undef T32
#undef T16
    free(g);
    free(u);
    free(a);
}

/*
 * layer_forward.h:1143-1305 (CPU path of moe_forward):
 *   moe_out = 0; for k: if valid, moe_out += w_k * expert_k(x)     (1257)
 *   shared_out = shared(x) * sigmoid(score)                          (1283-1292)
 *   out[i] = h_mid[i] + moe_out[i] + shared_out[i]                  (1295-1297)
 */
void fmo_moe_decode(int K, const uint8_t *const *blobs, const int *bits,
                    const float *w, const int *valid,
                    const uint8_t *shared_blob, int shared_bits, int shared_inter, float shared_gate_score,
                    int hidden, int inter, int group_size,
                    const float *x, const float *h_mid, float *out) {
    float *moe = (float *)calloc((size_t)hidden, sizeof(float));
    float *eo = (float *)malloc(sizeof(float) * (size_t)hidden);
    float *so = (float *)calloc((size_t)hidden, sizeof(float));
    for (int k = 0; k < K; k++) {
        if (valid && !valid[k]) continue;
        fmo_expert_forward(blobs[k], bits[k], hidden, inter, group_size, x, eo);
        fmo_vec_madd(moe, eo, w[k], hidden);
    }
    if (shared_blob) {
        fmo_expert_forward(shared_blob, shared_bits, hidden, shared_inter ? shared_inter : inter, group_size, x, so);
        float sw = fmo_sigmoid(shared_gate_score);
        for (int i = 0; i < hidden; i++) so[i] *= sw;
    }
    for (int i = 0; i < hidden; i++)
        out[i] = (h_mid ? h_mid[i] : 0.0f) + moe[i] + so[i];
    free(moe);
    free(eo);
    free(so);
}

/*
 * batched_prefill.h:241-308: for each token t, routed experts in slot order
 * accumulate with cpu_vec_madd, then h = h_mid + moe + sigmoid(g_t) * shared.
 */
void fmo_prefill_moe(int T, int K, const int *idx, const float *w,
                     const uint8_t *const *blob_table, const int *bits_table,
                     const uint8_t *shared_blob, int shared_bits, int shared_inter,
                     const float *shared_gate_scores,
                     int hidden, int inter, int group_size,
                     const float *X, const float *h_mid, float *out) {
    float *moe = (float *)malloc(sizeof(float) * (size_t)hidden);
    float *eo = (float *)malloc(sizeof(float) * (size_t)hidden);
    float *so = (float *)calloc((size_t)hidden, sizeof(float));
    for (int t = 0; t < T; t++) {
        const float *x = X + (size_t)t * hidden;
        memset(moe, 0, sizeof(float) * (size_t)hidden);
        for (int k = 0; k < K; k++) {
            int e = idx[t * K + k];
            fmo_expert_forward(blob_table[e], bits_table[e], hidden, inter, group_size, x, eo);
            fmo_vec_madd(moe, eo, w[t * K + k], hidden);
        }
        float sw = 0.0f;
        if (shared_blob) {
            fmo_expert_forward(shared_blob, shared_bits, hidden, shared_inter ? shared_inter : inter, group_size, x, so);
            sw = fmo_sigmoid(shared_gate_scores ? shared_gate_scores[t] : 0.0f);
        }
        float *o = out + (size_t)t * hidden;
        const float *hm = h_mid ? h_mid + (size_t)t * hidden : NULL;
        for (int i = 0; i < hidden; i++)
            o[i] = (hm ? hm[i] : 0.0f) + moe[i] + sw * so[i];
    }
    free(moe);
    free(eo);
    free(so);
}

/* shaders.metal:2140-2216: one fp32 dot per (token, row); CPU order of the matvec */
void fmo_dequant_gemm(int bits, const uint32_t *W, const uint16_t *scales,
                      const uint16_t *biases, const float *X, float *Y,
                      int N, int out_dim, int in_dim, int group_size) {
    for (int t = 0; t < N; t++)
        fmo_dequant_matvec(bits, W, scales, biases, X + (size_t)t * in_dim,
                           Y + (size_t)t * out_dim, out_dim, in_dim, group_size);
}
