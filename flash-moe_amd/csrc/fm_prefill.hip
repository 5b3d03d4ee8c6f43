// fm_prefill.hip -- batched-prefill MoE layer as a grouped dequant-GEMM on MFMA.
//
// The reference runs routed experts during prefill as per-token matvecs
// (batched_prefill.h:241-308) and only batches the shared expert / projections
// with dequant_gemm_4bit_batch (shaders.metal:2140-2216, N <= 32 tokens).  Here
// tokens are grouped by expert and every expert's weights stream once per 16
// token columns through v_mfma_f32_16x16x32_f16:
//
//   lists   routing idx -> per-expert entry lists + 16-entry chunks (device)
//   gemm1   act[e,t] = silu(Wg x_t) * (Wu x_t)   for every (expert, token)
//   gemm2   y[e,t]   = Wd act[e,t]               into the (token, slot) row
//   combine out[t]   = h_mid + sum_k w_tk y[t,k] + sigmoid(g_t) y_shared[t]
//                      in the slot order of batched_prefill.h:296-308
//
// Exactness.  Weights never round: a masked 4-bit field with a zero fp16
// exponent IS the fp16 subnormal code * 2^-24 (or * 2^-20), and MFMA consumes
// fp16 subnormals exactly.  Each 64-element group accumulates in its own fp32
// MFMA tile, then folds  acc += s_g * 2^24 * D_g + b_g * sum(x_g)  in fp32, as
// the reference's per-group affine dequant requires.  Token activations enter
// as fp16 hi (+ fp16 lo residual for fp32 inputs), pre-scaled to match the code
// field positions; group sums come from the fp32 source.
//
// MFMA 16x16x32 operand layouts (gfx950): lane l holds A[l%16][8*(l/16)+0..7],
// B[8*(l/16)+0..7][l%16], and D[4*(l/16)+v][l%16] for v = 0..3.  A = weight
// rows (16 output features), B = 16 token columns, K = 32 codes per MFMA.
// K order inside a group is a free permutation, chosen so each lane's 8 codes
// come from one packed word (4-bit) or one half word (2-bit).
#include "fm_device.h"
#include "fm_internal.h"

typedef _Float16 fm_h8 __attribute__((ext_vector_type(8)));
typedef float fm_f4v __attribute__((ext_vector_type(4)));

#define PF_TOK 16          // token columns per chunk (one MFMA N tile)
#define PF_FEAT_WAVE 64    // output features per wave (4 MFMA M tiles)
#define PF_KB 8            // groups per LDS stage (512 inputs)
#define FM_PREFILL_DECODE_MAX_T 8  // up to this many tokens: one fused decode step per token

// One expert's matrices.
struct PfMat {
    const uint32_t *w;
    const uint16_t *s, *b;
};

struct PfArgs {
    // expert pool (device tables) + the shared expert (id == E)
    const void *const *blobs;
    const uint8_t *bits_table;
    uint64_t off4[9], off2[9];
    const uint32_t *sh_w[3];
    const uint16_t *sh_s[3], *sh_b[3];
    int sh_bits;
    int E;
    // plain single-matrix mode (fm_pfb_gemm)
    const uint32_t *pw;
    const uint16_t *ps, *pb;
    int pbits;
    int mode;  // 0: gate/up + SwiGLU, 1: down -> y rows, 2: plain matrix -> Y rows
    // work lists
    const int *chunks;  // [max_chunks][4]: expert, entry offset, count, pad
    const int *nchunks;
    const int *entries;  // entry -> slot id
    int T, K;
    uint32_t max_chunks;
    // B source rows (fp32): mode 0/2 -> X[token], mode 1 -> act[entry]
    const float *src;
    uint32_t in_dim, out_dim;
    // outputs
    float *act;   // mode 0: [entries][inter]
    float *y;     // mode 1: [slots][hidden]; mode 2: [T][out_dim]
};

__device__ __forceinline__ PfMat pf_mat(const PfArgs &a, int e, int which, int &bits) {
    PfMat m;
    if (a.mode == 2) {
        bits = a.pbits;
        m.w = a.pw;
        m.s = a.ps;
        m.b = a.pb;
        return m;
    }
    if (e == a.E) {
        bits = a.sh_bits;
        m.w = a.sh_w[which];
        m.s = a.sh_s[which];
        m.b = a.sh_b[which];
        return m;
    }
    const char *blob = (const char *)a.blobs[e];
    bits = a.bits_table[e];
    const uint64_t *off = bits == 2 ? a.off2 : a.off4;
    m.w = (const uint32_t *)(blob + off[3 * which + 0]);
    m.s = (const uint16_t *)(blob + off[3 * which + 1]);
    m.b = (const uint16_t *)(blob + off[3 * which + 2]);
    return m;
}

// slot -> B source row: token for X (mode 0/2), entry position for act (mode 1)
__device__ __forceinline__ int pf_token_of_slot(const PfArgs &a, int slot) {
    return slot < a.T * a.K ? slot / a.K : slot - a.T * a.K;
}

// A operand (8 fp16 subnormal codes) for a lane, from its packed word(s).
// 4-bit: one word w -> [c0 c4 c1' c5' c2 c6 c3' c7'] (' = *16 field)
// 2-bit: half h of word w -> h=0: pairs n=0..3, h=1: pairs n=4..7
template <int BITS>
__device__ __forceinline__ fm_h8 pf_codes(uint32_t w, int h) {
    uint32_t r0, r1, r2, r3;
    if constexpr (BITS == 4) {
        const uint32_t t = w >> 8;
        r0 = w & 0x000F000Fu;
        r1 = w & 0x00F000F0u;
        r2 = t & 0x000F000Fu;
        r3 = t & 0x00F000F0u;
    } else {
        if (h == 0) {
            r0 = w & 0x00030003u;
            r1 = w & 0x000C000Cu;
            r2 = w & 0x00300030u;
            r3 = w & 0x00C000C0u;
        } else {
            const uint32_t t = w >> 10;
            r0 = w & 0x03000300u;
            r1 = t & 0x00030003u;
            r2 = t & 0x000C000Cu;
            r3 = t & 0x00300030u;
        }
    }
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    u4v v = {r0, r1, r2, r3};
    return __builtin_bit_cast(fm_h8, v);
}

// LDS stage for one K-block of PF_KB groups:
//  hi/lo  token operands: for each of PF_TOK tokens and PF_KB groups the 64
//         inputs laid out [h=0..1][lane chunk c=0..3][8 halves] to match
//         pf_codes, with the 2^-k field scales applied (fp16 hi + fp16 lo);
//  psum   partial fp32 sums per (token, group, slot) -> sum per (token, group);
//  sc     bf16 scales/biases of the block's 256 rows: [m][s|b][group][row].
struct PfStage {
    _Float16 hi[PF_TOK][PF_KB][64];
    _Float16 lo[PF_TOK][PF_KB][64];
    float psum[PF_TOK][PF_KB][8];
    float sum[PF_TOK][PF_KB];
    uint16_t sc[2][2][PF_KB][256];
};

// Fill: task = (token, group, j), j = 0..7 one 8-half operand slot
// (h = j / 4, c = j % 4) whose inputs are two float4 runs of the source row.
template <int BITS, bool LO>
__device__ void pf_stage_fill(PfStage &st, const float *src, const int *rows, int nrows, uint32_t in_dim, int g0,
                              const PfMat *mats, int nm, int rblk, uint32_t out_dim) {
    const uint32_t G = in_dim / 64;
    for (int task = threadIdx.x; task < PF_TOK * PF_KB * 8; task += blockDim.x) {
        const int j = task & 7, gg = (task >> 3) % PF_KB, tk = task / (8 * PF_KB);
        const int h = j >> 2, c = j & 3;
        const int g = g0 + gg;
        const bool live = tk < nrows && (uint32_t)g < G;
        fm_f4 va = {0.f, 0.f, 0.f, 0.f}, vb = {0.f, 0.f, 0.f, 0.f};
        int base_a, base_b;
        float sc[8];
        if constexpr (BITS == 4) {
            // word 2c + h: elements 8w .. 8w+7, pairs (n, n+4), n = 0..3; odd n carry 2^-4
            base_a = 8 * (2 * c + h);
            base_b = base_a + 4;
            const float m[8] = {1.f, 1.f, 0.0625f, 0.0625f, 1.f, 1.f, 0.0625f, 0.0625f};
#pragma unroll
            for (int q = 0; q < 8; q++) sc[q] = m[q];
        } else {
            // word c, pairs n = 4h..4h+3: elements 16c + n and 16c + 8 + n
            base_a = 16 * c + 4 * h;
            base_b = base_a + 8;
            const float mm[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
            for (int q = 0; q < 8; q++) sc[q] = mm[4 * h + (q >> 1)];
        }
        if (live) {
            const float *x = src + (size_t)rows[tk] * in_dim + 64 * g;
            va = fm_ldg_f4(x + base_a);
            vb = fm_ldg_f4(x + base_b);
        }
        // operand order: (a0, b0, a1, b1, a2, b2, a3, b3)
        const float v[8] = {va.x, vb.x, va.y, vb.y, va.z, vb.z, va.w, vb.w};
        _Float16 *dh = &st.hi[tk][gg][j * 8];
        _Float16 *dl = &st.lo[tk][gg][j * 8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float xs = v[q] * sc[q];
            const _Float16 vh = (_Float16)xs;
            dh[q] = vh;
            if (LO) dl[q] = (_Float16)(xs - (float)vh);
        }
        st.psum[tk][gg][j] = ((va.x + va.y) + (va.z + va.w)) + ((vb.x + vb.y) + (vb.z + vb.w));
    }
    // scales/biases of the block's rows for these groups
    for (int task = threadIdx.x; task < nm * 2 * 256; task += blockDim.x) {
        const int row = task & 255, sb = (task >> 8) & 1, m = task >> 9;
        const int frow = min(rblk + row, (int)out_dim - 1);
        const uint16_t *p = (sb ? mats[m].b : mats[m].s) + (size_t)frow * G + g0;
#pragma unroll
        for (int gg = 0; gg < PF_KB; gg++) st.sc[m][sb][gg][row] = (uint32_t)(g0 + gg) < G ? fm_ldg_u16(p + gg) : 0;
    }
    __syncthreads();
    for (int task = threadIdx.x; task < PF_TOK * PF_KB; task += blockDim.x) {
        const int gg = task % PF_KB, tk = task / PF_KB;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) s += st.psum[tk][gg][j];
        st.sum[tk][gg] = s;
    }
}

template <int BITS>
__device__ __forceinline__ uint64_t pf_load_w(const PfMat &m, int row, uint32_t wpr, uint32_t g, int c) {
    if constexpr (BITS == 4) {
        return *(const FM_GLOBAL uint64_t *)(m.w + (size_t)row * wpr + 8 * g + 2 * c);
    } else {
        return *(const FM_GLOBAL uint32_t *)(m.w + (size_t)row * wpr + 4 * g + c);
    }
}

template <int BITS, bool LO, bool GU>
__device__ void pf_gemm_body(const PfArgs &a, PfStage &st, const int *rows, int nrows, const PfMat *mats, int rblk,
                             int r0, fm_f4v (&acc)[2][4]) {
    const int lane = threadIdx.x & 63;
    const int c = lane >> 4, col = lane & 15;
    const uint32_t G = a.in_dim / 64;
    const uint32_t wpr = a.in_dim * BITS / 32;
    constexpr int NM = GU ? 2 : 1;
    const int wrow0 = r0 - rblk;  // this wave's first row within the block's 256
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[m][t] = (fm_f4v){0.f, 0.f, 0.f, 0.f};
    int arow[4];
#pragma unroll
    for (int t = 0; t < 4; t++) arow[t] = min(r0 + 16 * t + (lane & 15), (int)a.out_dim - 1);

    uint64_t wcur[NM][4], wnxt[NM][4];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < 4; t++) wcur[m][t] = pf_load_w<BITS>(mats[m], arow[t], wpr, 0, c);

    for (uint32_t g0 = 0; g0 < G; g0 += PF_KB) {
        __syncthreads();
        pf_stage_fill<BITS, LO>(st, a.src, rows, nrows, a.in_dim, g0, mats, NM, rblk, a.out_dim);
        __syncthreads();
        const int ng = min((int)PF_KB, (int)(G - g0));
        for (int gg = 0; gg < ng; gg++) {
            const uint32_t g = g0 + gg;
            if (g + 1 < G) {
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int t = 0; t < 4; t++) wnxt[m][t] = pf_load_w<BITS>(mats[m], arow[t], wpr, g + 1, c);
            }
            const fm_h8 bh0 = *(const fm_h8 *)&st.hi[col][gg][(0 * 4 + c) * 8];
            const fm_h8 bh1 = *(const fm_h8 *)&st.hi[col][gg][(1 * 4 + c) * 8];
            fm_h8 bl0, bl1;
            if (LO) {
                bl0 = *(const fm_h8 *)&st.lo[col][gg][(0 * 4 + c) * 8];
                bl1 = *(const fm_h8 *)&st.lo[col][gg][(1 * 4 + c) * 8];
            }
            const float xs = st.sum[col][gg];
#pragma unroll
            for (int m = 0; m < NM; m++) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint64_t wv = wcur[m][t];
                    const uint32_t w0 = (uint32_t)wv, w1 = BITS == 4 ? (uint32_t)(wv >> 32) : (uint32_t)wv;
                    fm_f4v d = (fm_f4v){0.f, 0.f, 0.f, 0.f};
                    const fm_h8 a0 = pf_codes<BITS>(w0, 0), a1 = pf_codes<BITS>(w1, 1);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bh0, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bh1, d, 0, 0, 0);
                    if (LO) {
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bl0, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bl1, d, 0, 0, 0);
                    }
                    // fold rows 4c..4c+3 of tile t: s*2^24*D + b*sum(x)
                    const int lr = wrow0 + 16 * t + 4 * c;
                    const uint64_t s4 = *(const uint64_t *)&st.sc[m][0][gg][lr];
                    const uint64_t b4 = *(const uint64_t *)&st.sc[m][1][gg][lr];
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const float sc = fm_bf16_to_f32((uint16_t)(s4 >> (16 * v))) * 16777216.0f;
                        const float bi = fm_bf16_to_f32((uint16_t)(b4 >> (16 * v)));
                        acc[m][t][v] = __builtin_fmaf(sc, d[v], __builtin_fmaf(bi, xs, acc[m][t][v]));
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int t = 0; t < 4; t++) wcur[m][t] = wnxt[m][t];
        }
    }
}

// One block = 4 waves = 256 consecutive output features of one 16-entry chunk.
template <bool LO>
__global__ __launch_bounds__(256) void fm_pf_gemm_kernel(PfArgs a) {
    __shared__ PfStage st;
    __shared__ int rows[PF_TOK];
    __shared__ int slots[PF_TOK];
    const uint32_t nfb = (a.out_dim + 255) / 256;
    const uint32_t fb = blockIdx.x / a.max_chunks;
    const uint32_t ci = blockIdx.x % a.max_chunks;
    if ((int)ci >= *a.nchunks || fb >= nfb) return;
    const int *ch = a.chunks + 4 * ci;
    const int e = ch[0], off = ch[1], n = ch[2];
    if (threadIdx.x < PF_TOK) {
        int sl = threadIdx.x < n ? a.entries[off + threadIdx.x] : 0;
        slots[threadIdx.x] = sl;
        if (a.mode == 1)
            rows[threadIdx.x] = off + threadIdx.x;  // act row = entry position
        else if (a.mode == 2)
            rows[threadIdx.x] = sl;  // plain GEMM: entry = token row
        else
            rows[threadIdx.x] = pf_token_of_slot(a, sl);
    }
    __syncthreads();
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = fb * 256 + wv * PF_FEAT_WAVE;
    int bits = 4, bits2 = 4;
    PfMat mats[2];
    if (a.mode == 0) {
        mats[0] = pf_mat(a, e, 0, bits);
        mats[1] = pf_mat(a, e, 1, bits2);
    } else {
        mats[0] = pf_mat(a, e, a.mode == 1 ? 2 : 0, bits);
        mats[1] = mats[0];
    }
    fm_f4v acc[2][4];
    const bool live = (uint32_t)r0 < a.out_dim;
    const int rblk = fb * 256;
    if (a.mode == 0) {
        if (bits == 4)
            pf_gemm_body<4, LO, true>(a, st, rows, n, mats, rblk, r0, acc);
        else
            pf_gemm_body<2, LO, true>(a, st, rows, n, mats, rblk, r0, acc);
    } else {
        if (bits == 4)
            pf_gemm_body<4, LO, false>(a, st, rows, n, mats, rblk, r0, acc);
        else
            pf_gemm_body<2, LO, false>(a, st, rows, n, mats, rblk, r0, acc);
    }
    if (!live) return;
    const int col = lane & 15, c = lane >> 4;
    if (col >= n) return;
    const int slot = slots[col];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint32_t f = r0 + 16 * t + 4 * c + v;
            if (f >= a.out_dim) continue;
            if (a.mode == 0) {
                a.act[(size_t)(off + col) * a.out_dim + f] = fm_silu_mul(acc[0][t][v], acc[1][t][v]);
            } else {
                a.y[(size_t)slot * a.out_dim + f] = acc[0][t][v];
            }
        }
}

// ---------------------------------------------------------------- lists ----
// Single block: count tokens per expert, scan, scatter entries, cut chunks.
// Entry order inside an expert is irrelevant to the result (each token column
// is computed independently), so LDS atomics are fine.
__global__ __launch_bounds__(1024) void fm_pf_lists_kernel(const int *idx, int T, int K, int E, int has_shared,
                                                           int *entries, int *chunks, int *nchunks,
                                                           uint32_t max_chunks, int *err) {
    extern __shared__ int sm[];
    int *cnt = sm;               // [E + 1]
    int *base = sm + (E + 1);    // [E + 2]
    int *cbase = base + (E + 2); // [E + 2]
    const int NE = E + (has_shared ? 1 : 0);
    for (int i = threadIdx.x; i <= E; i += blockDim.x) cnt[i] = 0;
    __syncthreads();
    const int n = T * K;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int e = idx[i];
        if (e < 0 || e >= E) {
            atomicOr(err, 1);
            continue;
        }
        atomicAdd(&cnt[e], 1);
    }
    if (has_shared && threadIdx.x == 0) cnt[E] = T;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0, cacc = 0;
        for (int e = 0; e < NE; e++) {
            base[e] = acc;
            cbase[e] = cacc;
            acc += cnt[e];
            cacc += (cnt[e] + PF_TOK - 1) / PF_TOK;
        }
        base[NE] = acc;
        cbase[NE] = cacc;
        *nchunks = cacc <= (int)max_chunks ? cacc : (int)max_chunks;
        if (cacc > (int)max_chunks) atomicOr(err, 2);
    }
    __syncthreads();
    // chunks
    for (int e = threadIdx.x; e < NE; e += blockDim.x) {
        const int ne = cnt[e];
        for (int j = 0; j * PF_TOK < ne; j++) {
            const int ci = cbase[e] + j;
            if (ci >= (int)max_chunks) break;
            chunks[4 * ci + 0] = e;
            chunks[4 * ci + 1] = base[e] + j * PF_TOK;
            chunks[4 * ci + 2] = min(PF_TOK, ne - j * PF_TOK);
            chunks[4 * ci + 3] = 0;
        }
    }
    __syncthreads();
    // scatter entries: reuse cnt as a running cursor
    for (int i = threadIdx.x; i <= E; i += blockDim.x) cnt[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int e = idx[i];
        if (e < 0 || e >= E) continue;
        const int p = atomicAdd(&cnt[e], 1);
        entries[base[e] + p] = i;  // slot id t*K + k
    }
    if (has_shared)
        for (int t = threadIdx.x; t < T; t += blockDim.x) entries[base[E] + t] = T * K + t;
}

// ---------------------------------------------------------------- combine --
__global__ __launch_bounds__(256) void fm_pf_combine_kernel(const float *y, const float *w, int T, int K, int H,
                                                            int has_shared, const float *g, const float *h_mid,
                                                            float *out, uint16_t *out_bf16) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H || t >= T) return;
    float moe = 0.f;
    for (int k = 0; k < K; k++)
        moe = __fadd_rn(moe, __fmul_rn(w[t * K + k], y[(size_t)(t * K + k) * H + i]));
    float v = h_mid ? __fadd_rn(h_mid[(size_t)t * H + i], moe) : moe;
    if (has_shared) {
        const float sw = g ? fm_sigmoid(g[t]) : 1.0f;
        v = __fadd_rn(v, __fmul_rn(sw, y[(size_t)(T * K + t) * H + i]));
    }
    out[(size_t)t * H + i] = v;
    if (out_bf16) out_bf16[(size_t)t * H + i] = fm_f32_to_bf16(v);
}

// ---------------------------------------------------------------- host -----
static uint32_t pf_max_chunks(int T, int K, uint32_t E, int has_shared) {
    // sum_e ceil(n_e / 16) <= min(E, T*K) + T*K / 16, plus the shared expert
    uint32_t n = (uint32_t)T * K;
    uint32_t m = (n < E ? n : E) + n / PF_TOK + 1;
    if (has_shared) m += (T + PF_TOK - 1) / PF_TOK;
    return m;
}

struct PfLayout {
    size_t entries, chunks, nchunks, err, act, y, total;
};

static PfLayout pf_layout(int T, int K, uint32_t E, uint32_t hidden, uint32_t inter, int has_shared) {
    PfLayout L;
    const size_t nent = (size_t)T * K + (has_shared ? T : 0);
    const uint32_t mc = pf_max_chunks(T, K, E, has_shared);
    size_t o = 0;
    L.entries = o;
    o += fm_align_up(nent * 4, 256);
    L.chunks = o;
    o += fm_align_up((size_t)mc * 16, 256);
    L.nchunks = o;
    o += 256;
    L.err = o;
    o += 256;
    L.act = o;
    o += fm_align_up(nent * inter * 4, 256);
    L.y = o;
    o += fm_align_up(nent * hidden * 4, 256);
    L.total = o;
    return L;
}

extern "C" size_t fm_prefill_moe_workspace_size(int T, int K, const fm_expert_pool *pool) {
    if (!pool || T <= 0 || K <= 0) return 0;
    return pf_layout(T, K, pool->num_experts, pool->hidden, pool->inter, 1).total;
}

static int pf_launch_gemm(PfArgs &a, bool lo, hipStream_t st) {
    const uint32_t nfb = (a.out_dim + 255) / 256;
    dim3 grid(nfb * a.max_chunks), block(256);
    if (lo)
        hipLaunchKernelGGL(fm_pf_gemm_kernel<true>, grid, block, 0, st, a);
    else
        hipLaunchKernelGGL(fm_pf_gemm_kernel<false>, grid, block, 0, st, a);
    return fm_check_launch("fm_pf_gemm_kernel");
}

extern "C" int fm_prefill_moe(const fm_expert_pool *pool, int T, int K, const int *idx, const float *weights,
                              const fm_expert_weights *shared, int shared_bits, const float *shared_gate_scores,
                              const float *X, const float *h_mid, float *out, uint16_t *out_bf16, void *ws,
                              size_t ws_bytes, void *stream) {
    const char *who = "fm_prefill_moe";
    fm_clear_error();
    FM_REQUIRE(pool && pool->blobs && pool->bits && pool->num_experts, "%s: invalid pool", who);
    FM_REQUIRE(T >= 1 && K >= 1 && K <= 64, "%s: T=%d K=%d out of range", who, T, K);
    FM_REQUIRE(idx && weights && X && out, "%s: NULL argument", who);
    FM_REQUIRE(pool->group_size == 64, "%s: group_size must be 64", who);
    FM_REQUIRE(pool->hidden % 256 == 0 && pool->inter % 256 == 0, "%s: hidden/inter must be multiples of 256", who);
    FM_REQUIRE(pool->num_experts <= 8192, "%s: at most 8192 experts", who);
    if (shared) {
        FM_REQUIRE(shared_bits == 2 || shared_bits == 4, "%s: shared_bits must be 2 or 4", who);
    }
    const int has_shared = shared ? 1 : 0;
    PfLayout L = pf_layout(T, K, pool->num_experts, pool->hidden, pool->inter, has_shared);
    if (!ws || ws_bytes < L.total)
        return fm_fail(FM_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu required", who, ws_bytes, L.total);
    // A few tokens (batched decode): one fused decode step per token streams
    // each token's experts once at decode efficiency; the grouped GEMM only pays
    // off once experts are shared by many tokens.  Same result per token
    // (batched_prefill.h:241-308 is per-token decode arithmetic).
    if (T <= FM_PREFILL_DECODE_MAX_T && K <= FM_MAX_K) {
        const size_t dws = fm_moe_decode_workspace_size(K + has_shared, pool->hidden, pool->inter);
        if (dws <= ws_bytes) {
            for (int t = 0; t < T; t++) {
                const int rc = fm_moe_decode_pool(pool, K, idx + (size_t)t * K, weights + (size_t)t * K, shared,
                                                  shared_bits, shared_gate_scores ? shared_gate_scores + t : nullptr,
                                                  X + (size_t)t * pool->hidden,
                                                  h_mid ? h_mid + (size_t)t * pool->hidden : nullptr,
                                                  out + (size_t)t * pool->hidden,
                                                  out_bf16 ? out_bf16 + (size_t)t * pool->hidden : nullptr, ws, dws,
                                                  stream);
                if (rc) return rc;
            }
            return FM_OK;
        }
    }
    char *p = (char *)ws;
    hipStream_t st = fm_stream(stream);
    const uint32_t mc = pf_max_chunks(T, K, pool->num_experts, has_shared);

    // lists
    size_t lds = ((size_t)pool->num_experts * 3 + 5) * sizeof(int);
    if (lds > 65536) return fm_fail(FM_ERR_UNSUPPORTED, "%s: too many experts", who);
    hipLaunchKernelGGL(fm_pf_lists_kernel, dim3(1), dim3(1024), lds, st, idx, T, K, (int)pool->num_experts,
                       has_shared, (int *)(p + L.entries), (int *)(p + L.chunks), (int *)(p + L.nchunks), mc,
                       (int *)(p + L.err));
    int rc = fm_check_launch("fm_pf_lists_kernel");
    if (rc) return rc;

    PfArgs a = {};
    a.blobs = pool->blobs;
    a.bits_table = pool->bits;
    fm_expert_layout l4, l2;
    fm_expert_layout_compute(pool->hidden, pool->inter, 64, 4, &l4);
    fm_expert_layout_compute(pool->hidden, pool->inter, 64, 2, &l2);
    for (int i = 0; i < 9; i++) {
        a.off4[i] = l4.off[i];
        a.off2[i] = l2.off[i];
    }
    if (shared) {
        const void *ws9[9] = {shared->gate_w, shared->gate_s, shared->gate_b, shared->up_w, shared->up_s,
                              shared->up_b, shared->down_w, shared->down_s, shared->down_b};
        for (int m = 0; m < 3; m++) {
            a.sh_w[m] = (const uint32_t *)ws9[3 * m];
            a.sh_s[m] = (const uint16_t *)ws9[3 * m + 1];
            a.sh_b[m] = (const uint16_t *)ws9[3 * m + 2];
        }
        a.sh_bits = shared_bits;
    }
    a.E = (int)pool->num_experts;
    a.chunks = (const int *)(p + L.chunks);
    a.nchunks = (const int *)(p + L.nchunks);
    a.entries = (const int *)(p + L.entries);
    a.T = T;
    a.K = K;
    a.max_chunks = mc;
    float *act = (float *)(p + L.act);
    float *y = (float *)(p + L.y);

    // gemm1: gate/up + SwiGLU (hidden states are bf16-exact: hi only)
    a.mode = 0;
    a.src = X;
    a.in_dim = pool->hidden;
    a.out_dim = pool->inter;
    a.act = act;
    rc = pf_launch_gemm(a, false, st);
    if (rc) return rc;
    // gemm2: down projection of the fp32 activations (hi + lo)
    a.mode = 1;
    a.src = act;
    a.in_dim = pool->inter;
    a.out_dim = pool->hidden;
    a.y = y;
    rc = pf_launch_gemm(a, true, st);
    if (rc) return rc;
    // combine
    dim3 cg((pool->hidden + 255) / 256, T);
    hipLaunchKernelGGL(fm_pf_combine_kernel, cg, dim3(256), 0, st, y, weights, T, K, (int)pool->hidden, has_shared,
                       shared_gate_scores, h_mid, out, out_bf16);
    return fm_check_launch("fm_pf_combine_kernel");
}

// ---------------------------------------------------------------- pfb gemm -
// Y[N, out] = X[N, in] dequant(W)^T, X fp32 (hi + lo), one "expert" whose
// entry list is the identity.
__global__ void fm_pfb_lists_kernel(int N, int *entries, int *chunks, int *nchunks) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < N) entries[i] = i;
    const int nc = (N + PF_TOK - 1) / PF_TOK;
    if (i < nc) {
        chunks[4 * i + 0] = 0;
        chunks[4 * i + 1] = i * PF_TOK;
        chunks[4 * i + 2] = min(PF_TOK, N - i * PF_TOK);
        chunks[4 * i + 3] = 0;
    }
    if (i == 0) *nchunks = nc;
}

extern "C" size_t fm_pfb_gemm_workspace_size(uint32_t N, uint32_t in_dim) {
    (void)in_dim;
    const size_t nc = (N + PF_TOK - 1) / PF_TOK;
    return fm_align_up((size_t)N * 4, 256) + fm_align_up(nc * 16, 256) + 256;
}

extern "C" int fm_pfb_gemm(const void *W, const void *scales, const void *biases, const float *X, float *Y,
                           uint32_t N, uint32_t out_dim, uint32_t in_dim, uint32_t group_size, int bits, void *ws,
                           size_t ws_bytes, void *stream) {
    const char *who = "fm_pfb_gemm";
    fm_clear_error();
    FM_REQUIRE(W && scales && biases && X && Y, "%s: NULL argument", who);
    int rc = fm_check_dims(who, out_dim, in_dim, group_size, bits);
    if (rc) return rc;
    FM_REQUIRE(N >= 1, "%s: N=%u", who, N);
    const size_t need = fm_pfb_gemm_workspace_size(N, in_dim);
    if (!ws || ws_bytes < need) return fm_fail(FM_ERR_WORKSPACE, "%s: workspace %zu < %zu", who, ws_bytes, need);
    char *p = (char *)ws;
    int *entries = (int *)p;
    int *chunks = (int *)(p + fm_align_up((size_t)N * 4, 256));
    const size_t nc = (N + PF_TOK - 1) / PF_TOK;
    int *nchunks = (int *)(p + fm_align_up((size_t)N * 4, 256) + fm_align_up(nc * 16, 256));
    hipStream_t st = fm_stream(stream);
    const uint32_t nt = (uint32_t)(N > nc ? N : nc);
    hipLaunchKernelGGL(fm_pfb_lists_kernel, dim3((nt + 255) / 256), dim3(256), 0, st, (int)N, entries, chunks, nchunks);
    rc = fm_check_launch("fm_pfb_lists_kernel");
    if (rc) return rc;
    PfArgs a = {};
    a.mode = 2;
    a.pw = (const uint32_t *)W;
    a.ps = (const uint16_t *)scales;
    a.pb = (const uint16_t *)biases;
    a.pbits = bits;
    a.chunks = chunks;
    a.nchunks = nchunks;
    a.entries = entries;
    a.T = (int)N;
    a.K = 1;
    a.max_chunks = (uint32_t)nc;
    a.src = X;
    a.in_dim = in_dim;
    a.out_dim = out_dim;
    a.y = Y;
    return pf_launch_gemm(a, true, st);
}
