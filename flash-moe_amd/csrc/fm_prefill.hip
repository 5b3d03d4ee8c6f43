// fm_prefill.hip -- batched-prefill MoE layer as a grouped dequant-GEMM on MFMA.
//
// The reference runs routed experts during prefill as per-token matvecs
// (batched_prefill.h:241-308) and only batches the shared expert / projections
// with dequant_gemm_4bit_batch (shaders.metal:2140-2216, N <= 32 tokens).  Here
// tokens are grouped by expert and every expert's weights stream once per 16
// tokens through v_mfma_f32_16x16x32_f16:
//
//   lists   routing idx -> per-expert entry lists + 16-entry chunks (device)
//   ops     X -> fp16 token operands (pair layouts of both code widths) + sums
//   gemm1   G[e,t] = Wg x_t, U[e,t] = Wu x_t          (separate blocks)
//   ops     act = silu(G) * U -> token operands + sums
//   gemm2   y[e,t] = Wd act[e,t]                       into the (token, slot) row
//   combine out[t] = h_mid + sum_k w_tk y[t,k] + sigmoid(g_t) y_shared[t]
//                    in the slot order of batched_prefill.h:296-308
//
// Exactness.  Weights never round: a masked 4-bit field with a zero fp16
// exponent IS the fp16 subnormal code * 2^-24 (or * 2^-20), and MFMA consumes
// fp16 subnormals exactly.  Each 64-element group accumulates in its own fp32
// MFMA tile, then folds  acc += s_g * 2^24 * D_g + b_g * sum(x_g)  in fp32, as
// the reference's per-group affine dequant requires.  Token inputs enter as
// fp16, scaled by one power of two per token row (largest |x| of the row
// lands in [2^14, 2^15), so no value overflows fp16 and small rows keep their
// precision), times the code field factors; plain fm_pfb_gemm adds an fp16
// residual term so fp32 inputs keep ~22 bits.  The row's scale is undone once,
// on the accumulated row; group sums are fp32, pre-multiplied by the same
// scale so the fold stays  acc += s_g * D_g + b_g * sum'(x_g).
//
// MFMA 16x16x32 operand layouts (gfx950): lane l holds A[l%16][8*(l/16)+0..7],
// B[8*(l/16)+0..7][l%16], and D[4*(l/16)+v][l%16] for v = 0..3.  Here A = 16
// token operands, B = 16 weight rows (codes), K = 32 codes per MFMA; a lane's
// D values are 4 tokens of one row, so the fold needs one scale per lane.
#include "fm_device.h"
#include "fm_internal.h"

typedef _Float16 fm_h8 __attribute__((ext_vector_type(8)));
typedef float fm_f4v __attribute__((ext_vector_type(4)));

#define PF_TOK 16    // token columns per MFMA N tile
#define PF_CROW 32   // ints per chunk row: expert, entry offset, count, bits, blob address (2), pad, 16 slot ids
#define PF_CHUNK PF_TOK  // entries per chunk (one block covers a chunk x 64 rows)
#define FM_PREFILL_DECODE_MAX_T 8  // up to this many tokens: decode-kernel steps instead of the grouped GEMM
#define PF_TS 36     // words per row of a wave's transpose buffer: half a 4-bit piece (32 + 4 pad: no bank conflicts)

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
    int mode;  // 0: gate and up -> G, U rows; 1: down -> y rows; 2: plain matrix -> Y rows
    // work lists
    const int *chunks;  // [max_chunks][PF_CROW] chunk rows (see fm_pf_lists_kernel)
    const int *nchunks;
    int T, K;
    uint32_t max_chunks;
    uint32_t xcd_slots;  // workgroups one XCD runs at once (eight-stage kernel: its CUs)
    // B operands: per source row and group, 32 fp16 pairs in the 4-bit [0] and
    // 2-bit [1] pair layouts (lo: residual terms, mode 2 only) + group sums.
    // Source row: mode 0 token, mode 1 entry position, mode 2 token.
    const fm_h2 *xop[2], *xlo[2];
    const float *xsum;  // group sums times the row's 2^(e - 24)
    const float *xinv;  // per source row: 2^(24 - e), applied to the finished accumulators
    uint32_t in_dim, out_dim;
    // outputs
    float *gout, *uout;  // mode 0: [entries][inter]
    float *y;            // mode 1: [slots][hidden]; mode 2: [T][out_dim]
};

// blob / cbits: the chunk row's resolved blob address and bit width (pool experts)
__device__ __forceinline__ PfMat pf_mat(const PfArgs &a, int e, int which, const char *blob, int cbits, int &bits) {
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
    bits = cbits;
    const uint64_t *off = bits == 2 ? a.off2 : a.off4;
    m.w = (const uint32_t *)(blob + off[3 * which + 0]);
    m.s = (const uint16_t *)(blob + off[3 * which + 1]);
    m.b = (const uint16_t *)(blob + off[3 * which + 2]);
    return m;
}

// slot -> source row of the B operand: token for X (mode 0/2), entry position for act
__device__ __forceinline__ int pf_token_of_slot(const PfArgs &a, int slot) {
    return slot < a.T * a.K ? slot / a.K : slot - a.T * a.K;
}

// A operand (8 fp16 subnormal codes) for a lane, from its packed word.
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
    fm_u4 v = {r0, r1, r2, r3};
    return __builtin_bit_cast(fm_h8, v);
}

// ---------------------------------------------------------------- operands -
// One source row per workgroup -> its B-operand pairs in both code layouts
// (4-bit words: (x_j, x_{j+4}) * (j odd ? 2^-4 : 1); 2-bit words:
// (x_n, x_{n+8}) / 4^(field of n)), all times the row's 2^e, optional residual
// terms, the group sums times 2^(e - 24) and the row's 2^(24 - e).  A thread
// takes 16 consecutive elements (a quarter group) per step: one pass for the
// row's largest |x|, one to convert.
__device__ __forceinline__ void pf_xop_load16(const float *src, const float *src2, size_t o, float (&v)[16]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const fm_f4 t = fm_ldg_f4(src + o + 4 * j);
        v[4 * j] = t.x;
        v[4 * j + 1] = t.y;
        v[4 * j + 2] = t.z;
        v[4 * j + 3] = t.w;
    }
    if (src2) {  // SwiGLU of separately computed gate and up rows
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const fm_f4 t = fm_ldg_f4(src2 + o + 4 * j);
            v[4 * j] = fm_silu_mul(v[4 * j], t.x);
            v[4 * j + 1] = fm_silu_mul(v[4 * j + 1], t.y);
            v[4 * j + 2] = fm_silu_mul(v[4 * j + 2], t.z);
            v[4 * j + 3] = fm_silu_mul(v[4 * j + 3], t.w);
        }
    }
}

__global__ __launch_bounds__(256) void fm_pf_xop_kernel(const float *__restrict__ src, const float *__restrict__ src2,
                                                        const int *__restrict__ nrows_dev, int nrows_max,
                                                        uint32_t in_dim, fm_h2 *x4, fm_h2 *x2, fm_h2 *l4, fm_h2 *l2,
                                                        float *xsum, float *xinv) {
    __shared__ float wmax[4];
    const uint32_t G = in_dim / 64, nq = in_dim / 16;
    const uint32_t row = blockIdx.x;
    const int nrows = nrows_dev ? *nrows_dev : nrows_max;
    if (row >= (uint32_t)nrows) return;
    const int tid = threadIdx.x;
    const size_t rbase = (size_t)row * in_dim;
    float v[16];
    float mx = 0.f;
    for (uint32_t qi = tid; qi < nq; qi += 256) {
        pf_xop_load16(src, src2, rbase + 16 * qi, v);
#pragma unroll
        for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
    }
    mx = fmaxf(mx, fm_row16_max(mx));
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 16)));
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 32)));
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 48)));
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int ex = fm_group_shift(mx);
    const float f = fm_exp2i(ex), fs = fm_exp2i(ex - 24);
    if (tid == 0) xinv[row] = fm_exp2i(24 - ex);
    float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
    for (int n = 0; n < 8; n++) mt[n] *= f;
    for (uint32_t qi = tid; qi < nq; qi += 256) {
        const uint32_t g = qi / 4, qq = qi & 3;
        pf_xop_load16(src, src2, rbase + 16 * qi, v);
        const size_t base = ((size_t)row * G + g) * 32;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float m = (j & 1) ? 0.0625f * f : f;
                const float a = v[8 * h + j] * m, b = v[8 * h + 4 + j] * m;
                const fm_h2 hi = fm_pack_h2(a, b);
                const size_t o = base + 4 * (2 * qq + h) + j;
                x4[o] = hi;
                if (l4) l4[o] = fm_pack_h2(a - (float)hi.x, b - (float)hi.y);
            }
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const float a = v[n] * mt[n], b = v[8 + n] * mt[n];
            const fm_h2 hi = fm_pack_h2(a, b);
            const size_t o = base + 8 * qq + n;
            x2[o] = hi;
            if (l2) l2[o] = fm_pack_h2(a - (float)hi.x, b - (float)hi.y);
        }
        float sm = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
        // the 4 quarters of a group are adjacent lanes (qi = tid + 256 k, 256 % 4 == 0)
        sm += __shfl_xor(sm, 1, 64);
        sm += __shfl_xor(sm, 2, 64);
        if (qq == 0) xsum[(size_t)row * G + g] = sm * fs;
    }
}

// Rows of up to 4096 inputs: each thread converts one quarter group (16
// elements) held in registers (one load pass), TPR = in_dim / 16 threads per
// row and 256 / TPR rows per workgroup, so short rows (the 1024 activations of
// an entry) fill the workgroup.  Same outputs as fm_pf_xop_kernel.
template <int TPR>
__global__ __launch_bounds__(256) void fm_pf_xop1_kernel(const float *__restrict__ src, const float *__restrict__ src2,
                                                         const int *__restrict__ nrows_dev, int nrows_max,
                                                         uint32_t in_dim, fm_h2 *x4, fm_h2 *x2, fm_h2 *l4, fm_h2 *l2,
                                                         float *xsum, float *xinv) {
    constexpr int RPW = 256 / TPR;  // rows per workgroup
    constexpr int WPR = TPR >= 64 ? TPR / 64 : 1;  // waves per row
    __shared__ float wmax[4];
    const uint32_t G = in_dim / 64;
    const int tid = threadIdx.x;
    const uint32_t row = blockIdx.x * RPW + tid / TPR, qi = tid % TPR;
    const int nrows = nrows_dev ? *nrows_dev : nrows_max;
    const bool live = row < (uint32_t)nrows;
    const size_t rbase = (size_t)(live ? row : 0) * in_dim;
    float v[16];
    pf_xop_load16(src, src2, rbase + 16 * qi, v);
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(v[j]));
#pragma unroll
    for (int o = 1; o < (TPR < 64 ? TPR : 64); o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if constexpr (WPR > 1) {
        if ((tid & 63) == 0) wmax[tid >> 6] = mx;
        __syncthreads();
        const int w0 = (tid >> 6) & ~(WPR - 1);
#pragma unroll
        for (int w = 0; w < WPR; w++) mx = fmaxf(mx, wmax[w0 + w]);
    }
    if (!live) return;
    const int ex = fm_group_shift(mx);
    const float f = fm_exp2i(ex), fs = fm_exp2i(ex - 24);
    if (qi == 0) xinv[row] = fm_exp2i(24 - ex);
    float mt[8] = {1.f, 0.25f, 0.0625f, 0.015625f, 0.00390625f, 1.f, 0.25f, 0.0625f};
#pragma unroll
    for (int n = 0; n < 8; n++) mt[n] *= f;
    const uint32_t g = qi / 4, qq = qi & 3;
    const size_t base = ((size_t)row * G + g) * 32;
    fm_h2 h4[8], h2[8];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float m = (j & 1) ? 0.0625f * f : f;
            const float a = v[8 * h + j] * m, b = v[8 * h + 4 + j] * m;
            h4[4 * h + j] = fm_pack_h2(a, b);
            if (l4) l4[base + 4 * (2 * qq + h) + j] = fm_pack_h2(a - (float)h4[4 * h + j].x, b - (float)h4[4 * h + j].y);
        }
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const float a = v[n] * mt[n], b = v[8 + n] * mt[n];
        h2[n] = fm_pack_h2(a, b);
        if (l2) l2[base + 8 * qq + n] = fm_pack_h2(a - (float)h2[n].x, b - (float)h2[n].y);
    }
    // this thread's eight pairs of either layout are contiguous: two 16-byte stores each
    fm_u4 *d4 = (fm_u4 *)(x4 + base + 8 * qq), *d2 = (fm_u4 *)(x2 + base + 8 * qq);
    d4[0] = (fm_u4){__builtin_bit_cast(uint32_t, h4[0]), __builtin_bit_cast(uint32_t, h4[1]), __builtin_bit_cast(uint32_t, h4[2]), __builtin_bit_cast(uint32_t, h4[3])};
    d4[1] = (fm_u4){__builtin_bit_cast(uint32_t, h4[4]), __builtin_bit_cast(uint32_t, h4[5]), __builtin_bit_cast(uint32_t, h4[6]), __builtin_bit_cast(uint32_t, h4[7])};
    d2[0] = (fm_u4){__builtin_bit_cast(uint32_t, h2[0]), __builtin_bit_cast(uint32_t, h2[1]), __builtin_bit_cast(uint32_t, h2[2]), __builtin_bit_cast(uint32_t, h2[3])};
    d2[1] = (fm_u4){__builtin_bit_cast(uint32_t, h2[4]), __builtin_bit_cast(uint32_t, h2[5]), __builtin_bit_cast(uint32_t, h2[6]), __builtin_bit_cast(uint32_t, h2[7])};
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j += 4) sm += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
    sm += __shfl_xor(sm, 1, 64);
    sm += __shfl_xor(sm, 2, 64);
    if (qq == 0) xsum[(size_t)row * G + g] = sm * fs;
}

// ---------------------------------------------------------------- gemm -----
// One block = 4 waves = 64 rows (16 per wave) of ONE matrix x one chunk of <=
// 16 entries of one expert.  The input dimension is walked in pieces of 8
// groups:
//  * weights stream row-contiguously (4-bit: load j gives lane l words
//    4(l%16) .. +3 of row 4j + l/16, four 256-byte row runs per instruction;
//    2-bit: 8 rows x 128 bytes per instruction) into a register ring
//    PF_RING pieces deep, together with each lane's scale/bias run of its row
//    (lane l%16 = row), and pass through the wave's LDS transpose buffer into
//    MFMA operand layout;
//  * the chunk's token operands (pre-converted fp16 pairs, 128 bytes per token
//    and group) and group sums are staged in LDS by the whole block, double
//    buffered, loaded one piece ahead: one barrier per piece.
// MFMA (src0 = tokens, src1 = codes): for group g, MFMA h takes in k slot kq
// the word 2kq + h of the group (4-bit) or half h of word kq (2-bit); the token
// operand holds the matching pairs (16(2kq + h) bytes into the group's 128-byte
// pair block).  D[token = 4q + v][row = l%16], folded per group:
//   acc_v += s_g * 2^24 * D_v + b_g * sum(x_g of token 4q + v).
#define PF_GPP 8    // groups per piece
#ifndef PF_RING
#define PF_RING 2   // pieces of weights in flight (static ring slots; even)
#endif
#define PF_XS (PF_GPP * 32 + 4)  // pairs per token row of the stage (+4: no LDS bank conflicts)
#ifndef PF_MINB
#define PF_MINB 3   // blocks per CU the register budget of the two-stage kernels is sized for (3 beats 2
                    // for the down GEMM despite register spills: more loads in flight per CU)
#endif
// 16-byte stage pieces per thread and operand array, for W waves per workgroup
#define PF_KS(W) (PF_TOK * PF_GPP * 8 / (64 * (W)))
#ifndef FM_PF_MARK
#define FM_PF_MARK(n)
#endif
#ifndef FM_PL_MARK
#define FM_PL_MARK(n)
#endif

template <bool LO>
struct PfStage {
    fm_h2 xop[LO ? 2 : 1][PF_TOK][PF_XS];
    float xsum[PF_GPP][PF_TOK];
};

template <bool LO, int W>
struct PfStageRegs {
    fm_u4 x[(LO ? 2 : 1) * PF_KS(W)];
    float xs;
};

template <int BITS>
struct PfPiece {
    fm_u4 c[BITS == 4 ? 4 : 2];
    fm_u4 s, b;  // this lane's row: scales / biases of the piece's 8 groups
};

// Branch-free stage loads (clamped addresses, zero by select) so the compiler
// keeps every load of the next piece in flight during the current one.
template <bool LO, int W>
__device__ __forceinline__ void pf_stage_load(const PfArgs &a, const int *srow, const fm_h2 *xop, const fm_h2 *xlo,
                                              uint32_t g0, PfStageRegs<LO, W> &r) {
    constexpr int KS = PF_KS(W);
    const int t = threadIdx.x;
    const uint32_t G = a.in_dim / 64;
#pragma unroll
    for (int k = 0; k < (LO ? 2 : 1) * KS; k++) {
        const int i = t + 64 * W * (k % KS);
        const int tok = i >> 6, gg = (i >> 3) & 7, part = i & 7;
        const int sr = srow[tok];
        const uint32_t g = g0 + gg;
        const bool ok = sr >= 0 && g < G;
        const fm_h2 *base = k < KS ? xop : xlo;
        const fm_u4 v = *(const FM_GLOBAL fm_u4 *)(base + ((size_t)(ok ? sr : 0) * G + (ok ? g : 0)) * 32 + 4 * part);
        r.x[k] = ok ? v : (fm_u4){0u, 0u, 0u, 0u};
    }
    const int tok = t & 15, gg = (t >> 4) & 7;
    const int sr = srow[tok];
    const bool ok = sr >= 0 && g0 + gg < G;
    const float v = fm_ldg_f32(a.xsum + (size_t)(ok ? sr : 0) * G + (ok ? g0 + gg : 0));
    r.xs = ok ? v : 0.f;
}

template <bool LO, int W>
__device__ __forceinline__ void pf_stage_store(PfStage<LO> &st, const PfStageRegs<LO, W> &r) {
    constexpr int KS = PF_KS(W);
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < (LO ? 2 : 1) * KS; k++) {
        const int i = t + 64 * W * (k % KS);
        const int tok = i >> 6, gg = (i >> 3) & 7, part = i & 7;
        *(fm_u4 *)&st.xop[k / KS][tok][32 * gg + 4 * part] = r.x[k];
    }
    if (t < PF_TOK * PF_GPP) st.xsum[(t >> 4) & 7][t & 15] = r.xs;
}

// Row-tile count of a workgroup: when the whole input fits the stages the
// chunk's operands stay resident in LDS and one workgroup walks PF_RL (PF_RL8
// for the eight-stage kernel) row blocks, the weight ring running on across
// them; otherwise one row block per workgroup.
#ifndef PF_WLOAD
#define PF_WLOAD fm_ldg_u4_nt  // weight pieces: streamed once per chunk
#endif
#ifndef PF_RL
#define PF_RL 8
#endif
#ifndef PF_RING8
#define PF_RING8 2  // weight ring depth of the eight-stage (gate/up) kernel
#endif
#ifndef PF_RL8
#define PF_RL8 4    // row blocks of a workgroup holding eight stages (8 waves: 512 rows of 1024)
#endif
__host__ __device__ constexpr int pf_row_tiles(bool res, int nst) { return res ? (nst == 8 ? PF_RL8 : PF_RL) : 1; }
// weight ring depth (pieces in flight per wave); the resident kernels' step
// counts (pieces x row tiles) are multiples of it
__host__ __device__ constexpr int pf_ring(int nst) { return nst == 8 ? PF_RING8 : PF_RING; }
static_assert(PF_RL % PF_RING == 0 && PF_RL8 % PF_RING8 == 0, "a resident workgroup's steps fill whole ring turns");

// DUAL: the workgroup computes the same rows of two matrices (gate and up)
// from one token stage, so the chunk's operands stream once for both.
// RES: the whole input fits the stages (operands resident); else streamed.
template <int BITS, bool LO, bool VEC, bool DUAL, int NST, int W, bool RES, typename Emit>
__device__ void pf_block(const PfArgs &a, const PfMat &mat, const PfMat &mat2, int rb, int rl, const int *srow,
                         PfStage<LO> (&st)[NST], uint32_t *T, Emit emit) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, n = lane & 15, kq = lane >> 4;
    const uint32_t G = a.in_dim / 64;
    constexpr int WPG = 2 * BITS;     // words per group
    constexpr int PW = PF_GPP * WPG;  // words per piece row (64 | 32)
    constexpr int NL = PW / 16;       // loads per piece (4 | 2)
    constexpr int RS = BITS == 4 ? 4 : 8;  // rows between a lane's loads
    const uint32_t wpr = G * WPG;
    const int np = (int)((G + PF_GPP - 1) / PF_GPP);
    const int nq = np * rl;  // (row tile, piece) steps
    const fm_h2 *xop = a.xop[BITS == 4 ? 0 : 1];
    const fm_h2 *xlo = a.xlo[BITS == 4 ? 0 : 1];
    const int lrow = BITS == 4 ? kq : (lane >> 3);
    const int lw = BITS == 4 ? 4 * n : 4 * (lane & 7);
    const int last_row = (int)a.out_dim - 1;
    // step q: piece q % np of row tile q / np (past the end: re-read the last step, no branch)
    auto load_piece = [&](const PfMat &mat, int q, PfPiece<BITS> &d) {
        const int qc = min(q, nq - 1);
        const int rt = qc / np, pc = qc - rt * np;
        const int r0 = rb + 16 * W * rt + 16 * wv;
        const uint32_t w = min((uint32_t)(PW * pc + lw), wpr - 4);
#pragma unroll
        for (int j = 0; j < NL; j++) d.c[j] = PF_WLOAD(mat.w + (size_t)min(r0 + RS * j + lrow, last_row) * wpr + w);
        const size_t so = (size_t)min(r0 + n, last_row) * G;  // this lane's fold row
        const uint32_t g0 = PF_GPP * pc;
        if constexpr (VEC) {  // G % PF_GPP == 0: the piece's 8 scales are one 16-byte run
            d.s = *(const FM_GLOBAL fm_u4 *)(mat.s + so + g0);
            d.b = *(const FM_GLOBAL fm_u4 *)(mat.b + so + g0);
        } else {
            uint32_t ws_[4] = {0u, 0u, 0u, 0u}, wb_[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int gg = 0; gg < PF_GPP; gg++) {
                const uint32_t gi = min(g0 + gg, G - 1);
                const uint32_t vs = fm_ldg_u16(mat.s + so + gi), vb = fm_ldg_u16(mat.b + so + gi);
                ws_[gg >> 1] |= (g0 + gg < G ? vs : 0u) << (16 * (gg & 1));
                wb_[gg >> 1] |= (g0 + gg < G ? vb : 0u) << (16 * (gg & 1));
            }
            d.s = (fm_u4){ws_[0], ws_[1], ws_[2], ws_[3]};
            d.b = (fm_u4){wb_[0], wb_[1], wb_[2], wb_[3]};
        }
    };
    // one piece: transpose this wave's 16 rows through LDS, 2 (4 with LO)
    // MFMAs and one fold per group
    // (4-bit pieces pass in two halves of four groups: half the LDS per wave)
    auto compute = [&](const PfPiece<BITS> &cur, const PfStage<LO> &cs, fm_f4v &acc) {
        const uint32_t sw[4] = {cur.s.x, cur.s.y, cur.s.z, cur.s.w};
        const uint32_t bw[4] = {cur.b.x, cur.b.y, cur.b.z, cur.b.w};
#pragma unroll
        for (int gg = 0; gg < PF_GPP; gg++) {
            if (gg == 0 || (BITS == 4 && gg == PF_GPP / 2)) {
                const int hf = BITS == 4 ? gg / (PF_GPP / 2) : 0;
#pragma unroll
                for (int j = 0; j < NL; j++)
                    if (BITS != 4 || (lw >> 5) == hf) *(fm_u4 *)&T[(RS * j + lrow) * PF_TS + lw - 32 * hf] = cur.c[j];
                __builtin_amdgcn_sched_barrier(0);
            }
            fm_h8 c0, c1;
            if constexpr (BITS == 4) {
                const uint64_t w2 = *(const uint64_t *)&T[n * PF_TS + 8 * (gg % (PF_GPP / 2)) + 2 * kq];
                c0 = pf_codes<4>((uint32_t)w2, 0);
                c1 = pf_codes<4>((uint32_t)(w2 >> 32), 0);
            } else {
                const uint32_t w = T[n * PF_TS + 4 * gg + kq];
                c0 = pf_codes<2>(w, 0);
                c1 = pf_codes<2>(w, 1);
            }
            const fm_h8 x0 = __builtin_bit_cast(fm_h8, *(const fm_u4 *)&cs.xop[0][n][32 * gg + 8 * kq]);
            const fm_h8 x1 = __builtin_bit_cast(fm_h8, *(const fm_u4 *)&cs.xop[0][n][32 * gg + 8 * kq + 4]);
            fm_f4v d = {0.f, 0.f, 0.f, 0.f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, c0, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, c1, d, 0, 0, 0);
            if constexpr (LO) {
                const fm_h8 l0 = __builtin_bit_cast(fm_h8, *(const fm_u4 *)&cs.xop[LO ? 1 : 0][n][32 * gg + 8 * kq]);
                const fm_h8 l1 = __builtin_bit_cast(fm_h8, *(const fm_u4 *)&cs.xop[LO ? 1 : 0][n][32 * gg + 8 * kq + 4]);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(l0, c0, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(l1, c1, d, 0, 0, 0);
            }
            const fm_f4 xs = *(const fm_f4 *)&cs.xsum[gg][4 * kq];
            const float sc = fm_bf16_to_f32((uint16_t)(sw[gg >> 1] >> (16 * (gg & 1))));
            const float bi = fm_bf16_to_f32((uint16_t)(bw[gg >> 1] >> (16 * (gg & 1))));
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] = __builtin_fmaf(sc, d[v], __builtin_fmaf(bi, xs[v], acc[v]));
            if (gg & 1) __builtin_amdgcn_sched_barrier(0);  // bound the read-ahead (registers)
        }
    };
    // DUAL: the gate and up pieces of the same rows together -- each group's
    // codes of both matrices come out of the transpose buffer first (raw
    // words), then the group's operands and sums are read from the stage once
    // for the four MFMAs and two folds
    auto compute2 = [&](const PfPiece<BITS> &cg, const PfPiece<BITS> &cu, const PfStage<LO> &cs, fm_f4v &acc,
                        fm_f4v &acc2) {
        constexpr int HG = BITS == 4 ? PF_GPP / 2 : PF_GPP;  // groups per transpose pass
        const uint32_t sg[4] = {cg.s.x, cg.s.y, cg.s.z, cg.s.w}, bg[4] = {cg.b.x, cg.b.y, cg.b.z, cg.b.w};
        const uint32_t su[4] = {cu.s.x, cu.s.y, cu.s.z, cu.s.w}, bu[4] = {cu.b.x, cu.b.y, cu.b.z, cu.b.w};
#pragma unroll
        for (int hf = 0; hf < PF_GPP / HG; hf++) {
            uint64_t rg[HG], ru[HG];  // 4-bit: two words per group; 2-bit: one
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const PfPiece<BITS> &cur = m == 0 ? cg : cu;
#pragma unroll
                for (int j = 0; j < NL; j++)
                    if (BITS != 4 || (lw >> 5) == hf) *(fm_u4 *)&T[(RS * j + lrow) * PF_TS + lw - 32 * hf] = cur.c[j];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int k = 0; k < HG; k++) {
                    uint64_t w;
                    if constexpr (BITS == 4)
                        w = *(const uint64_t *)&T[n * PF_TS + 8 * k + 2 * kq];
                    else
                        w = T[n * PF_TS + 4 * k + kq];
                    (m == 0 ? rg : ru)[k] = w;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int k = 0; k < HG; k++) {
                const int gg = HG * hf + k;
                fm_h8 g0, g1, u0, u1;
                if constexpr (BITS == 4) {
                    g0 = pf_codes<4>((uint32_t)rg[k], 0);
                    g1 = pf_codes<4>((uint32_t)(rg[k] >> 32), 0);
                    u0 = pf_codes<4>((uint32_t)ru[k], 0);
                    u1 = pf_codes<4>((uint32_t)(ru[k] >> 32), 0);
                } else {
                    g0 = pf_codes<2>((uint32_t)rg[k], 0);
                    g1 = pf_codes<2>((uint32_t)rg[k], 1);
                    u0 = pf_codes<2>((uint32_t)ru[k], 0);
                    u1 = pf_codes<2>((uint32_t)ru[k], 1);
                }
                const float scg = fm_bf16_to_f32((uint16_t)(sg[gg >> 1] >> (16 * (gg & 1))));
                const float big = fm_bf16_to_f32((uint16_t)(bg[gg >> 1] >> (16 * (gg & 1))));
                const float scu = fm_bf16_to_f32((uint16_t)(su[gg >> 1] >> (16 * (gg & 1))));
                const float biu = fm_bf16_to_f32((uint16_t)(bu[gg >> 1] >> (16 * (gg & 1))));
                const fm_h8 x0 = __builtin_bit_cast(fm_h8, *(const fm_u4 *)&cs.xop[0][n][32 * gg + 8 * kq]);
                const fm_h8 x1 = __builtin_bit_cast(fm_h8, *(const fm_u4 *)&cs.xop[0][n][32 * gg + 8 * kq + 4]);
                fm_f4v dg = {0.f, 0.f, 0.f, 0.f}, du = dg;
                dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, g0, dg, 0, 0, 0);
                du = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, u0, du, 0, 0, 0);
                dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, g1, dg, 0, 0, 0);
                du = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, u1, du, 0, 0, 0);
                const fm_f4 xs = *(const fm_f4 *)&cs.xsum[gg][4 * kq];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    acc[v] = __builtin_fmaf(scg, dg[v], __builtin_fmaf(big, xs[v], acc[v]));
                    acc2[v] = __builtin_fmaf(scu, du[v], __builtin_fmaf(biu, xs[v], acc2[v]));
                }
                if (k & 1) __builtin_amdgcn_sched_barrier(0);  // bound the read-ahead (registers)
            }
        }
    };
    // Ring of R pieces with static slots: the step loop is unrolled by R, so
    // no register ever moves between slots (a move would wait for the slot's
    // loads) and every step issues the same loads -- the in-order wait counts
    // stay exact and R - 1 pieces stay in flight while one is computed.
    constexpr int R = pf_ring(NST);
    PfPiece<BITS> ring[R], ring2[DUAL ? R : 1];
    if constexpr (RES) {
        // resident operands: the stages hold the whole input, loaded once
        // (before the weights: piece 0 needs them as early as its weights).
        // Outputs are stored after the step loop: gfx9 counts loads and
        // stores in one counter, and a store pending anywhere in the loop
        // turns every wait for a weight piece into a full drain (vmcnt(0))
        // instead of "all but the younger ring slots".  Finished row tiles
        // wait in a register bank.
        constexpr int RT = pf_row_tiles(true, NST);
        fm_f4v acc = (fm_f4v){0.f, 0.f, 0.f, 0.f}, acc2 = acc, bank[RT], bank2[DUAL ? RT : 1];
#pragma unroll
        for (int j = 0; j < RT; j++) bank[j] = acc;
#pragma unroll
        for (int j = 0; j < (DUAL ? RT : 1); j++) bank2[j] = acc;
        PfStageRegs<LO, W> sr[NST];
#pragma unroll
        for (int k = 0; k < NST; k++)
            if (k < np) pf_stage_load<LO, W>(a, srow, xop, xlo, (uint32_t)k * PF_GPP, sr[k]);
#pragma unroll
        for (int k = 0; k < R; k++) {
            load_piece(mat, k, ring[k]);
            if constexpr (DUAL) load_piece(mat2, k, ring2[k]);
        }
#pragma unroll
        for (int k = 0; k < NST; k++)
            if (k < np) pf_stage_store<LO, W>(st[k], sr[k]);
        __syncthreads();
        FM_PF_MARK(1);
        // nq is a multiple of R (the launch guarantees it): no step is
        // conditional, so every path through the loop has the same loads in
        // flight and each wait leaves the younger ring slots outstanding
        for (int q0 = 0; q0 < nq; q0 += R) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int q = q0 + i;
                __builtin_amdgcn_sched_barrier(0);  // keep the unrolled steps apart (registers)
                const int rt = q / np, pc = q - rt * np;
                if constexpr (DUAL) {
                    compute2(ring[i], ring2[i], st[pc], acc, acc2);
                    load_piece(mat, q + R, ring[i]);
                    load_piece(mat2, q + R, ring2[i]);
                } else {
                    compute(ring[i], st[pc], acc);
                    load_piece(mat, q + R, ring[i]);
                }
                if (pc == np - 1) {  // row tile rt done: into the bank (tile k ends at RT - rl + k)
#pragma unroll
                    for (int j = 0; j + 1 < RT; j++) {
                        bank[j] = bank[j + 1];
                        if constexpr (DUAL) bank2[j] = bank2[j + 1];
                    }
                    bank[RT - 1] = acc;
                    if constexpr (DUAL) bank2[RT - 1] = acc2;
                    acc = acc2 = (fm_f4v){0.f, 0.f, 0.f, 0.f};
                }
            }
        }
#pragma unroll
        for (int j = 0; j < RT; j++)
            if (j >= RT - rl) emit(j - (RT - rl), bank[j], DUAL ? bank2[j] : bank[j]);
    } else {
        static_assert(NST == 2 && !DUAL, "streamed operands: two stages, one matrix");
        // streamed operands: piece p + 1's stage registers go to LDS while
        // piece p + 2's are already loading; one barrier per piece
        fm_f4v acc = (fm_f4v){0.f, 0.f, 0.f, 0.f};
        PfStageRegs<LO, W> sr[2];
        pf_stage_load<LO, W>(a, srow, xop, xlo, 0, sr[0]);
#pragma unroll
        for (int k = 0; k < R; k++) load_piece(mat, k, ring[k]);
        pf_stage_load<LO, W>(a, srow, xop, xlo, (uint32_t)min(1, np - 1) * PF_GPP, sr[1]);
        pf_stage_store<LO, W>(st[0], sr[0]);
        __syncthreads();
        FM_PF_MARK(1);
        for (int p0 = 0; p0 < np; p0 += R) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int p = p0 + i;
                __builtin_amdgcn_sched_barrier(0);  // keep the unrolled steps apart (registers)
                if (p < np) {
                    pf_stage_load<LO, W>(a, srow, xop, xlo, (uint32_t)min(p + 2, np - 1) * PF_GPP, sr[i & 1]);
                    compute(ring[i], st[i & 1], acc);
                    if (p == 0) FM_PF_MARK(2);
                    load_piece(mat, p + R, ring[i]);
                    if (p + 1 < np) pf_stage_store<LO, W>(st[(i + 1) & 1], sr[(i + 1) & 1]);
                    __syncthreads();
                }
            }
        }
        emit(0, acc, acc);
    }
    FM_PF_MARK(3);
}

// grid: one block per (chunk, matrix, row block) unit of max_chunks chunks;
// units are consecutive chunks first, so the blocks that read the same
// weights for consecutive chunks run side by side
// W waves per workgroup (16 rows each): 4 for the two-stage kernels (three
// workgroups per CU when resident), 8 for the eight-stage gate/up kernel (one
// per CU).  RES / VEC select one operand path and one scale-load path at
// compile time, so the registers are sized for the path the launch takes.
template <bool LO, bool DUAL, int NST, int W, bool RES, bool VEC>
__global__ __launch_bounds__(64 * W, NST == 8 ? 1 : (LO || !RES ? 2 : PF_MINB)) void fm_pf_gemm_kernel(PfArgs a) {
    __shared__ PfStage<LO> st[NST];
    __shared__ uint32_t tbuf[W][16 * PF_TS];
    __shared__ int srow_s[PF_TOK], slot_s[PF_TOK];
    __shared__ float tinv_s[PF_TOK];  // each token column's 2^(24 - e)
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    FM_PF_MARK(5);
    // Units are (chunk, matrix, row block) over the LIVE chunks only (the grid is
    // sized for max_chunks; surplus blocks exit).  XCD-aware order: the 8 XCDs
    // take blocks round-robin, so XCD x gets the contiguous eighth x of the
    // units -- equal work per XCD, and the chunks of one expert (consecutive
    // units) share that XCD's L2 instead of fetching the weights once per XCD.
    // mode 0 without DUAL: gate and up rows are separate units (matrix = mat)
    const uint32_t nmat = (a.mode == 0 && !DUAL) ? 2 : 1;
    const int rl_big = pf_row_tiles(RES, NST);
    const uint32_t rows_per_wg = 16 * W * rl_big;
    const uint32_t nrb = (a.out_dim + rows_per_wg - 1) / rows_per_wg;
    const uint32_t nch = (uint32_t)*a.nchunks;
    const uint32_t live = nch * nmat * nrb, per_xcd = (live + 7) / 8;
    // Eight-stage kernel (one workgroup per CU, long units): the units of an
    // XCD's last partial round run as single row tiles, so that round ends
    // after about one row tile instead of one whole unit (the grid has room
    // for the extra workgroups; the others exit).  Single row tiles need a
    // piece count that fills whole ring turns.
    const uint32_t np = (a.in_dim / 64 + PF_GPP - 1) / PF_GPP;
    const uint32_t full =
        (NST == 8 && rl_big > 1 && np % pf_ring(NST) == 0) ? per_xcd / a.xcd_slots * a.xcd_slots : per_xcd;
    const uint32_t nsplit = (per_xcd - full) * (uint32_t)rl_big;
    const uint32_t lb = blockIdx.x / 8;
    uint32_t u, tile0 = 0;
    int rl = rl_big;
    if (lb < full) {
        u = (blockIdx.x % 8) * per_xcd + lb;
    } else if (lb < full + nsplit) {
        u = (blockIdx.x % 8) * per_xcd + full + (lb - full) / rl_big;
        tile0 = (lb - full) % rl_big;
        rl = 1;
    } else {
        return;
    }
    if (u >= live) return;
    const uint32_t ci = u % nch, rest = u / nch;
    const uint32_t mat = rest % nmat, rbk = rest / nmat;
    FM_PF_MARK(0);
    // one 128-byte chunk row holds everything this workgroup needs
    const int *ch = a.chunks + (size_t)PF_CROW * ci;
    const int e = ch[0], off = ch[1], n = ch[2], cbits = ch[3];
    const char *blob = (const char *)(((uint64_t)(uint32_t)ch[5] << 32) | (uint32_t)ch[4]);
    if (threadIdx.x < PF_TOK) {
        const int ei = threadIdx.x;
        const int sl = ei < n ? ch[16 + ei] : -1;  // ids past the count are not written
        const int sr = sl < 0 ? -1 : (a.mode == 1 ? off + ei : (a.mode == 2 ? sl : pf_token_of_slot(a, sl)));
        slot_s[ei] = sl;
        srow_s[ei] = sr;
        tinv_s[ei] = sr < 0 ? 0.f : a.xinv[sr];
    }
    __syncthreads();
    FM_PF_MARK(6);
    int bits = 4;
    // mode 0: gate (matrix 0) and up (matrix 1) rows together
    const PfMat m = pf_mat(a, e, a.mode == 0 ? (int)mat : (a.mode == 1 ? 2 : 0), blob, cbits, bits);
    const PfMat m2 = DUAL ? pf_mat(a, e, 1, blob, cbits, bits) : m;
    const int rb = (int)(rbk * rows_per_wg + tile0 * 16 * W);
    uint32_t *T = tbuf[wv];
    // lane (row n, q) holds tokens 4q .. 4q+3 of row rb + 16 W rt + 16 wv + n
    auto emit = [&](int rt, const fm_f4v &acc, const fm_f4v &acc2) {
        const int row = rb + 16 * W * rt + 16 * wv + (lane & 15), q = lane >> 4;
        if (row >= (int)a.out_dim) return;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int tk = 4 * q + v;
            if (tk >= n) continue;
            const float ti = tinv_s[tk];
            if constexpr (DUAL) {  // SwiGLU in the epilogue: gout receives the activation
                a.gout[(size_t)(off + tk) * a.out_dim + row] = fm_silu_mul(acc[v] * ti, acc2[v] * ti);
            } else if (a.mode == 0) {
                (mat == 0 ? a.gout : a.uout)[(size_t)(off + tk) * a.out_dim + row] = acc[v] * ti;
            } else {
                a.y[(size_t)slot_s[tk] * a.out_dim + row] = acc[v] * ti;
            }
        }
    };
    // VEC: the scales of a piece are one 16-byte run (in_dim a multiple of 512;
    // DUAL kernels are only launched then)
    if (bits == 4)
        pf_block<4, LO, VEC, DUAL, NST, W, RES>(a, m, m2, rb, rl, srow_s, st, T, emit);
    else
        pf_block<2, LO, VEC, DUAL, NST, W, RES>(a, m, m2, rb, rl, srow_s, st, T, emit);
    FM_PF_MARK(4);
}

// ---------------------------------------------------------------- lists ----
// Single block: count tokens per expert, scan, scatter entries, cut chunks.
// Entry order inside an expert is irrelevant to the result (each token column
// is computed independently), so LDS atomics are fine.
// Chunk row (PF_CROW ints, one 128-byte line): [0] expert, [1] entry offset,
// [2] entry count, [3] bit width, [4..5] blob address (pool experts), [16..31]
// the chunk's slot ids (-1 past the count) -- everything a GEMM workgroup
// needs in ONE dependent load.
__global__ __launch_bounds__(1024) void fm_pf_lists_kernel(const int *idx, int T, int K, int E, int has_shared,
                                                           const void *const *blobs, const uint8_t *bits_table,
                                                           int sh_bits, int *chunks, int *nchunks,
                                                           uint32_t max_chunks, int *err, int tstage) {
    extern __shared__ int sm[];
    int *cnt = sm;               // [E + 1]
    int *base = sm + (E + 1);    // [E + 2]
    int *cbase = base + (E + 2); // [E + 2]
    int *tbits = cbase + (E + 2);  // [E + 1] bit widths
    uint64_t *tblob = (uint64_t *)(((uintptr_t)(tbits + E + 1) + 7) & ~(uintptr_t)7);  // [E] blob addresses
    __shared__ int wsum[2][16];
    FM_PL_MARK(0);
    const int NE = E + (has_shared ? 1 : 0);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // the pool table entries the chunk rows need, loaded now (they arrive
    // while the entries are counted) and staged in LDS before the scan; the
    // host sets tstage when E <= 4096 and the extra LDS fits
    constexpr int PF_LT = 4;  // entries per thread
    uint64_t pbl[PF_LT];
    int pbt[PF_LT];
#pragma unroll
    for (int j = 0; j < PF_LT; j++) {
        const int e = tid + 1024 * j;
        pbl[j] = tstage && e < E ? (uint64_t)(uintptr_t)blobs[e] : 0ull;
        pbt[j] = tstage && e < E ? (int)bits_table[e] : 0;
    }
    for (int i = tid; i <= E; i += blockDim.x) cnt[i] = 0;
    __syncthreads();
    FM_PL_MARK(1);
    const int n = T * K;
    // up to PF_LQ entries per thread keep their expert and their place in its
    // list (the count's atomic result) in registers for the scatter below
    constexpr int PF_LQ = 16;
    const bool inreg = n <= PF_LQ * 1024;
    int le[PF_LQ], lp[PF_LQ];
#pragma unroll
    for (int j = 0; j < PF_LQ; j++) {
        const int i = tid + 1024 * j;
        le[j] = -1;
        lp[j] = 0;
        if (inreg && i < n) le[j] = idx[i];
    }
    if (inreg) {
#pragma unroll
        for (int j = 0; j < PF_LQ; j++) {
            const int e = le[j];
            if (tid + 1024 * j >= n) continue;
            if (e < 0 || e >= E) {
                atomicOr(err, FM_STATUS_BAD_EXPERT);
                le[j] = -1;
                continue;
            }
            lp[j] = atomicAdd(&cnt[e], 1);
        }
    } else {
        for (int i = tid; i < n; i += blockDim.x) {
            int e = idx[i];
            if (e < 0 || e >= E) {
                atomicOr(err, FM_STATUS_BAD_EXPERT);
                continue;
            }
            atomicAdd(&cnt[e], 1);
        }
    }
    if (has_shared && tid == 0) cnt[E] = T;
    __syncthreads();
    FM_PL_MARK(2);
#pragma unroll
    for (int j = 0; j < PF_LT; j++) {
        const int e = tid + 1024 * j;
        if (tstage && e < E) {
            tblob[e] = pbl[j];
            tbits[e] = pbt[j];
        }
    }
    // exclusive scans of entries and chunks over experts: thread t owns the
    // run of PER consecutive experts starting at t * PER
    {
        const int PER = (NE + 1023) / 1024;
        int se = 0, sc = 0;
        for (int k = 0; k < PER; k++) {
            const int e = tid * PER + k;
            if (e < NE) {
                se += cnt[e];
                sc += (cnt[e] + PF_CHUNK - 1) / PF_CHUNK;
            }
        }
        int ie = se, ic = sc;  // inclusive wave scans
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int oe = __shfl_up(ie, d, 64), oc = __shfl_up(ic, d, 64);
            if (lane >= d) {
                ie += oe;
                ic += oc;
            }
        }
        if (lane == 63) {
            wsum[0][wv] = ie;
            wsum[1][wv] = ic;
        }
        __syncthreads();
    FM_PL_MARK(3);
        int pe = 0, pc = 0;
        for (int w = 0; w < wv; w++) {
            pe += wsum[0][w];
            pc += wsum[1][w];
        }
        int ae = pe + ie - se, ac = pc + ic - sc;
        for (int k = 0; k < PER; k++) {
            const int e = tid * PER + k;
            if (e < NE) {
                base[e] = ae;
                cbase[e] = ac;
                ae += cnt[e];
                ac += (cnt[e] + PF_CHUNK - 1) / PF_CHUNK;
            }
        }
        if (tid == 1023) {
            base[NE] = ae;
            cbase[NE] = ac;
            *nchunks = ac <= (int)max_chunks ? ac : (int)max_chunks;
            if (ac > (int)max_chunks) atomicOr(err, FM_STATUS_CHUNKS);
        }
    }
    __syncthreads();
    FM_PL_MARK(4);
    // chunk rows: the header (the scatter fills the live slot ids; the GEMMs
    // read none past the count), one thread per chunk; its expert is the last
    // e with cbase[e] <= chunk
    {
        const int nc = min(cbase[NE], (int)max_chunks);
        for (int ci = tid; ci < nc; ci += blockDim.x) {
            int lo = 0, hi = NE;  // cbase[lo] <= ci < cbase[hi]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (cbase[mid] <= ci)
                    lo = mid;
                else
                    hi = mid;
            }
            const int e = lo, j = ci - cbase[e], ne = cnt[e];
            const uint64_t blob = e < E ? (tstage ? tblob[e] : (uint64_t)(uintptr_t)blobs[e]) : 0ull;
            int *row = chunks + (size_t)PF_CROW * ci;
            const int nn = min(PF_CHUNK, ne - j * PF_CHUNK);
            row[0] = e;
            row[1] = base[e] + j * PF_CHUNK;
            row[2] = nn;
            row[3] = e < E ? (tstage ? tbits[e] : (int)bits_table[e]) : sh_bits;
            row[4] = (int)(uint32_t)blob;
            row[5] = (int)(uint32_t)(blob >> 32);
        }
    }
    // scatter the entries (slot id t*K + k) into the chunk rows
    __syncthreads();
    FM_PL_MARK(5);
    if (inreg) {
#pragma unroll
        for (int j = 0; j < PF_LQ; j++) {
            const int e = le[j], p = lp[j], i = tid + 1024 * j;
            if (e < 0) continue;
            const int ci = cbase[e] + p / PF_CHUNK;
            if (ci < (int)max_chunks) chunks[(size_t)PF_CROW * ci + 16 + p % PF_CHUNK] = i;
        }
    } else {
        // cnt becomes a running cursor
        for (int i = tid; i <= E; i += blockDim.x) cnt[i] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += blockDim.x) {
            const int e = idx[i];
            if (e < 0 || e >= E) continue;
            const int p = atomicAdd(&cnt[e], 1);
            const int ci = cbase[e] + p / PF_CHUNK;
            if (ci < (int)max_chunks) chunks[(size_t)PF_CROW * ci + 16 + p % PF_CHUNK] = i;
        }
    }
    if (has_shared)
        for (int t = tid; t < T; t += blockDim.x) {
            const int ci = cbase[E] + t / PF_CHUNK;
            if (ci < (int)max_chunks) chunks[(size_t)PF_CROW * ci + 16 + t % PF_CHUNK] = T * K + t;
        }
    FM_PL_MARK(9);
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

// The same combine, four consecutive elements a thread (16-byte loads and
// stores; every slot's row issued before the sums, which run in slot order as
// above).  Needs hidden % 4 == 0 and 16-byte aligned y / h_mid / out.
__global__ __launch_bounds__(256) void fm_pf_combine4_kernel(const float *y, const float *w, int T, int K, int H,
                                                             int has_shared, const float *g, const float *h_mid,
                                                             float *out, uint16_t *out_bf16) {
    const int t = blockIdx.y;
    const int i = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= H || t >= T) return;
    fm_f4 yk[FM_MAX_K + 1];
#pragma unroll
    for (int k = 0; k < FM_MAX_K; k++)
        if (k < K) yk[k] = fm_ldg_f4(y + (size_t)(t * K + k) * H + i);
    if (has_shared) yk[FM_MAX_K] = fm_ldg_f4(y + (size_t)(T * K + t) * H + i);
    float m[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < FM_MAX_K; k++) {
        if (k < K) {
            const float wk = w[t * K + k];
            m[0] = __fadd_rn(m[0], __fmul_rn(wk, yk[k].x));
            m[1] = __fadd_rn(m[1], __fmul_rn(wk, yk[k].y));
            m[2] = __fadd_rn(m[2], __fmul_rn(wk, yk[k].z));
            m[3] = __fadd_rn(m[3], __fmul_rn(wk, yk[k].w));
        }
    }
    float v[4] = {m[0], m[1], m[2], m[3]};
    if (h_mid) {
        const fm_f4 hm = fm_ldg_f4(h_mid + (size_t)t * H + i);
        v[0] = __fadd_rn(hm.x, m[0]);
        v[1] = __fadd_rn(hm.y, m[1]);
        v[2] = __fadd_rn(hm.z, m[2]);
        v[3] = __fadd_rn(hm.w, m[3]);
    }
    if (has_shared) {
        const float sw = g ? fm_sigmoid(g[t]) : 1.0f;
        const float ys[4] = {yk[FM_MAX_K].x, yk[FM_MAX_K].y, yk[FM_MAX_K].z, yk[FM_MAX_K].w};
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = __fadd_rn(v[j], __fmul_rn(sw, ys[j]));
    }
    *(fm_f4 *)(out + (size_t)t * H + i) = (fm_f4){v[0], v[1], v[2], v[3]};
    if (out_bf16) {
        const uint32_t lo = (uint32_t)fm_f32_to_bf16(v[0]) | ((uint32_t)fm_f32_to_bf16(v[1]) << 16);
        const uint32_t hi = (uint32_t)fm_f32_to_bf16(v[2]) | ((uint32_t)fm_f32_to_bf16(v[3]) << 16);
        *(uint2 *)(out_bf16 + (size_t)t * H + i) = make_uint2(lo, hi);
    }
}

// SwiGLU of the apart shared expert's gate and up rows, in place into g.
__global__ __launch_bounds__(256) void fm_pf_swiglu_kernel(float *g, const float *u, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) g[i] = fm_silu_mul(g[i], u[i]);
}

// ---------------------------------------------------------------- host -----
static uint32_t pf_max_chunks(int T, int K, uint32_t E, int has_shared) {
    // sum_e ceil(n_e / 64) <= min(E, T*K) + T*K / 64, plus the shared expert
    uint32_t n = (uint32_t)T * K;
    uint32_t m = (n < E ? n : E) + n / PF_CHUNK + 1;
    if (has_shared) m += (T + PF_CHUNK - 1) / PF_CHUNK;
    return m;
}

// B-operand block for `rows` source rows of in_dim inputs: pairs in both code
// layouts (+ residual terms when lo), group sums.
struct PfOps {
    size_t x4, x2, l4, l2, sum, inv, total;
};

static PfOps pf_ops_layout(size_t rows, uint32_t in_dim, bool lo, size_t o) {
    PfOps P;
    const size_t pairs = rows * (in_dim / 64) * 32 * sizeof(fm_h2);
    P.x4 = o;
    o += fm_align_up(pairs, 256);
    P.x2 = o;
    o += fm_align_up(pairs, 256);
    P.l4 = lo ? o : 0;
    if (lo) o += fm_align_up(pairs, 256);
    P.l2 = lo ? o : 0;
    if (lo) o += fm_align_up(pairs, 256);
    P.sum = o;
    o += fm_align_up(rows * (in_dim / 64) * sizeof(float), 256);
    P.inv = o;
    o += fm_align_up(rows * sizeof(float), 256);
    P.total = o;
    return P;
}

struct PfLayout {
    size_t chunks, nchunks, err, gout, uout, y, total;
    PfOps xo, ao;
    size_t sh_ws, sh_ws_bytes, sh_g, sh_u;  // shared expert of its own intermediate size (sh_ws_bytes > 0)
};

// A shared expert whose intermediate size differs from the routed experts'
// (config.h:23 shared_intermediate) runs apart, as three plain dequant GEMMs
// over all tokens (as pfb_batched_shared_expert does, batched_prefill.h:122-226).
static bool pf_shared_apart(int has_shared, uint32_t inter, uint32_t shared_inter) {
    return has_shared && shared_inter != 0 && shared_inter != inter;
}

static PfLayout pf_layout(int T, int K, uint32_t E, uint32_t hidden, uint32_t inter, int has_shared,
                          uint32_t shared_inter = 0) {
    PfLayout L;
    const size_t nent = (size_t)T * K + (has_shared ? T : 0);
    const uint32_t mc = pf_max_chunks(T, K, E, has_shared);
    size_t o = 0;
    L.err = o;  // header first: status word (fm_workspace_status), decode epoch
    // the decode kernels' tagged region for the few-token paths (T <= 8): kept
    // apart from the GEMM arrays below, so it only ever holds tagged words
    o = fm_moe_decode_workspace_size(FM_PREFILL_DECODE_MAX_T * (FM_MAX_K + 1), hidden, inter);
    L.chunks = o;
    o += fm_align_up((size_t)mc * PF_CROW * 4, 256);
    L.nchunks = o;
    o += 256;
    L.gout = o;
    o += fm_align_up(nent * inter * 4, 256);
    L.uout = o;
    o += fm_align_up(nent * inter * 4, 256);
    L.y = o;
    o += fm_align_up(nent * hidden * 4, 256);
    L.xo = pf_ops_layout((size_t)T, hidden, false, o);
    o = L.xo.total;
    L.ao = pf_ops_layout(nent, inter, false, o);
    o = L.ao.total;
    L.sh_ws = L.sh_ws_bytes = L.sh_g = L.sh_u = 0;
    if (pf_shared_apart(has_shared, inter, shared_inter)) {
        L.sh_ws = o;
        L.sh_ws_bytes = fm_align_up(fm_pfb_gemm_workspace_size((uint32_t)T, hidden > shared_inter ? hidden : shared_inter), 256);
        o += L.sh_ws_bytes;
        L.sh_g = o;
        o += fm_align_up((size_t)T * shared_inter * 4, 256);
        L.sh_u = o;
        o += fm_align_up((size_t)T * shared_inter * 4, 256);
    }
    L.total = o;
    return L;
}

extern "C" size_t fm_prefill_moe_workspace_size(int T, int K, const fm_expert_pool *pool, uint32_t shared_inter) {
    if (!pool || T <= 0 || K <= 0) return 0;
    return pf_layout(T, K, pool->num_experts, pool->hidden, pool->inter, 1, shared_inter).total;
}

static int pf_launch_ops(const float *src, const float *src2, const int *nrows_dev, int nrows_max, uint32_t in_dim,
                         char *base, const PfOps &P, bool lo, hipStream_t st) {
    fm_h2 *x4 = (fm_h2 *)(base + P.x4), *x2 = (fm_h2 *)(base + P.x2);
    fm_h2 *l4 = lo ? (fm_h2 *)(base + P.l4) : nullptr, *l2 = lo ? (fm_h2 *)(base + P.l2) : nullptr;
    float *sum = (float *)(base + P.sum), *inv = (float *)(base + P.inv);
    const uint32_t tpr = in_dim / 16;
#define PF_XOP1(TPR)                                                                                             \
    if (tpr == TPR) {                                                                                            \
        hipLaunchKernelGGL(fm_pf_xop1_kernel<TPR>, dim3((unsigned)((nrows_max + 256 / TPR - 1) / (256 / TPR))), \
                           dim3(256), 0, st, src, src2, nrows_dev, nrows_max, in_dim, x4, x2, l4, l2, sum, inv); \
        return fm_check_launch("fm_pf_xop1_kernel");                                                             \
    }
    PF_XOP1(256) PF_XOP1(128) PF_XOP1(64) PF_XOP1(32) PF_XOP1(16) PF_XOP1(8) PF_XOP1(4)
#undef PF_XOP1
    hipLaunchKernelGGL(fm_pf_xop_kernel, dim3((unsigned)nrows_max), dim3(256), 0, st, src, src2, nrows_dev,
                       nrows_max, in_dim, x4, x2, l4, l2, sum, inv);
    return fm_check_launch("fm_pf_xop_kernel");
}

static void pf_bind_ops(PfArgs &a, char *base, const PfOps &P, bool lo) {
    a.xop[0] = (const fm_h2 *)(base + P.x4);
    a.xop[1] = (const fm_h2 *)(base + P.x2);
    a.xlo[0] = lo ? (const fm_h2 *)(base + P.l4) : nullptr;
    a.xlo[1] = lo ? (const fm_h2 *)(base + P.l2) : nullptr;
    a.xsum = (const float *)(base + P.sum);
    a.xinv = (const float *)(base + P.inv);
}

// Gate and up rows in one workgroup with the whole input resident (eight
// stages, one workgroup per CU) when a piece's scales are one 16-byte run; that
// kernel applies SwiGLU itself (gout receives the activations, uout unused).
static bool pf_dual(uint32_t in_dim) {
    const uint32_t G = in_dim / 64;
    return G % PF_GPP == 0 && (G + PF_GPP - 1) / PF_GPP <= 8;
}

static int pf_launch_gemm(PfArgs &a, bool lo, hipStream_t st) {
    const uint32_t G = a.in_dim / 64;
    const uint32_t np = (G + PF_GPP - 1) / PF_GPP;
    const bool dual = !lo && a.mode == 0 && pf_dual(a.in_dim);
    const int nst = dual ? 8 : 2;
    const int W = dual ? 8 : 4;
    const bool res = dual || np <= 2;  // operands resident in the stages
    const uint32_t rows_per_wg = 16 * W * pf_row_tiles(res, nst);
    const uint32_t rowblocks = (a.out_dim + rows_per_wg - 1) / rows_per_wg;
    const uint32_t nmat = (a.mode == 0 && !dual) ? 2 : 1;
    // whole multiple of 8 blocks (the XCD-aware unit order), room for the
    // eight-stage kernel's split last round; extra blocks exit
    const size_t units = (size_t)a.max_chunks * rowblocks * nmat;
    a.xcd_slots = (uint32_t)((fm_num_cus() + 7) / 8);
    const size_t per_xcd = (units + 7) / 8 + (dual ? (size_t)a.xcd_slots * (pf_row_tiles(true, 8) - 1) : 0);
    dim3 grid((unsigned)(per_xcd * 8)), block(64 * W);
    const bool vec = G % PF_GPP == 0;  // a piece's scales are one 16-byte run
#define PF_GO(LO_, R_, V_) hipLaunchKernelGGL((fm_pf_gemm_kernel<LO_, false, 2, 4, R_, V_>), grid, block, 0, st, a)
#define PF_GO4(LO_)                      \
    if (res && vec) PF_GO(LO_, true, true);  \
    else if (res) PF_GO(LO_, true, false);   \
    else if (vec) PF_GO(LO_, false, true);   \
    else PF_GO(LO_, false, false);
    if (lo) {
        PF_GO4(true)
    } else if (dual) {
        hipLaunchKernelGGL((fm_pf_gemm_kernel<false, true, 8, 8, true, true>), grid, block, 0, st, a);
    } else {
        PF_GO4(false)
    }
#undef PF_GO4
#undef PF_GO
    return fm_check_launch("fm_pf_gemm_kernel");
}

extern "C" int fm_prefill_moe(const fm_expert_pool *pool, int T, int K, const int *idx, const float *weights,
                              const fm_expert_weights *shared, int shared_bits, uint32_t shared_inter,
                              const float *shared_gate_scores,
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
    if (shared_inter == pool->inter) shared_inter = 0;
    if (has_shared && shared_inter)
        FM_REQUIRE(shared_inter % 64 == 0 && shared_inter <= 16384, "%s: shared_inter %u", who, shared_inter);
    const bool apart = pf_shared_apart(has_shared, pool->inter, shared_inter);
    PfLayout L = pf_layout(T, K, pool->num_experts, pool->hidden, pool->inter, has_shared, shared_inter);
    if (!ws || ws_bytes < L.total)
        return fm_fail(FM_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu required", who, ws_bytes, L.total);
    // A few tokens (batched decode): fused decode steps stream
    // each token's experts once at decode efficiency; the grouped GEMM only pays
    // off once experts are shared by many tokens.  Same result per token
    // (batched_prefill.h:241-308 is per-token decode arithmetic).
    if (T <= FM_PREFILL_DECODE_MAX_T && K <= FM_MAX_K && !apart) {
        if (T > 1 && fm_moe_decode_tokens_workspace_size(T, K, has_shared, pool->hidden, pool->inter) <= ws_bytes) {
            // all tokens in one decode launch when the kernel takes T x (K + shared) slots
            const int rc = fm_moe_decode_pool_tokens(pool, T, K, idx, weights, shared, shared_bits,
                                                     shared_gate_scores, X, h_mid, out, out_bf16, ws, ws_bytes,
                                                     stream);
            if (rc != FM_ERR_UNSUPPORTED) return rc;
            fm_clear_error();
        }
        const size_t dws = fm_moe_decode_workspace_size(K + has_shared, pool->hidden, pool->inter);
        if (dws <= ws_bytes) {
            for (int t = 0; t < T; t++) {
                const int rc = fm_moe_decode_pool(pool, K, idx + (size_t)t * K, weights + (size_t)t * K, shared,
                                                  shared_bits, 0, shared_gate_scores ? shared_gate_scores + t : nullptr,
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
    if ((uintptr_t)X & 15) return fm_fail(FM_ERR_INVALID, "%s: X not 16-byte aligned", who);
    if ((uintptr_t)ws & 255) return fm_fail(FM_ERR_INVALID, "%s: workspace not 256-byte aligned", who);
    char *p = (char *)ws;
    hipStream_t st = fm_stream(stream);
    // the grouped GEMM takes the shared expert as one more expert unless it runs apart
    const int grouped_shared = apart ? 0 : has_shared;
    const uint32_t mc = pf_max_chunks(T, K, pool->num_experts, grouped_shared);
    const size_t nent = (size_t)T * K + grouped_shared * T;

    // lists
    // (the pool table staged in LDS only where it fits beside the lists)
    size_t lds = ((size_t)pool->num_experts * 3 + 5) * sizeof(int);
    const size_t tab_lds = ((size_t)pool->num_experts + 1) * sizeof(int) + 8 + (size_t)pool->num_experts * 8;
    const int tstage = pool->num_experts <= 4096 && lds + tab_lds <= 65536;
    if (tstage) lds += tab_lds;
    if (lds > 65536) return fm_fail(FM_ERR_UNSUPPORTED, "%s: too many experts", who);
    hipLaunchKernelGGL(fm_pf_lists_kernel, dim3(1), dim3(1024), lds, st, idx, T, K, (int)pool->num_experts,
                       grouped_shared, pool->blobs, pool->bits, shared ? shared_bits : 4,
                       (int *)(p + L.chunks), (int *)(p + L.nchunks), mc, (int *)(p + L.err), tstage);
    int rc = fm_check_launch("fm_pf_lists_kernel");
    if (rc) return rc;
    // token operands of X (fp16, one power-of-two scale per token)
    rc = pf_launch_ops(X, nullptr, nullptr, T, pool->hidden, p, L.xo, false, st);
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
    a.T = T;
    a.K = K;
    a.max_chunks = mc;
    float *gout = (float *)(p + L.gout), *uout = (float *)(p + L.uout);
    float *y = (float *)(p + L.y);

    // gemm1: gate and up rows -> G, U [entry][inter] fp32
    a.mode = 0;
    pf_bind_ops(a, p, L.xo, false);
    a.in_dim = pool->hidden;
    a.out_dim = pool->inter;
    a.gout = gout;
    a.uout = uout;
    rc = pf_launch_gemm(a, false, st);
    if (rc) return rc;
    // act = silu(G) * U as fp16 token operands, then gemm2 (down projection)
    rc = pf_launch_ops(gout, pf_dual(pool->hidden) ? nullptr : uout, nullptr, (int)nent, pool->inter, p, L.ao, false,
                       st);
    if (rc) return rc;
    a.mode = 1;
    pf_bind_ops(a, p, L.ao, false);
    a.in_dim = pool->inter;
    a.out_dim = pool->hidden;
    a.y = y;
    rc = pf_launch_gemm(a, false, st);
    if (rc) return rc;
    if (apart) {
        // shared expert over all tokens: gate, up (X -> [T][shared_inter]), SwiGLU, down into y rows T*K + t
        float *g = (float *)(p + L.sh_g), *u = (float *)(p + L.sh_u);
        void *gw = p + L.sh_ws;
        rc = fm_pfb_gemm(shared->gate_w, shared->gate_s, shared->gate_b, X, g, (uint32_t)T, shared_inter,
                         pool->hidden, 64, shared_bits, gw, L.sh_ws_bytes, stream);
        if (!rc)
            rc = fm_pfb_gemm(shared->up_w, shared->up_s, shared->up_b, X, u, (uint32_t)T, shared_inter,
                             pool->hidden, 64, shared_bits, gw, L.sh_ws_bytes, stream);
        if (rc) return rc;
        const size_t n = (size_t)T * shared_inter;
        hipLaunchKernelGGL(fm_pf_swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, n);
        rc = fm_check_launch("fm_pf_swiglu_kernel");
        if (!rc)
            rc = fm_pfb_gemm(shared->down_w, shared->down_s, shared->down_b, g, y + (size_t)T * K * pool->hidden,
                             (uint32_t)T, pool->hidden, shared_inter, 64, shared_bits, gw, L.sh_ws_bytes, stream);
        if (rc) return rc;
    }
    // combine
    const bool vec4 = pool->hidden % 4 == 0 && K <= FM_MAX_K && !(((uintptr_t)y | (uintptr_t)out) & 15) &&
                      !((uintptr_t)h_mid & 15) && !((uintptr_t)out_bf16 & 7);
    if (vec4) {
        dim3 cg4((pool->hidden / 4 + 255) / 256, T);
        hipLaunchKernelGGL(fm_pf_combine4_kernel, cg4, dim3(256), 0, st, y, weights, T, K, (int)pool->hidden,
                           has_shared, shared_gate_scores, h_mid, out, out_bf16);
        return fm_check_launch("fm_pf_combine4_kernel");
    }
    dim3 cg((pool->hidden + 255) / 256, T);
    hipLaunchKernelGGL(fm_pf_combine_kernel, cg, dim3(256), 0, st, y, weights, T, K, (int)pool->hidden, has_shared,
                       shared_gate_scores, h_mid, out, out_bf16);
    return fm_check_launch("fm_pf_combine_kernel");
}

// ---------------------------------------------------------------- pfb gemm -
// Y[N, out] = X[N, in] dequant(W)^T, X fp32 (fp16 hi + lo terms), one
// "expert" whose entry list is the identity.
__global__ void fm_pfb_lists_kernel(int N, int *chunks, int *nchunks) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int nc = (N + PF_CHUNK - 1) / PF_CHUNK;
    if (i < nc) {
        int *row = chunks + (size_t)PF_CROW * i;
        const int n = min(PF_CHUNK, N - i * PF_CHUNK);
        row[0] = 0;
        row[1] = i * PF_CHUNK;
        row[2] = n;
        row[3] = 0;
        row[4] = row[5] = 0;
        for (int ei = 0; ei < PF_CHUNK; ei++) row[16 + ei] = ei < n ? i * PF_CHUNK + ei : -1;
    }
    if (i == 0) *nchunks = nc;
}

// [256 B left alone: the status word of a layer workspace that shares this
// region][chunk rows][nchunks], then the operands
static size_t pfb_head(uint32_t N) {
    const size_t nc = (N + PF_CHUNK - 1) / PF_CHUNK;
    return 256 + fm_align_up(nc * PF_CROW * 4, 256) + 256;
}

extern "C" size_t fm_pfb_gemm_workspace_size(uint32_t N, uint32_t in_dim) {
    return pf_ops_layout(N, in_dim, true, pfb_head(N)).total;
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
    if ((uintptr_t)X & 15) return fm_fail(FM_ERR_INVALID, "%s: X not 16-byte aligned", who);
    if ((uintptr_t)ws & 255) return fm_fail(FM_ERR_INVALID, "%s: workspace not 256-byte aligned", who);
    char *p = (char *)ws;
    int *chunks = (int *)(p + 256);
    const size_t nc = (N + PF_CHUNK - 1) / PF_CHUNK;
    int *nchunks = (int *)(p + 256 + fm_align_up(nc * PF_CROW * 4, 256));
    hipStream_t st = fm_stream(stream);
    hipLaunchKernelGGL(fm_pfb_lists_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, (int)N, chunks,
                       nchunks);
    rc = fm_check_launch("fm_pfb_lists_kernel");
    if (rc) return rc;
    const PfOps P = pf_ops_layout(N, in_dim, true, pfb_head(N));
    rc = pf_launch_ops(X, nullptr, nullptr, (int)N, in_dim, p, P, true, st);
    if (rc) return rc;
    PfArgs a = {};
    a.mode = 2;
    a.pw = (const uint32_t *)W;
    a.ps = (const uint16_t *)scales;
    a.pb = (const uint16_t *)biases;
    a.pbits = bits;
    a.chunks = chunks;
    a.nchunks = nchunks;
    a.T = (int)N;
    a.K = 1;
    a.max_chunks = (uint32_t)nc;
    pf_bind_ops(a, p, P, true);
    a.in_dim = in_dim;
    a.out_dim = out_dim;
    a.y = Y;
    return pf_launch_gemm(a, true, st);
}
