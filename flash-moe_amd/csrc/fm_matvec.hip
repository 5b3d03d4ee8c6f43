// fm_matvec.hip -- group-wise affine 2/4-bit dequant matvec for gfx950.
//
// Replaces dequant_matvec_4bit_v3 / dequant_matvec_2bit (shaders.metal:266-359,
// 447-537) and their dispatch (gpu_dispatch.h:23-147, metal_ctx.h:907-929).
//
// Mapping: 64-lane wavefront; LPR lanes share one output row, each lane owns
// whole 64-element groups (32 B of packed 4-bit codes = two 128-bit loads,
// one bf16 scale, one bf16 bias).  A wave issues all of its weight loads
// first; the workgroup then stages x once in LDS as fp16 pairs in the operand
// layout of every group (a per-lane copy would read all of x per wave).
// Rows are reduced across the LPR lanes with cross-lane adds; fp32 throughout.
// Several matvecs sharing x (a BatchMatvecSpec list) go in ONE launch: the
// block index is mapped to (spec, row block) through a prefix table.
#include "fm_device.h"
#include "fm_internal.h"

#define FM_MV_MAX_SPECS 16
#define FM_MV_NP 2  // row passes per wave (eight-wave workgroups: 256 of them for 4096 rows)

struct FmMvSpec {
    const uint32_t *W;
    const uint16_t *s;
    const uint16_t *b;
    float *out;
    uint32_t out_dim;
    int bits;
    uint32_t block_start;
    uint32_t pad;
};

struct FmMvArgs {
    FmMvSpec spec[FM_MV_MAX_SPECS];
    int nspec;
    uint32_t in_dim;
    const float *x;
};

template <int BITS, int LPR, int GPL>
__device__ __forceinline__ void fm_mv_body(const FmMvSpec &sp, const float *__restrict__ x,
                                           uint32_t in_dim, uint32_t row0, FmXGroup *xs) {
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, gl = lane % LPR;
    const uint32_t G = in_dim / 64;
    const uint32_t wpr = in_dim * BITS / 32;  // u32 words per row
    constexpr int WPG = 2 * BITS;              // words per group

    // weights first: all of this wave's rows in flight before x is staged
    FmWGroup wv[FM_MV_NP][GPL];
    float sv[FM_MV_NP][GPL], bv[FM_MV_NP][GPL];
#pragma unroll
    for (int p = 0; p < FM_MV_NP; p++) {
        uint32_t row = row0 + p * RPP + sub;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < sp.out_dim && g < G) {
                fm_load_wgroup<BITS>(sp.W + (size_t)row * wpr + g * WPG, wv[p][j]);
                sv[p][j] = fm_bf16_to_f32(fm_ldg_u16(sp.s + (size_t)row * G + g));
                bv[p][j] = fm_bf16_to_f32(fm_ldg_u16(sp.b + (size_t)row * G + g));
            }
        }
    }
    // x once per workgroup, as the lane operand layout of every group, in LDS
    fm_stage_xgroups<BITS>(x, G, xs);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < FM_MV_NP; p++) {
        uint32_t row = row0 + p * RPP + sub;
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            uint32_t g = gl + j * LPR;
            if (row < sp.out_dim && g < G) part += fm_group_dot<BITS>(wv[p][j], xs[g], sv[p][j], bv[p][j]);
        }
        float tot = fm_lane_sum<LPR>(part);
        if (gl == 0 && row < sp.out_dim) sp.out[row] = tot;
    }
}

template <int LPR, int GPL, int W>  // W waves per workgroup
__global__ __launch_bounds__(64 * W) void fm_matvec_kernel(FmMvArgs a) {
    constexpr int RPP = 64 / LPR;
    constexpr int RB = W * FM_MV_NP * RPP;  // rows per block
    __shared__ FmXGroup xs[256];            // in_dim <= 16384
    const uint32_t blk = blockIdx.x;
    int si = 0;
    while (si + 1 < a.nspec && blk >= a.spec[si + 1].block_start) si++;
    const FmMvSpec &sp = a.spec[si];
    const uint32_t row0 = (blk - sp.block_start) * RB + (threadIdx.x >> 6) * (FM_MV_NP * RPP);
    if (sp.bits == 4)
        fm_mv_body<4, LPR, GPL>(sp, a.x, a.in_dim, row0, xs);
    else
        fm_mv_body<2, LPR, GPL>(sp, a.x, a.in_dim, row0, xs);
}

static int fm_launch_matvec(const FmMvArgs &a, int lpr, int gpl, int w, uint32_t blocks, hipStream_t st) {
    dim3 grid(blocks), block(64 * w);
#define FM_MV_CASE(L, G, W_)                                                     \
    if (lpr == L && gpl == G && w == W_) {                                       \
        hipLaunchKernelGGL((fm_matvec_kernel<L, G, W_>), grid, block, 0, st, a); \
        return fm_check_launch("fm_matvec_kernel");                              \
    }
    FM_MV_CASE(16, 1, 4)
    FM_MV_CASE(32, 1, 4)
    FM_MV_CASE(64, 1, 4)
    FM_MV_CASE(64, 2, 4)
    FM_MV_CASE(64, 4, 4)
    FM_MV_CASE(16, 1, 8)
    FM_MV_CASE(32, 1, 8)
    FM_MV_CASE(64, 1, 8)
    FM_MV_CASE(64, 2, 8)
    FM_MV_CASE(64, 4, 8)
#undef FM_MV_CASE
    return fm_fail(FM_ERR_UNSUPPORTED, "fm_matvec: no kernel for lpr=%d gpl=%d", lpr, gpl);
}

static uint32_t fm_mv_rows_per_block(int lpr, int w) { return (uint32_t)w * FM_MV_NP * (64u / lpr); }

extern "C" int fm_batch_matvec(const float *x, uint32_t x_dim, const fm_batch_matvec_spec *specs,
                               int num_specs, void *stream) {
    fm_clear_error();
    FM_REQUIRE(x && specs, "fm_batch_matvec: NULL x or specs");
    FM_REQUIRE(num_specs >= 1 && num_specs <= 64, "fm_batch_matvec: num_specs %d outside 1..64", num_specs);
    for (int i = 0; i < num_specs; i++) {
        const fm_batch_matvec_spec &s = specs[i];
        FM_REQUIRE(s.W && s.scales && s.biases && s.out, "fm_batch_matvec: spec %d has a NULL pointer", i);
        FM_REQUIRE(s.in_dim == x_dim, "fm_batch_matvec: spec %d in_dim %u != x_dim %u", i, s.in_dim, x_dim);
        int rc = fm_check_dims("fm_batch_matvec", s.out_dim, s.in_dim, s.group_size, s.bits);
        if (rc) return rc;
    }
    int lpr, gpl;
    fm_pick_lanes(x_dim / 64, &lpr, &gpl);
    // eight waves a workgroup (rows per workgroup doubled, so x is staged
    // half as often: 5.27 against 5.45 us for 4096 x 4096) while that still
    // leaves a workgroup for every CU, else four
    uint32_t rows = 0;
    for (int i = 0; i < num_specs; i++) rows += specs[i].out_dim;
    const int w = rows >= fm_mv_rows_per_block(lpr, 8) * (uint32_t)fm_num_cus() ? 8 : 4;
    const uint32_t rb = fm_mv_rows_per_block(lpr, w);
    for (int base = 0; base < num_specs; base += FM_MV_MAX_SPECS) {
        FmMvArgs a = {};
        a.nspec = num_specs - base < FM_MV_MAX_SPECS ? num_specs - base : FM_MV_MAX_SPECS;
        a.in_dim = x_dim;
        a.x = x;
        uint32_t blocks = 0;
        for (int i = 0; i < a.nspec; i++) {
            const fm_batch_matvec_spec &s = specs[base + i];
            a.spec[i].W = (const uint32_t *)s.W;
            a.spec[i].s = (const uint16_t *)s.scales;
            a.spec[i].b = (const uint16_t *)s.biases;
            a.spec[i].out = s.out;
            a.spec[i].out_dim = s.out_dim;
            a.spec[i].bits = s.bits;
            a.spec[i].block_start = blocks;
            blocks += (s.out_dim + rb - 1) / rb;
        }
        int rc = fm_launch_matvec(a, lpr, gpl, w, blocks, fm_stream(stream));
        if (rc) return rc;
    }
    return FM_OK;
}

extern "C" int fm_dequant_matvec(const void *W, const void *scales, const void *biases,
                                 const float *x, float *out, uint32_t out_dim, uint32_t in_dim,
                                 uint32_t group_size, int bits, void *stream) {
    fm_batch_matvec_spec s = {W, scales, biases, out, out_dim, in_dim, group_size, bits};
    fm_clear_error();
    FM_REQUIRE(W && scales && biases && x && out, "fm_dequant_matvec: NULL pointer argument");
    int rc = fm_check_dims("fm_dequant_matvec", out_dim, in_dim, group_size, bits);
    if (rc) return rc;
    return fm_batch_matvec(x, in_dim, &s, 1, stream);
}
