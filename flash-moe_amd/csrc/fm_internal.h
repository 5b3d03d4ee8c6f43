// fm_internal.h -- host-side helpers shared by the C-ABI launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/fm_gpu_dispatch.h"

// Records a message for fm_last_error() and returns `code`.
int fm_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void fm_clear_error(void);

// Checks the launch just issued; maps a HIP failure to FM_ERR_HIP.
int fm_check_launch(const char *what);

#define FM_REQUIRE(cond, ...)                                   \
    do {                                                        \
        if (!(cond)) return fm_fail(FM_ERR_INVALID, __VA_ARGS__); \
    } while (0)

static inline hipStream_t fm_stream(void *s) { return (hipStream_t)s; }

static inline size_t fm_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Lanes per row and 64-element groups per lane for a row of `groups` groups.
// Returns 0 if the row is longer than the kernels are instantiated for.
static inline int fm_pick_lanes(uint32_t groups, int *lpr, int *gpl) {
    if (groups == 0) return 0;
    if (groups <= 16) { *lpr = 16; *gpl = 1; return 1; }
    if (groups <= 32) { *lpr = 32; *gpl = 1; return 1; }
    if (groups <= 64) { *lpr = 64; *gpl = 1; return 1; }
    if (groups <= 128) { *lpr = 64; *gpl = 2; return 1; }
    if (groups <= 256) { *lpr = 64; *gpl = 4; return 1; }
    return 0;
}

// Validation shared by launchers: returns FM_OK or an FM_ERR_* (message set).
int fm_check_dims(const char *who, uint32_t out_dim, uint32_t in_dim, uint32_t group_size,
                  int bits);

// Compute units of the current device (cached per device).
int fm_num_cus(void);

// T tokens' decode steps in one launch of the mfma decode kernel (pool mode):
// rows t of idx/weights [T][K], X/h_mid/out/out_bf16 [T][hidden] and
// shared_gate_scores[t].  FM_ERR_UNSUPPORTED (message set) when that kernel
// cannot take the shape or T x (K + shared) slots.
size_t fm_moe_decode_tokens_workspace_size(int T, int K, int has_shared, uint32_t hidden, uint32_t inter);
int fm_moe_decode_pool_tokens(const fm_expert_pool *pool, int T, int K, const int *idx, const float *weights,
                              const fm_expert_weights *shared, int shared_bits, const float *shared_gate_scores,
                              const float *X, const float *h_mid, float *out, uint16_t *out_bf16, void *ws,
                              size_t ws_bytes, void *stream);
