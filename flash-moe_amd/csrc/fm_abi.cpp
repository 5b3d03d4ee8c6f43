// fm_abi.cpp -- error reporting, version, expert layout (host only).
#include <stdio.h>
#include <string.h>

#include "fm_internal.h"

static thread_local char g_err[512];

int fm_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

void fm_clear_error(void) { g_err[0] = 0; }

int fm_check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return FM_OK;
}

int fm_check_dims(const char *who, uint32_t out_dim, uint32_t in_dim, uint32_t group_size,
                  int bits) {
    if (bits != 2 && bits != 4) return fm_fail(FM_ERR_INVALID, "%s: bits must be 2 or 4 (got %d)", who, bits);
    if (group_size != 64)
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: group_size must be 64 (got %u)", who, group_size);
    if (out_dim == 0 || in_dim == 0) return fm_fail(FM_ERR_INVALID, "%s: empty matrix %ux%u", who, out_dim, in_dim);
    if (in_dim % group_size)
        return fm_fail(FM_ERR_INVALID, "%s: in_dim %u not a multiple of group_size %u", who, in_dim, group_size);
    int lpr, gpl;
    if (!fm_pick_lanes(in_dim / group_size, &lpr, &gpl))
        return fm_fail(FM_ERR_UNSUPPORTED, "%s: in_dim %u exceeds 16384", who, in_dim);
    return FM_OK;
}

extern "C" const char *fm_last_error(void) { return g_err; }

// Error reporting for the host C layer driver (same thread-local message).
extern "C" int fm_host_fail(int code, const char *msg) { return fm_fail(code, "%s", msg); }

extern "C" const char *fm_version(void) { return "flash-moe-amd 0.1 (gfx950)"; }

// config.h:94-137: nine tensors in the order gate_w, gate_s, gate_b, up_w,
// up_s, up_b, down_w, down_s, down_b; W rows hold ceil(in / (32/bits)) u32,
// scale/bias rows ceil(in / group_size) bf16.
extern "C" int fm_expert_layout_compute(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                        int bits, fm_expert_layout *out) {
    fm_clear_error();
    FM_REQUIRE(out, "fm_expert_layout_compute: out is NULL");
    FM_REQUIRE(bits == 2 || bits == 4, "fm_expert_layout_compute: bits must be 2 or 4 (got %d)", bits);
    FM_REQUIRE(hidden && inter && group_size, "fm_expert_layout_compute: zero dimension");
    size_t per = 32 / bits;
    size_t gw = (size_t)inter * ((hidden + per - 1) / per) * 4;
    size_t gsz = (size_t)inter * ((hidden + group_size - 1) / group_size) * 2;
    size_t dw = (size_t)hidden * ((inter + per - 1) / per) * 4;
    size_t dsz = (size_t)hidden * ((inter + group_size - 1) / group_size) * 2;
    size_t sizes[9] = {gw, gsz, gsz, gw, gsz, gsz, dw, dsz, dsz};
    size_t o = 0;
    for (int i = 0; i < 9; i++) {
        out->off[i] = o;
        o += sizes[i];
    }
    out->size = o;
    return FM_OK;
}

extern "C" int fm_expert_from_blob(const void *blob, const fm_expert_layout *L,
                                   fm_expert_weights *out) {
    fm_clear_error();
    FM_REQUIRE(blob && L && out, "fm_expert_from_blob: NULL argument");
    const char *b = (const char *)blob;
    out->gate_w = b + L->off[0];
    out->gate_s = b + L->off[1];
    out->gate_b = b + L->off[2];
    out->up_w = b + L->off[3];
    out->up_s = b + L->off[4];
    out->up_b = b + L->off[5];
    out->down_w = b + L->off[6];
    out->down_s = b + L->off[7];
    out->down_b = b + L->off[8];
    return FM_OK;
}

int fm_num_cus(void) {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

extern "C" int fm_workspace_status(void *ws, uint32_t *status, void *stream) {
    fm_clear_error();
    FM_REQUIRE(ws && status, "fm_workspace_status: NULL argument");
    hipStream_t st = fm_stream(stream);
    uint32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, ws, sizeof v, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) e = hipMemsetAsync(ws, 0, sizeof v, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "fm_workspace_status: %s", hipGetErrorString(e));
    *status = v;
    return FM_OK;
}
