/*
 * fm_consumer.c -- a C host program bound to libfmoe exactly as the
 * reference's C host code would be: it includes only the headers in include/ (plus the HIP
 * runtime API for device memory), links -lfmoe, and runs one decode step of a
 * MoE layer through fm_moe_forward (the moe_forward replacement,
 * layer_forward.h:1071-1322) and, when asked, the prefill layer through
 * fm_moe_prefill_forward (batched_prefill.h:122-308).
 *
 * Usage: fm_consumer <case dir>
 *   meta.txt   "hidden inter num_experts K shared_inter T"
 *   bits.bin   uint8 [E]            blobs.bin  E packed experts, each of its own size
 *   router_{w,s,b}.bin, seg_{w,s,b}.bin (4-bit), shared.bin (4-bit blob)
 *   h_post.bin fp32 [hidden]  h_mid.bin fp32 [hidden]  (X.bin fp32 [T][hidden] when T > 0)
 * Writes out.bin (fp32 [hidden]) and, when T > 0, out_prefill.bin (fp32 [T][hidden]).
 * Test infrastructure: tests/test_gpu_c_consumer.py checks the outputs.
 */
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fm_layer_forward.h"

static void *slurp(const char *dir, const char *name, size_t *len) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", path); exit(2); }
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *p = malloc((size_t)n ? (size_t)n : 1);
    if (fread(p, 1, (size_t)n, f) != (size_t)n) { fprintf(stderr, "short read %s\n", path); exit(2); }
    fclose(f);
    if (len) *len = (size_t)n;
    return p;
}

static void *upload(const char *dir, const char *name, size_t *len) {
    size_t n;
    void *h = slurp(dir, name, &n);
    void *d = NULL;
    if (hipMalloc(&d, n) != hipSuccess || hipMemcpy(d, h, n, hipMemcpyHostToDevice) != hipSuccess) {
        fprintf(stderr, "upload %s failed\n", name);
        exit(3);
    }
    free(h);
    if (len) *len = n;
    return d;
}

static void dump(const char *dir, const char *name, const void *dev, size_t n) {
    char path[4096];
    void *h = malloc(n);
    if (hipMemcpy(h, dev, n, hipMemcpyDeviceToHost) != hipSuccess) { fprintf(stderr, "download failed\n"); exit(3); }
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    fwrite(h, 1, n, f);
    fclose(f);
    free(h);
}

#define CHECK(call)                                                                \
    do {                                                                           \
        int rc_ = (call);                                                          \
        if (rc_ < 0) { fprintf(stderr, "%s: %s\n", #call, fm_last_error()); return 1; } \
    } while (0)

int main(int argc, char **argv) {
    if (argc != 2) { fprintf(stderr, "usage: %s <case dir>\n", argv[0]); return 2; }
    const char *dir = argv[1];
    unsigned H, I, E, K, SI, T;
    char *meta = slurp(dir, "meta.txt", NULL);
    if (sscanf(meta, "%u %u %u %u %u %u", &H, &I, &E, &K, &SI, &T) != 6) { fprintf(stderr, "bad meta\n"); return 2; }
    free(meta);
    printf("fm_consumer: %s, hidden %u inter %u experts %u K %u shared_inter %u T %u\n", fm_version(), H, I, E, K,
           SI, T);

    /* the expert pool: one device copy of all blobs, blob address + bits tables */
    uint8_t *bits = slurp(dir, "bits.bin", NULL);
    size_t blob_bytes;
    char *d_blobs = upload(dir, "blobs.bin", &blob_bytes);
    const void **tab = malloc(E * sizeof(void *));
    size_t off = 0;
    for (unsigned e = 0; e < E; e++) {
        fm_expert_layout L;
        CHECK(fm_expert_layout_compute(H, I, 64, bits[e], &L));
        tab[e] = d_blobs + off;
        off += L.size;
    }
    if (off != blob_bytes) { fprintf(stderr, "blobs.bin holds %zu bytes, layouts need %zu\n", blob_bytes, off); return 2; }
    void *d_tab, *d_bits;
    hipMalloc(&d_tab, E * sizeof(void *));
    hipMalloc(&d_bits, E);
    hipMemcpy(d_tab, tab, E * sizeof(void *), hipMemcpyHostToDevice);
    hipMemcpy(d_bits, bits, E, hipMemcpyHostToDevice);

    fm_moe_layer layer;
    memset(&layer, 0, sizeof layer);
    layer.pool.blobs = (const void *const *)d_tab;
    layer.pool.bits = (const uint8_t *)d_bits;
    layer.pool.num_experts = E;
    layer.pool.hidden = H;
    layer.pool.inter = I;
    layer.pool.group_size = 64;
    layer.router_w = upload(dir, "router_w.bin", NULL);
    layer.router_s = upload(dir, "router_s.bin", NULL);
    layer.router_b = upload(dir, "router_b.bin", NULL);
    layer.router_bits = 4;
    layer.seg_w = upload(dir, "seg_w.bin", NULL);
    layer.seg_s = upload(dir, "seg_s.bin", NULL);
    layer.seg_b = upload(dir, "seg_b.bin", NULL);
    layer.seg_bits = 4;
    fm_expert_layout SL;
    CHECK(fm_expert_layout_compute(H, SI ? SI : I, 64, 4, &SL));
    CHECK(fm_expert_from_blob(upload(dir, "shared.bin", NULL), &SL, &layer.shared));
    layer.shared_bits = 4;
    layer.has_shared = 1;
    layer.shared_inter = SI;

    /* decode step: fm_moe_forward replaces moe_forward() */
    size_t ws_bytes = fm_moe_forward_workspace_size(&layer, (int)K);
    void *ws, *d_out;
    hipMalloc(&ws, ws_bytes);
    hipMalloc(&d_out, H * sizeof(float));
    CHECK(fm_workspace_init(ws, ws_bytes, NULL));
    void *d_hp = upload(dir, "h_post.bin", NULL), *d_hm = upload(dir, "h_mid.bin", NULL);
    CHECK(fm_moe_forward(&layer, (int)K, d_hp, d_hm, d_out, NULL, ws, ws_bytes, NULL));
    if (hipDeviceSynchronize() != hipSuccess) { fprintf(stderr, "sync failed\n"); return 3; }
    uint32_t status = 0;
    CHECK(fm_workspace_status(ws, &status, NULL));
    if (status) { fprintf(stderr, "workspace status %u\n", status); return 4; }
    dump(dir, "out.bin", d_out, H * sizeof(float));

    if (T > 0) { /* prefill: fm_moe_prefill_forward replaces the batched prefill MoE */
        size_t pws_bytes = fm_moe_prefill_workspace_size(&layer, (int)K, (int)T);
        void *pws, *d_pout;
        hipMalloc(&pws, pws_bytes);
        hipMalloc(&d_pout, (size_t)T * H * sizeof(float));
        CHECK(fm_workspace_init(pws, pws_bytes, NULL));
        void *d_X = upload(dir, "X.bin", NULL);
        CHECK(fm_moe_prefill_forward(&layer, (int)K, (int)T, d_X, NULL, d_pout, NULL, pws, pws_bytes, NULL));
        if (hipDeviceSynchronize() != hipSuccess) { fprintf(stderr, "sync failed\n"); return 3; }
        CHECK(fm_workspace_status(pws, &status, NULL));
        if (status) { fprintf(stderr, "prefill workspace status %u\n", status); return 4; }
        dump(dir, "out_prefill.bin", d_pout, (size_t)T * H * sizeof(float));
    }
    printf("fm_consumer: ok\n");
    return 0;
}
