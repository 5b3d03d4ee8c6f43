/*
 * fm_expert_io.h -- on-disk expert formats and expert staging into HBM.
 *
 * Replaces the expert file handling of metal_infer: the per-layer packed
 * expert files and their tiered manifest (config.h:78-92, 318-408;
 * generate.h:1813-1870), the expert offset lookup (timing.h:138-148) and the
 * pread pipeline that moves expert blobs into GPU-visible buffers
 * (expert_io.h:150-340).  On MI355X the whole expert pool of a model fits in
 * 288 GB of HBM, so the primary path loads a layer file once into device
 * memory (fm_expert_load_layer) and the decode/prefill kernels read experts
 * from there; the per-token staging path (fm_expert_stage_*) serves pools
 * larger than HBM.
 *
 * Files (relative to model_dir), exactly the reference's:
 *   packed_experts/layer_XX.bin         experts back to back, 4-bit, expert e at e * size4
 *   packed_experts_2bit/layer_XX.bin    same with 2-bit blobs (e * size2)
 *   packed_experts_tiered/layer_XX.bin  mixed 4/2-bit blobs at manifest offsets
 *   packed_experts_tiered/tiered_manifest.json
 *       {"expert_size_4bit": N, "expert_size_2bit": N, "num_layers": L,
 *        "num_experts": E, "threshold": x,
 *        "layers": {"0": {"experts": [{"offset": o, "size": s, "bits": b}, ...],
 *                         "file_size": n}, ...}}
 *   (writer: repack_experts_tiered.py:345-425).  Blob layout inside a file
 *   entry: fm_expert_layout_compute().
 *
 * Conventions as in fm_gpu_dispatch.h: 0 / negative FM_ERR_* plus
 * fm_last_error().  A store is used by one thread at a time; its I/O worker
 * threads are internal.
 */
#ifndef FM_EXPERT_IO_H
#define FM_EXPERT_IO_H

#include <stddef.h>
#include <stdint.h>

#include "fm_gpu_dispatch.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FM_ERR_IO (-5) /* a file could not be opened or read */

/* Which expert files a store reads. */
#define FM_STORE_AUTO 0   /* generate.h:1813-1848: tiered if its manifest exists, else 2-bit if only
                             packed_experts_2bit/layer_00.bin exists, else 4-bit */
#define FM_STORE_4BIT 1   /* packed_experts/ */
#define FM_STORE_2BIT 2   /* packed_experts_2bit/ (--2bit) */
#define FM_STORE_TIERED 3 /* packed_experts_tiered/ + tiered_manifest.json (--tiered) */

typedef struct fm_expert_store fm_expert_store;

/* Where one expert lives in its layer file: TieredExpertInfo (config.h:81-86). */
typedef struct {
    uint64_t offset; /* byte offset in layer_XX.bin */
    uint64_t size;   /* bytes of the blob (0: entry missing from the manifest) */
    int32_t bits;    /* 2 or 4 (0: entry missing) */
    int32_t reserved;
} fm_expert_extent;

typedef struct {
    int mode;                  /* FM_STORE_4BIT / _2BIT / _TIERED after auto-detection */
    uint32_t num_layers, num_experts;
    uint32_t layers_available; /* layer files that opened (generate.h:1862-1870 counts these) */
    uint32_t manifest_warnings;/* missing layers (defaulted to 4-bit), invalid bits (-> 4), missing entries */
    uint64_t expert_size_4bit, expert_size_2bit;
} fm_expert_store_info;

/* Open the expert files of a model.  Mirrors the reference's start-up: mode
 * detection (generate.h:1813-1848), manifest load and validation
 * (config.h:318-408: num_layers/num_experts and, when present, both expert
 * sizes must match, else FM_ERR_INVALID; a missing layer defaults to 4-bit
 * sequential offsets; bits outside {2,4} fall back to 4 -- both counted in
 * manifest_warnings).  A layer file that does not open leaves that layer
 * unavailable (its reads report invalid) rather than failing the open.
 * io_threads: pread workers (<= 0: 8, expert_io.h:9 NUM_IO_THREADS).
 * No GPU call is made. */
int fm_expert_store_open(const char *model_dir, int mode, uint32_t num_layers, uint32_t num_experts,
                         uint32_t hidden, uint32_t inter, uint32_t group_size, int io_threads,
                         fm_expert_store **out);

/* Joins the workers, waits for in-flight staging copies, frees pinned buffers. */
void fm_expert_store_close(fm_expert_store *store);

int fm_expert_store_get_info(const fm_expert_store *store, fm_expert_store_info *out);

/* expert_offset_size (timing.h:138-148) plus the bit width. */
int fm_expert_get_extent(const fm_expert_store *store, int layer, int expert, fm_expert_extent *out);

/* Bytes a device copy of the layer needs: max over experts of offset + size. */
int fm_expert_layer_bytes(const fm_expert_store *store, int layer, uint64_t *out);

/* Parallel pread of n experts of `layer` into host buffers (parallel_pread_experts,
 * expert_io.h:284-329): blobs are split into page-aligned chunks spread over the
 * workers (expert_io.h:156-170).  valid[k] = 1 iff all size bytes of expert k were
 * read.  Returns the number of valid experts (>= 0) or FM_ERR_INVALID. */
int fm_expert_read(fm_expert_store *store, int layer, int n, const int *experts, void *const *host_dst,
                   int *valid);

/* Per-token staging into HBM (async_pread_start / async_pread_wait,
 * expert_io.h:183-266).  start: queues the preads of n <= FM_MAX_K + 1 experts
 * (host index array) into the store's pinned staging set and returns at once;
 * dev_dst[k] (host array of device pointers, copied by the call) must hold
 * extent.size bytes.  wait: as each expert's reads complete it enqueues its
 * host->device copy on `stream`, so later reads overlap earlier copies; returns
 * the number of valid experts and fills valid[k] (host).  Kernels launched on
 * `stream` after wait see the data.  Two pinned sets alternate (the
 * reference's A/B buffer sets): a set is refilled only after its previous
 * copies finished.  One staging operation may be in flight per store. */
int fm_expert_stage_start(fm_expert_store *store, int layer, int n, const int *experts,
                          void *const *dev_dst, void *stream);
int fm_expert_stage_wait(fm_expert_store *store, int *valid);

/* Copy a whole layer file into device memory at dev_dst (dev_bytes >=
 * fm_expert_layer_bytes) and fill the pool tables: blob_table[e] = dev_dst +
 * offset(e) (device array, num_experts pointers), bits_table[e] (device array,
 * num_experts bytes).  Every blob must be 256-byte aligned in the file (the
 * reference's sizes 7,077,888 / 3,932,160 are).  Synchronous: returns after the
 * copies completed.  *pool_out describes the result for fm_moe_decode_pool /
 * fm_prefill_moe.  FM_ERR_IO if the file is unavailable or short. */
int fm_expert_load_layer(fm_expert_store *store, int layer, void *dev_dst, size_t dev_bytes,
                         const void **blob_table, uint8_t *bits_table, fm_expert_pool *pool_out,
                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FM_EXPERT_IO_H */
