"""Expert files on disk (packed_experts*/layer_XX.bin + tiered manifest) and
their movement into HBM, over the fm_expert_io.h C ABI.

`ExpertStore` mirrors the reference's start-up and I/O functions:
mode detection (generate.h:1813-1848), load_tiered_manifest (config.h:318-408),
expert_offset_size (timing.h:138-148), parallel_pread_experts
(expert_io.h:284-329) and async_pread_start/wait (expert_io.h:183-266).
"""
import ctypes

import numpy as np

from . import ExpertExtent, ExpertPool, ExpertStoreInfo, check, lib, stream_ptr

__all__ = ["ExpertStore", "STORE_AUTO", "STORE_4BIT", "STORE_2BIT", "STORE_TIERED", "write_layer_files"]

STORE_AUTO, STORE_4BIT, STORE_2BIT, STORE_TIERED = 0, 1, 2, 3


class ExpertStore:
    def __init__(self, model_dir, num_layers, num_experts, hidden, inter, group_size=64, mode=STORE_AUTO,
                 io_threads=0):
        h = ctypes.c_void_p()
        check(lib().fm_expert_store_open(str(model_dir).encode(), mode, num_layers, num_experts, hidden, inter,
                                         group_size, io_threads, ctypes.byref(h)))
        self.h = h
        self.hidden, self.inter, self.group_size = hidden, inter, group_size

    def close(self):
        if self.h:
            lib().fm_expert_store_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def info(self):
        i = ExpertStoreInfo()
        check(lib().fm_expert_store_get_info(self.h, ctypes.byref(i)))
        return i

    def extent(self, layer, expert):
        """(offset, size, bits) of one expert in its layer file."""
        x = ExpertExtent()
        check(lib().fm_expert_get_extent(self.h, layer, expert, ctypes.byref(x)))
        return x.offset, x.size, x.bits

    def layer_bytes(self, layer):
        v = ctypes.c_uint64()
        check(lib().fm_expert_layer_bytes(self.h, layer, ctypes.byref(v)))
        return v.value

    def read(self, layer, experts):
        """Parallel pread of the given experts -> (list of uint8 arrays, valid list)."""
        experts = [int(e) for e in experts]
        n = len(experts)
        bufs = [np.zeros(max(1, self.extent(layer, e)[1]), np.uint8) for e in experts]
        ids = (ctypes.c_int * max(1, n))(*experts)
        dst = (ctypes.c_void_p * max(1, n))(*[b.ctypes.data for b in bufs])
        valid = (ctypes.c_int * max(1, n))()
        check(lib().fm_expert_read(self.h, layer, n, ids, dst, valid))
        return [b[: self.extent(layer, e)[1]] for b, e in zip(bufs, experts)], list(valid)[:n]

    def stage_start(self, layer, experts, dev_ptrs, stream=None):
        experts = [int(e) for e in experts]
        n = len(experts)
        ids = (ctypes.c_int * n)(*experts)
        dst = (ctypes.c_void_p * n)(*[int(p) for p in dev_ptrs])
        check(lib().fm_expert_stage_start(self.h, layer, n, ids, dst, stream_ptr(stream)))
        self._n = n

    def stage_wait(self):
        valid = (ctypes.c_int * self._n)()
        loaded = check(lib().fm_expert_stage_wait(self.h, valid))
        return loaded, list(valid)

    def stage(self, layer, experts, dev_ptrs, stream=None):
        self.stage_start(layer, experts, dev_ptrs, stream)
        return self.stage_wait()

    def load_layer(self, layer, device="cuda", stream=None):
        """Whole layer file -> one device allocation; returns a LayerPool."""
        return LayerPool(self, layer, device, stream)


class LayerPool:
    """A layer's experts resident in HBM (fm_expert_load_layer): device storage,
    blob/bits tables and the fm_expert_pool describing them."""

    def __init__(self, store, layer, device, stream):
        import torch
        nbytes = store.layer_bytes(layer)
        E = store.info().num_experts
        self.storage = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
        base = (self.storage.data_ptr() + 255) // 256 * 256
        self.blob_table = torch.empty(E, dtype=torch.int64, device=device)
        self.bits_table = torch.empty(E, dtype=torch.uint8, device=device)
        self.c = ExpertPool()
        check(lib().fm_expert_load_layer(store.h, layer, ctypes.c_void_p(base), nbytes,
                                         ctypes.c_void_p(self.blob_table.data_ptr()),
                                         ctypes.c_void_p(self.bits_table.data_ptr()), ctypes.byref(self.c),
                                         stream_ptr(stream)))
        self.base = base


def write_layer_files(model_dir, layers, mode, size4, size2, threshold=None):
    """Write expert files in the reference's on-disk format (repack_experts_tiered.py:345-425
    for the tiered manifest).  layers: list over layers of lists of (blob uint8 array, bits).
    mode: "4bit" (packed_experts/), "2bit" (packed_experts_2bit/) or "tiered"."""
    import json
    import os
    sub = {"4bit": "packed_experts", "2bit": "packed_experts_2bit", "tiered": "packed_experts_tiered"}[mode]
    d = os.path.join(str(model_dir), sub)
    os.makedirs(d, exist_ok=True)
    manifest = {"expert_size_4bit": size4, "expert_size_2bit": size2, "num_layers": len(layers),
                "num_experts": len(layers[0]) if layers else 0, "threshold": threshold, "gptq_source": None,
                "layers": {}}
    for l, experts in enumerate(layers):
        off = 0
        entries = []
        with open(os.path.join(d, f"layer_{l:02d}.bin"), "wb") as f:
            for blob, bits in experts:
                f.write(np.ascontiguousarray(blob, dtype=np.uint8).tobytes())
                entries.append({"offset": off, "size": int(blob.size), "bits": int(bits)})
                off += int(blob.size)
        manifest["layers"][str(l)] = {"experts": entries, "file_size": off}
    if mode == "tiered":
        with open(os.path.join(d, "tiered_manifest.json"), "w") as f:
            json.dump(manifest, f, indent=2)
    return manifest
