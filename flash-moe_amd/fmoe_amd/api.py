"""Thin torch-facing wrappers over the libfmoe C ABI.

Tensors passed here must already live on the GPU (torch is plumbing: it owns
device memory and streams).  Every wrapper checks the C status and raises
FmError on failure; none of them computes anything itself.
"""
import ctypes

import numpy as np

from . import BatchMatvecSpec, ExpertLayout, ExpertPool, ExpertWeights, MoeLayer, check, lib, ptr, stream_ptr

__all__ = [
    "layout_of", "experts_from_blob", "dequant_matvec", "batch_matvec", "decode_workspace_bytes",
    "moe_decode", "moe_decode_pool", "encode_experts_batched", "moe_combine", "route_topk",
    "prefill_workspace_bytes", "prefill_moe", "pfb_gemm", "DevicePool", "moe_forward",
    "moe_prefill_forward", "moe_forward_workspace_bytes", "moe_prefill_workspace_bytes",
    "moe_decode_pool_norm", "rms_norm", "moe_forward_norm", "workspace_status",
    "STATUS_WAIT_TIMEOUT", "STATUS_BAD_EXPERT", "STATUS_CHUNKS", "STATUS_EPOCH_WRAP", "workspace_init",
    "workspace", "moe_decode_pool_noalloc", "decode_workspace_bytes_ex", "moe_route_decode_pool",
    "noalloc_status", "moe_forward_checked", "moe_decode_pool_stepwise", "STATUS_RECOVERED",
]

STATUS_WAIT_TIMEOUT, STATUS_BAD_EXPERT, STATUS_CHUNKS, STATUS_EPOCH_WRAP, STATUS_RECOVERED = 1, 2, 4, 8, 16


def _i32_array(vals):
    return (ctypes.c_int * len(vals))(*[int(v) for v in vals])


def _f32_array(vals):
    return (ctypes.c_float * len(vals))(*[float(v) for v in vals])


def layout_of(hidden, inter, group_size, bits):
    L = ExpertLayout()
    check(lib().fm_expert_layout_compute(hidden, inter, group_size, bits, ctypes.byref(L)))
    return L


def experts_from_blob(blob, bits, hidden, inter, group_size=64, offset=0):
    """ExpertWeights pointing into a device uint8 tensor holding one blob at `offset`."""
    L = layout_of(hidden, inter, group_size, bits)
    e = ExpertWeights()
    check(lib().fm_expert_from_blob(ctypes.c_void_p(blob.data_ptr() + offset), ctypes.byref(L),
                                    ctypes.byref(e)))
    # the struct holds raw device addresses: keep the tensor alive with it (a
    # freed block can be returned to the driver, e.g. by torch.cuda.empty_cache
    # at the start of a graph capture, and a later launch would then fault)
    e._blob = blob
    return e


def dequant_matvec(W, scales, biases, x, out, bits, group_size=64, stream=None):
    out_dim = out.numel()
    in_dim = x.numel()
    check(lib().fm_dequant_matvec(ptr(W), ptr(scales), ptr(biases), ptr(x), ptr(out), out_dim, in_dim,
                                  group_size, bits, stream_ptr(stream)))


def batch_matvec(x, specs, stream=None):
    """specs: list of (W, scales, biases, out, bits) device tensors."""
    arr = (BatchMatvecSpec * len(specs))()
    for i, (W, s, b, out, bits) in enumerate(specs):
        arr[i] = BatchMatvecSpec(ptr(W), ptr(s), ptr(b), ptr(out), out.numel(), x.numel(), 64, bits)
    check(lib().fm_batch_matvec(ptr(x), x.numel(), arr, len(specs), stream_ptr(stream)))


def decode_workspace_bytes(n_slots, hidden, inter):
    return lib().fm_moe_decode_workspace_size(n_slots, hidden, inter)


def decode_workspace_bytes_ex(K, has_shared, hidden, inter, shared_inter):
    return lib().fm_moe_decode_workspace_size_ex(K, int(bool(has_shared)), hidden, inter, shared_inter)


def _experts_array(experts):
    arr = (ExpertWeights * max(1, len(experts)))()
    for i, e in enumerate(experts):
        arr[i] = e
    return arr


def moe_decode(experts, bits, weights, x, out, ws, hidden, inter, valid=None, shared=None,
               shared_bits=4, shared_score=0.0, h_mid=None, out_bf16=None, stream=None, shared_inter=0):
    K = len(experts)
    check(lib().fm_moe_decode(
        K, _experts_array(experts), _i32_array(bits), _f32_array(weights),
        _i32_array(valid) if valid is not None else None,
        ctypes.byref(shared) if shared is not None else None, shared_bits, shared_inter, float(shared_score),
        hidden, inter, 64, ptr(x), ptr(h_mid), ptr(out), ptr(out_bf16), ptr(ws), ws.numel() * ws.element_size(),
        stream_ptr(stream)))


def moe_decode_pool(pool, idx, weights, x, out, ws, shared=None, shared_bits=4, shared_score=None,
                    h_mid=None, out_bf16=None, stream=None, shared_inter=0):
    K = idx.numel()
    check(lib().fm_moe_decode_pool(
        ctypes.byref(pool.c), K, ptr(idx), ptr(weights), ctypes.byref(shared) if shared is not None else None,
        shared_bits, shared_inter, ptr(shared_score), ptr(x), ptr(h_mid), ptr(out), ptr(out_bf16), ptr(ws),
        ws.numel() * ws.element_size(), stream_ptr(stream)))


def moe_route_decode_pool(pool, logits, idx, weights, x, out, ws, shared=None, shared_bits=4, shared_score=None,
                          h_mid=None, out_bf16=None, stream=None, shared_inter=0):
    """Routing of `logits` ([E] or [1, E]) and the decode step in one launch
    (fm_moe_route_decode_pool); idx / weights ([K]) receive the routing."""
    K = idx.numel()
    E = logits.numel()
    check(lib().fm_moe_route_decode_pool(
        ctypes.byref(pool.c), ptr(logits), E, K, ptr(idx), ptr(weights),
        ctypes.byref(shared) if shared is not None else None, shared_bits, shared_inter, ptr(shared_score), ptr(x),
        ptr(h_mid), ptr(out), ptr(out_bf16), ptr(ws), ws.numel() * ws.element_size(), stream_ptr(stream)))


def moe_decode_pool_noalloc(pool, idx, weights, x, out, shared=None, shared_bits=4, shared_score=None,
                            h_mid=None, out_bf16=None, stream=None, shared_inter=0):
    """fm_moe_decode_pool on the library's static per-GPU workspace (no allocation)."""
    K = idx.numel()
    check(lib().fm_moe_decode_pool_noalloc(
        ctypes.byref(pool.c), K, ptr(idx), ptr(weights), ctypes.byref(shared) if shared is not None else None,
        shared_bits, shared_inter, ptr(shared_score), ptr(x), ptr(h_mid), ptr(out), ptr(out_bf16), stream_ptr(stream)))


def moe_decode_pool_norm(pool, idx, weights, x, out, ws, norm_w, eps, normed, shared=None, shared_bits=4,
                         shared_score=None, h_mid=None, out_bf16=None, stream=None, shared_inter=0):
    K = idx.numel()
    check(lib().fm_moe_decode_pool_norm(
        ctypes.byref(pool.c), K, ptr(idx), ptr(weights), ctypes.byref(shared) if shared is not None else None,
        shared_bits, shared_inter, ptr(shared_score), ptr(x), ptr(h_mid), ptr(out), ptr(out_bf16), ptr(norm_w), float(eps),
        ptr(normed), ptr(ws), ws.numel() * ws.element_size(), stream_ptr(stream)))


def workspace_status(ws, stream=None):
    """FM_STATUS_* bits accumulated in a decode/prefill workspace since the last call (then cleared)."""
    v = ctypes.c_uint32()
    check(lib().fm_workspace_status(ptr(ws), ctypes.byref(v), stream_ptr(stream)))
    return v.value


def noalloc_status(stream=None):
    """Status bits of the no-allocation calls on this device since the last read (then cleared)."""
    v = ctypes.c_uint32(0)
    check(lib().fm_noalloc_status(ctypes.byref(v), stream_ptr(stream)))
    return v.value


def workspace_init(ws, stream=None):
    """Zero a workspace with the library's fill kernel (fm_workspace_init)."""
    check(lib().fm_workspace_init(ptr(ws), ws.numel() * ws.element_size(), stream_ptr(stream)))


def workspace(nbytes, device, stream=None):
    """A freshly allocated, initialised (zeroed) device workspace of nbytes."""
    import torch
    ws = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
    workspace_init(ws, stream)
    return ws


def rms_norm(x, w_bf16, eps, out, out_bf16=None, stream=None):
    check(lib().fm_rms_norm(ptr(x), ptr(w_bf16), x.numel(), float(eps), ptr(out), ptr(out_bf16), stream_ptr(stream)))


def encode_experts_batched(experts, bits, x, expert_out, ws, hidden, inter, valid=None, stream=None):
    K = len(experts)
    check(lib().fm_encode_experts_batched(
        K, _i32_array(valid) if valid is not None else None, _experts_array(experts), _i32_array(bits),
        hidden, inter, 64, ptr(x), ptr(expert_out), ptr(ws), ws.numel() * ws.element_size(),
        stream_ptr(stream)))


def moe_combine(expert_outs, weights, out, K, h_mid=None, valid=None, shared_out=None, shared_score=None,
                out_bf16=None, stream=None):
    check(lib().fm_moe_combine(ptr(h_mid), ptr(expert_outs), ptr(weights), ptr(valid), K, ptr(shared_out),
                               ptr(shared_score), ptr(out), ptr(out_bf16), out.numel(), stream_ptr(stream)))


def route_topk(logits, K, idx, weights, stream=None):
    T, E = logits.shape
    check(lib().fm_route_topk(ptr(logits), T, E, K, ptr(idx), ptr(weights), stream_ptr(stream)))


def prefill_workspace_bytes(T, K, pool, shared_inter=0):
    return lib().fm_prefill_moe_workspace_size(T, K, ctypes.byref(pool.c), shared_inter)


def prefill_moe(pool, idx, weights, X, out, ws, shared=None, shared_bits=4, shared_scores=None, h_mid=None,
                out_bf16=None, stream=None, shared_inter=0):
    T, K = idx.shape
    check(lib().fm_prefill_moe(
        ctypes.byref(pool.c), T, K, ptr(idx), ptr(weights), ctypes.byref(shared) if shared is not None else None,
        shared_bits, shared_inter, ptr(shared_scores), ptr(X), ptr(h_mid), ptr(out), ptr(out_bf16), ptr(ws),
        ws.numel() * ws.element_size(), stream_ptr(stream)))


def pfb_gemm(W, scales, biases, X, Y, bits, ws, stream=None):
    N, in_dim = X.shape
    out_dim = Y.shape[1]
    check(lib().fm_pfb_gemm(ptr(W), ptr(scales), ptr(biases), ptr(X), ptr(Y), N, out_dim, in_dim, 64, bits,
                            ptr(ws), ws.numel() * ws.element_size(), stream_ptr(stream)))


class DevicePool:
    """A device-resident expert pool: all blobs in one HBM allocation, plus the
    device tables (blob address, bit width) an fm_expert_pool points at."""

    def __init__(self, blobs, bits, hidden, inter, group_size=64, device="cuda"):
        import torch
        sizes = [int(b.size) for b in blobs]
        offs = np.zeros(len(blobs), dtype=np.int64)
        o = 0
        for i, s in enumerate(sizes):
            offs[i] = o
            o += (s + 4095) // 4096 * 4096
        self.storage = torch.empty(o, dtype=torch.uint8, device=device)
        for i, b in enumerate(blobs):
            self.storage[offs[i]: offs[i] + sizes[i]].copy_(torch.from_numpy(b))
        base = self.storage.data_ptr()
        self.addrs = (base + offs).astype(np.int64)
        self.blob_table = torch.from_numpy(self.addrs.copy()).to(device)
        self.bits_host = np.asarray(bits, dtype=np.uint8)
        self.bits_table = torch.from_numpy(self.bits_host.copy()).to(device)
        self.offsets = offs
        self.hidden, self.inter, self.group_size = hidden, inter, group_size
        self.c = ExpertPool(self.blob_table.data_ptr(), self.bits_table.data_ptr(), len(blobs), hidden, inter,
                            group_size)

    def expert(self, e):
        """ExpertWeights of expert e."""
        return experts_from_blob(self.storage, int(self.bits_host[e]), self.hidden, self.inter,
                                 self.group_size, int(self.offsets[e]))


def moe_forward_workspace_bytes(layer, K):
    return lib().fm_moe_forward_workspace_size(ctypes.byref(layer), K)


def moe_forward(layer, K, h_post, h_mid, out, ws, out_bf16=None, stream=None):
    check(lib().fm_moe_forward(ctypes.byref(layer), K, ptr(h_post), ptr(h_mid), ptr(out), ptr(out_bf16),
                               ptr(ws), ws.numel() * ws.element_size(), stream_ptr(stream)))


def moe_forward_checked(layer, K, h_post, h_mid, out, ws, out_bf16=None, stream=None):
    """fm_moe_forward plus the status check and recovery; returns the FM_STATUS_* bits."""
    st = ctypes.c_uint32(0)
    check(lib().fm_moe_forward_checked(ctypes.byref(layer), K, ptr(h_post), ptr(h_mid), ptr(out), ptr(out_bf16),
                                       ptr(ws), ws.numel() * ws.element_size(), stream_ptr(stream), ctypes.byref(st)))
    return st.value


def moe_decode_pool_stepwise(pool, idx, weights, x, out, ws, shared=None, shared_bits=4, shared_score=None,
                             h_mid=None, out_bf16=None, stream=None, shared_inter=0):
    K = idx.numel()
    check(lib().fm_moe_decode_pool_stepwise(
        ctypes.byref(pool.c), K, ptr(idx), ptr(weights), ctypes.byref(shared) if shared is not None else None,
        shared_bits, shared_inter, ptr(shared_score), ptr(x), ptr(h_mid), ptr(out), ptr(out_bf16), ptr(ws),
        ws.numel() * ws.element_size(), stream_ptr(stream)))


def moe_forward_norm(layer, K, h_post, h_mid, out, ws, norm_w, eps, normed, out_bf16=None, stream=None):
    check(lib().fm_moe_forward_norm(ctypes.byref(layer), K, ptr(h_post), ptr(h_mid), ptr(out), ptr(out_bf16),
                                    ptr(norm_w), float(eps), ptr(normed), ptr(ws), ws.numel() * ws.element_size(),
                                    stream_ptr(stream)))


def moe_prefill_workspace_bytes(layer, K, T):
    return lib().fm_moe_prefill_workspace_size(ctypes.byref(layer), K, T)


def moe_prefill_forward(layer, K, T, h_post, h_mid, out, ws, out_bf16=None, stream=None):
    check(lib().fm_moe_prefill_forward(ctypes.byref(layer), K, T, ptr(h_post), ptr(h_mid), ptr(out),
                                       ptr(out_bf16), ptr(ws), ws.numel() * ws.element_size(),
                                       stream_ptr(stream)))
