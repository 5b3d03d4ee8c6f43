"""Python binding of libfmoe.so, the gfx950 quantized-expert backend.

The product is the C ABI in include/fm_gpu_dispatch.h and
include/fm_layer_forward.h; this module binds it with ctypes so tests and
bench.py can drive it with torch device tensors (torch supplies device memory
and streams only).  There is no fallback: if libfmoe.so is missing or a call
fails, an exception is raised.
"""
import ctypes
import os

from . import layout  # noqa: F401  (re-exported helpers)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libfmoe.so")

FM_MAX_K = 16


class FmError(RuntimeError):
    """A libfmoe entry point returned a negative status."""

    def __init__(self, code, msg):
        super().__init__(f"libfmoe error {code}: {msg}")
        self.code = code


class ExpertWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")]


class ExpertLayout(ctypes.Structure):
    _fields_ = [("off", ctypes.c_size_t * 9), ("size", ctypes.c_size_t)]


class ExpertPool(ctypes.Structure):
    _fields_ = [("blobs", ctypes.c_void_p), ("bits", ctypes.c_void_p),
                ("num_experts", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
                ("inter", ctypes.c_uint32), ("group_size", ctypes.c_uint32)]


class BatchMatvecSpec(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
                ("out", ctypes.c_void_p), ("out_dim", ctypes.c_uint32), ("in_dim", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32), ("bits", ctypes.c_int)]


class MoeLayer(ctypes.Structure):
    _fields_ = [("router_w", ctypes.c_void_p), ("router_s", ctypes.c_void_p),
                ("router_b", ctypes.c_void_p), ("router_bits", ctypes.c_int),
                ("seg_w", ctypes.c_void_p), ("seg_s", ctypes.c_void_p), ("seg_b", ctypes.c_void_p),
                ("seg_bits", ctypes.c_int),
                ("shared", ExpertWeights), ("shared_bits", ctypes.c_int), ("has_shared", ctypes.c_int),
                ("pool", ExpertPool), ("shared_inter", ctypes.c_uint32)]


class ExpertExtent(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_uint64), ("size", ctypes.c_uint64), ("bits", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class ExpertStoreInfo(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int), ("num_layers", ctypes.c_uint32), ("num_experts", ctypes.c_uint32),
                ("layers_available", ctypes.c_uint32), ("manifest_warnings", ctypes.c_uint32),
                ("expert_size_4bit", ctypes.c_uint64), ("expert_size_2bit", ctypes.c_uint64)]


_lib = None

P = ctypes.c_void_p
U32 = ctypes.c_uint32
I32 = ctypes.c_int
SZ = ctypes.c_size_t
F32 = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "fm_last_error": (ctypes.c_char_p, []),
    "fm_version": (ctypes.c_char_p, []),
    "fm_expert_layout_compute": (I32, [U32, U32, U32, I32, ctypes.POINTER(ExpertLayout)]),
    "fm_expert_from_blob": (I32, [P, ctypes.POINTER(ExpertLayout), ctypes.POINTER(ExpertWeights)]),
    "fm_dequant_matvec": (I32, [P, P, P, P, P, U32, U32, U32, I32, P]),
    "fm_batch_matvec": (I32, [P, U32, ctypes.POINTER(BatchMatvecSpec), I32, P]),
    "fm_moe_decode_workspace_size": (SZ, [I32, U32, U32]),
    "fm_moe_decode_workspace_size_ex": (SZ, [I32, I32, U32, U32, U32]),
    "fm_encode_experts_batched": (I32, [I32, P, ctypes.POINTER(ExpertWeights), P, U32, U32, U32, P, P,
                                        P, SZ, P]),
    "fm_moe_combine": (I32, [P, P, P, P, I32, P, P, P, P, U32, P]),
    "fm_moe_decode": (I32, [I32, ctypes.POINTER(ExpertWeights), P, P, P, ctypes.POINTER(ExpertWeights),
                            I32, U32, F32, U32, U32, U32, P, P, P, P, P, SZ, P]),
    "fm_moe_decode_pool": (I32, [ctypes.POINTER(ExpertPool), I32, P, P, ctypes.POINTER(ExpertWeights),
                                 I32, U32, P, P, P, P, P, P, SZ, P]),
    "fm_moe_route_decode_pool": (I32, [ctypes.POINTER(ExpertPool), P, I32, I32, P, P,
                                       ctypes.POINTER(ExpertWeights), I32, U32, P, P, P, P, P, P, SZ, P]),
    "fm_moe_decode_pool_norm": (I32, [ctypes.POINTER(ExpertPool), I32, P, P, ctypes.POINTER(ExpertWeights),
                                      I32, U32, P, P, P, P, P, P, F32, P, P, SZ, P]),
    "fm_rms_norm": (I32, [P, P, U32, F32, P, P, P]),
    "fm_swiglu": (I32, [P, P, P, U32, P]),
    "fm_moe_decode_pool_stepwise": (I32, [ctypes.POINTER(ExpertPool), I32, P, P, ctypes.POINTER(ExpertWeights),
                                          I32, U32, P, P, P, P, P, P, SZ, P]),
    "fm_workspace_status": (I32, [P, ctypes.POINTER(ctypes.c_uint32), P]),
    "fm_noalloc_workspace_bytes": (ctypes.c_size_t, []),
    "fm_noalloc_status": (I32, [ctypes.POINTER(ctypes.c_uint32), P]),
    "fm_moe_decode_pool_noalloc": (I32, [ctypes.POINTER(ExpertPool), I32, P, P, ctypes.POINTER(ExpertWeights),
                                         I32, U32, P, P, P, P, P, P]),
    "fm_workspace_init": (I32, [P, ctypes.c_size_t, P]),
    "fm_route_topk": (I32, [P, I32, I32, I32, P, P, P]),
    "fm_prefill_moe_workspace_size": (SZ, [I32, I32, ctypes.POINTER(ExpertPool), U32]),
    "fm_prefill_moe": (I32, [ctypes.POINTER(ExpertPool), I32, I32, P, P, ctypes.POINTER(ExpertWeights),
                             I32, U32, P, P, P, P, P, P, SZ, P]),
    "fm_pfb_gemm_workspace_size": (SZ, [U32, U32]),
    "fm_pfb_gemm": (I32, [P, P, P, P, P, U32, U32, U32, U32, I32, P, SZ, P]),
    "fm_moe_forward_workspace_size": (SZ, [ctypes.POINTER(MoeLayer), I32]),
    "fm_moe_forward": (I32, [ctypes.POINTER(MoeLayer), I32, P, P, P, P, P, SZ, P]),
    "fm_moe_forward_norm": (I32, [ctypes.POINTER(MoeLayer), I32, P, P, P, P, P, F32, P, P, SZ, P]),
    "fm_moe_forward_checked": (I32, [ctypes.POINTER(MoeLayer), I32, P, P, P, P, P, SZ, P,
                                     ctypes.POINTER(ctypes.c_uint32)]),
    "fm_moe_prefill_workspace_size": (SZ, [ctypes.POINTER(MoeLayer), I32, I32]),
    "fm_moe_prefill_forward": (I32, [ctypes.POINTER(MoeLayer), I32, I32, P, P, P, P, P, SZ, P]),
    "fm_expert_store_open": (I32, [ctypes.c_char_p, I32, U32, U32, U32, U32, U32, I32,
                                   ctypes.POINTER(P)]),
    "fm_expert_store_close": (None, [P]),
    "fm_expert_store_get_info": (I32, [P, ctypes.POINTER(ExpertStoreInfo)]),
    "fm_expert_get_extent": (I32, [P, I32, I32, ctypes.POINTER(ExpertExtent)]),
    "fm_expert_layer_bytes": (I32, [P, I32, ctypes.POINTER(ctypes.c_uint64)]),
    "fm_expert_read": (I32, [P, I32, I32, P, P, P]),
    "fm_expert_stage_start": (I32, [P, I32, I32, P, P, P]),
    "fm_expert_stage_wait": (I32, [P, P]),
    "fm_expert_load_layer": (I32, [P, I32, P, SZ, P, P, ctypes.POINTER(ExpertPool), P]),
}


def lib():
    """Load libfmoe.so (once); raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FmError(-100, f"{LIB_PATH} missing: run __graft_entry__.build() first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    """Raise FmError for a negative status; return non-negative results (counts) unchanged."""
    if rc < 0:
        raise FmError(rc, lib().fm_last_error().decode())
    return rc


def ptr(t):
    """Device (or host) address of a torch tensor / None -> NULL."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


from .api import *  # noqa: E402,F401,F403
from .expert_io import *  # noqa: E402,F401,F403
