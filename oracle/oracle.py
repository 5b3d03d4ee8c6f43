"""ctypes binding of the CPU checker libraries.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.

  OracleLib  -- liboracle_fm.so, this build's C restatement (fm_oracle.c)
  RefLib     -- _ref/libref_kernels.so, the reference's own cpu_kernels.h
                functions compiled from their source text (optional: only
                built where the reference tree is present)
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle_fm.so")
REF_SO = os.path.join(HERE, "_ref", "libref_kernels.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class OracleLib:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(path)
        sig = {
            "fmo_bf16_to_f32": (_F, [ctypes.c_uint16]),
            "fmo_f32_to_bf16_trunc": (ctypes.c_uint16, [_F]),
            "fmo_f32_to_bf16_rne": (ctypes.c_uint16, [_F]),
            "fmo_dequant_matvec": (None, [_I, _P, _P, _P, _P, _P, _I, _I, _I]),
            "fmo_unpack_codes": (None, [_I, _P, ctypes.c_size_t, _P]),
            "fmo_pack_codes": (None, [_I, _P, ctypes.c_size_t, _P]),
            "fmo_swiglu": (None, [_P, _P, _P, _I]),
            "fmo_sigmoid": (_F, [_F]),
            "fmo_softmax": (None, [_P, _I]),
            "fmo_rms_norm": (None, [_P, _P, _P, _I, _F]),
            "fmo_topk": (None, [_P, _I, _I, _P, _P]),
            "fmo_normalize_weights": (None, [_P, _I]),
            "fmo_vec_madd": (None, [_P, _P, _F, _I]),
            "fmo_route": (None, [_P, _I, _I, _P, _P, _P]),
            "fmo_expert_offsets": (ctypes.c_size_t, [_I, _I, _I, _I, _P]),
            "fmo_expert_forward": (None, [_P, _I, _I, _I, _I, _P, _P]),
            "fmo_moe_decode": (None, [_I, _P, _P, _P, _P, _P, _I, _I, _F, _I, _I, _I, _P, _P, _P]),
            "fmo_prefill_moe": (None, [_I, _I, _P, _P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P, _P, _P]),
            "fmo_dequant_gemm": (None, [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        self.L = L

    # -- scalar / vector kernels ---------------------------------------------
    def matvec(self, bits, W, s, b, x, group_size=64):
        W, s, b, x = _c(W, np.uint32), _c(s, np.uint16), _c(b, np.uint16), _c(x, np.float32)
        out_dim = W.shape[0]
        in_dim = x.shape[0]
        out = np.empty(out_dim, dtype=np.float32)
        self.L.fmo_dequant_matvec(bits, _p(W), _p(s), _p(b), _p(x), _p(out), out_dim, in_dim, group_size)
        return out

    def gemm(self, bits, W, s, b, X, group_size=64):
        W, s, b, X = _c(W, np.uint32), _c(s, np.uint16), _c(b, np.uint16), _c(X, np.float32)
        N, in_dim = X.shape
        Y = np.empty((N, W.shape[0]), dtype=np.float32)
        self.L.fmo_dequant_gemm(bits, _p(W), _p(s), _p(b), _p(X), _p(Y), N, W.shape[0], in_dim, group_size)
        return Y

    def unpack(self, bits, packed):
        packed = _c(packed, np.uint32).reshape(-1)
        out = np.empty(packed.size * (32 // bits), dtype=np.uint8)
        self.L.fmo_unpack_codes(bits, _p(packed), packed.size, _p(out))
        return out

    def pack(self, bits, codes):
        codes = _c(codes, np.uint8).reshape(-1)
        out = np.empty(codes.size // (32 // bits), dtype=np.uint32)
        self.L.fmo_pack_codes(bits, _p(codes), codes.size, _p(out))
        return out

    def swiglu(self, g, u):
        g, u = _c(g, np.float32), _c(u, np.float32)
        o = np.empty_like(g)
        self.L.fmo_swiglu(_p(g), _p(u), _p(o), g.size)
        return o

    def sigmoid(self, x):
        return self.L.fmo_sigmoid(float(x))

    def softmax(self, x):
        x = _c(x, np.float32).copy()
        self.L.fmo_softmax(_p(x), x.size)
        return x

    def rms_norm(self, x, w_bf16, eps):
        x, w = _c(x, np.float32), _c(w_bf16, np.uint16)
        o = np.empty_like(x)
        self.L.fmo_rms_norm(_p(x), _p(w), _p(o), x.size, eps)
        return o

    def topk(self, scores, K):
        scores = _c(scores, np.float32)
        idx = np.empty(K, dtype=np.int32)
        val = np.empty(K, dtype=np.float32)
        self.L.fmo_topk(_p(scores), scores.size, K, _p(idx), _p(val))
        return idx, val

    def normalize(self, w):
        w = _c(w, np.float32).copy()
        self.L.fmo_normalize_weights(_p(w), w.size)
        return w

    def route(self, logits, K):
        """Per-row softmax/top-K/renormalise of a [T,E] (or [E]) logits array."""
        lg = _c(logits, np.float32)
        if lg.ndim == 1:
            lg = lg[None]
        T, E = lg.shape
        idx = np.empty((T, K), dtype=np.int32)
        w = np.empty((T, K), dtype=np.float32)
        for t in range(T):
            row = np.ascontiguousarray(lg[t])
            self.L.fmo_route(_p(row), E, K, _p(idx[t]), _p(w[t]), None)
        return idx, w

    def expert_offsets(self, hidden, inter, group_size, bits):
        off = (ctypes.c_size_t * 9)()
        size = self.L.fmo_expert_offsets(hidden, inter, group_size, bits, ctypes.cast(off, _P))
        return list(off), size

    def expert_forward(self, blob, bits, hidden, inter, x, group_size=64):
        blob, x = _c(blob, np.uint8), _c(x, np.float32)
        out = np.empty(hidden, dtype=np.float32)
        self.L.fmo_expert_forward(_p(blob), bits, hidden, inter, group_size, _p(x), _p(out))
        return out

    def moe_decode(self, blobs, bits, w, x, hidden, inter, valid=None, shared_blob=None, shared_bits=4,
                   shared_score=0.0, h_mid=None, group_size=64, shared_inter=0):
        K = len(blobs)
        blobs = [_c(b, np.uint8) for b in blobs]
        ptrs = (ctypes.c_void_p * max(1, K))(*[b.ctypes.data for b in blobs])
        bits_a = _c(bits, np.int32)
        w_a = _c(w, np.float32)
        valid_a = None if valid is None else _c(valid, np.int32)
        sb = None if shared_blob is None else _c(shared_blob, np.uint8)
        x = _c(x, np.float32)
        hm = None if h_mid is None else _c(h_mid, np.float32)
        out = np.empty(hidden, dtype=np.float32)
        self.L.fmo_moe_decode(K, ctypes.cast(ptrs, _P), _p(bits_a), _p(w_a), _p(valid_a), _p(sb), shared_bits,
                              shared_inter, float(shared_score), hidden, inter, group_size, _p(x), _p(hm), _p(out))
        return out

    def prefill_moe(self, idx, w, blob_table, bits_table, X, hidden, inter, shared_blob=None, shared_bits=4,
                    shared_scores=None, h_mid=None, group_size=64, shared_inter=0):
        idx, w = _c(idx, np.int32), _c(w, np.float32)
        T, K = idx.shape
        blob_table = [_c(b, np.uint8) if b is not None else None for b in blob_table]
        ptrs = (ctypes.c_void_p * len(blob_table))(*[b.ctypes.data if b is not None else 0 for b in blob_table])
        bits_a = _c(bits_table, np.int32)
        sb = None if shared_blob is None else _c(shared_blob, np.uint8)
        ss = None if shared_scores is None else _c(shared_scores, np.float32)
        X = _c(X, np.float32)
        hm = None if h_mid is None else _c(h_mid, np.float32)
        out = np.empty((T, hidden), dtype=np.float32)
        self.L.fmo_prefill_moe(T, K, _p(idx), _p(w), ctypes.cast(ptrs, _P), _p(bits_a), _p(sb), shared_bits,
                               shared_inter, _p(ss), hidden, inter, group_size, _p(X), _p(hm), _p(out))
        return out


class RefLib:
    """The reference's own CPU kernels (cpu_kernels.h:192-387, weights.h:9-21,
    main.m:108-160), compiled by oracle/Makefile `ref` from the reference tree."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = ctypes.CDLL(path)
        sig = {
            "ref_bf16_to_f32": (_F, [ctypes.c_uint16]),
            "ref_f32_to_bf16": (ctypes.c_uint16, [_F]),
            "ref_cpu_dequant_matvec": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
            "ref_main_dequant_matvec_4bit": (None, [_P, _P, _P, _P, _P, ctypes.c_uint32, ctypes.c_uint32,
                                                    ctypes.c_uint32]),
            "ref_cpu_swiglu": (None, [_P, _P, _P, _I]),
            "ref_main_swiglu": (None, [_P, _P, _P, ctypes.c_uint32]),
            "ref_cpu_sigmoid": (_F, [_F]),
            "ref_cpu_softmax": (None, [_P, _I]),
            "ref_cpu_topk": (None, [_P, _I, _I, _P, _P]),
            "ref_cpu_normalize_weights": (None, [_P, _I]),
            "ref_cpu_vec_madd": (None, [_P, _P, _F, _I]),
            "ref_cpu_rms_norm": (None, [_P, _P, _P, _I, _F]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        self.L = L

    def matvec4(self, W, s, b, x, group_size=64, copy="cpu_kernels"):
        W, s, b, x = _c(W, np.uint32), _c(s, np.uint16), _c(b, np.uint16), _c(x, np.float32)
        out = np.empty(W.shape[0], dtype=np.float32)
        fn = self.L.ref_cpu_dequant_matvec if copy == "cpu_kernels" else self.L.ref_main_dequant_matvec_4bit
        fn(_p(W), _p(s), _p(b), _p(x), _p(out), W.shape[0], x.shape[0], group_size)
        return out

    def swiglu(self, g, u, copy="cpu_kernels"):
        g, u = _c(g, np.float32), _c(u, np.float32)
        o = np.empty_like(g)
        fn = self.L.ref_cpu_swiglu if copy == "cpu_kernels" else self.L.ref_main_swiglu
        fn(_p(g), _p(u), _p(o), g.size)
        return o

    def softmax(self, x):
        x = _c(x, np.float32).copy()
        self.L.ref_cpu_softmax(_p(x), x.size)
        return x

    def rms_norm(self, x, w_bf16, eps):
        x, w = _c(x, np.float32), _c(w_bf16, np.uint16)
        o = np.empty_like(x)
        self.L.ref_cpu_rms_norm(_p(x), _p(w), _p(o), x.size, eps)
        return o

    def topk(self, scores, K):
        scores = _c(scores, np.float32)
        idx = np.empty(K, dtype=np.int32)
        val = np.empty(K, dtype=np.float32)
        self.L.ref_cpu_topk(_p(scores), scores.size, K, _p(idx), _p(val))
        return idx, val

    def normalize(self, w):
        w = _c(w, np.float32).copy()
        self.L.ref_cpu_normalize_weights(_p(w), w.size)
        return w

    def vec_madd(self, dst, src, scale):
        dst = _c(dst, np.float32).copy()
        src = _c(src, np.float32)
        self.L.ref_cpu_vec_madd(_p(dst), _p(src), float(scale), dst.size)
        return dst
