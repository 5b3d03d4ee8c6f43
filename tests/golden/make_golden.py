"""Writes tests/golden/ref_kernels.npz: input/output vectors of the
reference's own CPU kernels (cpu_kernels.h:192-387, weights.h:9-21,
main.m:108-160), compiled from the reference tree by `make -C oracle ref`.

The reference ships no fixtures for this path, so these vectors are produced
here from its compiled C and committed as data; tests check the restated
oracle against them bit for bit (no reference tree needed at test time).

Run: make -C oracle all ref && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "flash-moe_amd"))

from oracle import RefLib  # noqa: E402
from fmoe_amd import synth  # noqa: E402


def main():
    ref = RefLib()
    rng = synth.rng_for(424242)
    out = {}
    # 4-bit matvec: shapes (rows, in_dim)
    for name, (r, n) in {"mv_a": (3, 128), "mv_b": (5, 4096), "mv_c": (7, 1024)}.items():
        W, s, b = synth.quant_matrix(rng, r, n, 4)
        x = synth.hidden_vec(rng, n)
        y = ref.matvec4(W, s, b, x)
        y2 = ref.matvec4(W, s, b, x, copy="main_m")
        assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "cpu_kernels.h and main.m copies differ"
        out.update({f"{name}_W": W, f"{name}_s": s, f"{name}_b": b, f"{name}_x": x, f"{name}_y": y})
    # SwiGLU incl. extremes
    g = np.concatenate([rng.normal(0, 4, 250), [0.0, -0.0, 1e-8, -1e-8, 88.0, -88.0, 100.0, -100.0]]).astype(np.float32)
    u = rng.normal(0, 4, g.size).astype(np.float32)
    out.update(sw_g=g, sw_u=u, sw_y=ref.swiglu(g, u))
    assert np.array_equal(ref.swiglu(g, u).view(np.uint32), ref.swiglu(g, u, copy="main_m").view(np.uint32))
    # softmax
    lg = rng.normal(0, 1, 512).astype(np.float32)
    lg2 = np.round(rng.normal(0, 1, 512), 1).astype(np.float32)  # many exact duplicates
    out.update(sm_x=lg, sm_y=ref.softmax(lg), sm2_x=lg2, sm2_y=ref.softmax(lg2))
    # top-K on softmax outputs (slot order), incl. ties and K = E
    for name, (sc, K) in {"tk_a": (ref.softmax(lg), 10), "tk_b": (ref.softmax(lg2), 10),
                          "tk_c": (np.array([.1, .5, .3, .5], np.float32), 2),
                          "tk_d": (rng.random(16).astype(np.float32), 16),
                          "tk_e": (ref.softmax(lg), 64)}.items():
        idx, val = ref.topk(sc, K)
        out.update({f"{name}_s": sc, f"{name}_K": np.int32(K), f"{name}_idx": idx, f"{name}_val": val})
    # renormalisation and madd
    w = rng.random(10).astype(np.float32)
    out.update(nw_x=w, nw_y=ref.normalize(w))
    d = rng.normal(0, 1, 64).astype(np.float32)
    s_ = rng.normal(0, 1, 64).astype(np.float32)
    out.update(ma_d=d, ma_s=s_, ma_c=np.float32(0.37), ma_y=ref.vec_madd(d, s_, np.float32(0.37)))
    # bf16 conversions
    bits = rng.integers(0, 2 ** 16, 64, dtype=np.uint32).astype(np.uint16)
    out.update(bf_in=bits, bf_f32=np.array([ref.L.ref_bf16_to_f32(int(v)) for v in bits], np.float32))
    f = rng.normal(0, 10, 64).astype(np.float32)
    out.update(tr_in=f, tr_out=np.array([ref.L.ref_f32_to_bf16(float(v)) for v in f], np.uint16))
    # RMS norm with bf16 weights (cpu_kernels.h:235-246)
    x = rng.normal(0, 2, 4096).astype(np.float32)
    wn = synth.bf16_bits(rng.normal(1, 0.2, 4096).astype(np.float32))
    out.update(rn_x=x, rn_w=wn, rn_eps=np.float32(1e-6), rn_y=ref.rms_norm(x, wn, np.float32(1e-6)))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_kernels.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
