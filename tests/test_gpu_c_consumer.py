"""The C ABI driven by a C program (tests/c_consumer/fm_consumer.c, built by
__graft_entry__.build()): a MoE layer's decode step through fm_moe_forward and
its prefill through fm_moe_prefill_forward, as the reference's C host code
would call them (INTEGRATION.md's binding), checked against the oracle
(fp32 norm_err <= 1e-3, helpers.py)."""
import os
import subprocess

import numpy as np
import pytest

from fmoe_amd import synth
from helpers import TOL_F32, experts, matrix, norm_err

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_consumer", "fm_consumer")


@pytest.mark.parametrize("H,I,E,K,SI,Tn", [(4096, 1024, 64, 10, 0, 24), (2048, 512, 32, 8, 768, 5)])
def test_c_consumer_layer(orc, dev, tmp_path, H, I, E, K, SI, Tn):
    print("[case] c consumer", H, I, E, K, SI, Tn, flush=True)
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} not built: run __graft_entry__.build()")
    bits = [4 if e % 4 else 2 for e in range(E)]
    blobs = experts(range(9600, 9600 + E), bits, H, I)
    Wr, sr, br = matrix(960 + H, E, H, 4)
    Wg, sg, bg = matrix(961 + H, 1, H, 4)
    sb = synth.expert_blob((9700, H), H, SI or I, 4)
    rng = synth.rng_for(96, H)
    hp = synth.hidden_vec(rng, H)
    hm = rng.normal(0, 1, H).astype(np.float32)
    X = synth.hidden_vec(rng, H, (Tn, H))
    d = tmp_path
    (d / "meta.txt").write_text(f"{H} {I} {E} {K} {SI} {Tn}\n")
    np.asarray(bits, np.uint8).tofile(d / "bits.bin")
    np.concatenate(blobs).tofile(d / "blobs.bin")
    for name, a in (("router_w", Wr), ("router_s", sr), ("router_b", br), ("seg_w", Wg), ("seg_s", sg),
                    ("seg_b", bg), ("shared", sb), ("h_post", hp), ("h_mid", hm), ("X", X)):
        np.ascontiguousarray(a).tofile(d / f"{name}.bin")
    r = subprocess.run([EXE, str(d)], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    out = np.fromfile(d / "out.bin", np.float32)
    ri, rw = orc.route(orc.matvec(4, Wr, sr, br, hp), K)
    score = orc.matvec(4, Wg, sg, bg, hp)[0]
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], hp, H, I, shared_blob=sb,
                         shared_bits=4, shared_score=float(score), h_mid=hm, shared_inter=SI)
    assert norm_err(out - hm, ref - hm) <= TOL_F32
    outp = np.fromfile(d / "out_prefill.bin", np.float32).reshape(Tn, H)
    pi, pw = orc.route(orc.gemm(4, Wr, sr, br, X), K)
    sc = orc.gemm(4, Wg, sg, bg, X)[:, 0]
    refp = orc.prefill_moe(pi, pw, blobs, bits, X, H, I, shared_blob=sb, shared_bits=4, shared_scores=sc,
                           shared_inter=SI)
    assert norm_err(outp, refp) <= TOL_F32
