"""GPU parity outside the N(0,1) input regime.

The kernels feed x (and the SwiGLU activations) to the fp16 dot / MFMA
instructions, so the operands are scaled by powers of two first (per 64-element
group in the decode and matvec kernels, per token row in the prefill GEMM).
These tests drive every path with inputs scaled by 1e-3, 1e-2 and 1e2, with a
few outliers near 3e4 (whose SwiGLU activations reach ~1e7, far beyond fp16's
range), with groups of wildly different magnitudes, and check them against the
oracle at the same bars as the N(0,1) tests (helpers.py): fp32 outputs
norm_err <= 1e-3.
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_F32, experts, matrix, norm_err

pytestmark = pytest.mark.gpu

REGIMES = ["1e-3", "1e-2", "1e2", "outliers", "mixed"]


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


def x_regime(rng, n, regime, shape=None):
    """bf16-valued inputs of a given dynamic range (last axis has n elements)."""
    x = synth.hidden_vec(rng, n, shape)
    if regime == "outliers":
        flat = x.reshape(-1, n)
        for row in flat:
            pos = rng.choice(n, 4, replace=False)
            row[pos] = rng.choice([-1.0, 1.0], 4) * rng.uniform(2.5e4, 3.2e4, 4)
        return synth.bf16_round(x)
    if regime == "mixed":  # each 64-element group at its own scale, 1e-4 .. 1e3
        g = 10.0 ** rng.uniform(-4, 3, x.shape[:-1] + (n // 64,))
        return synth.bf16_round((x.reshape(x.shape[:-1] + (n // 64, 64)) * g[..., None]).reshape(x.shape))
    return synth.bf16_round(x * np.float32(float(regime)))


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("bits", [4, 2])
def test_matvec_range(orc, dev, bits, regime):
    import torch
    say("matvec range", bits, regime)
    W, s, b = matrix(500 + bits, 1024, 4096, bits)
    x = x_regime(synth.rng_for(41, bits, REGIMES.index(regime)), 4096, regime)
    out = torch.empty(1024, dtype=torch.float32, device=dev)
    fm.dequant_matvec(T(W, dev), T(s, dev), T(b, dev), T(x, dev), out, bits)
    torch.cuda.synchronize()
    assert norm_err(out.cpu().numpy(), orc.matvec(bits, W, s, b, x)) <= TOL_F32


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("hidden,inter", [(HIDDEN, INTER), (2048, 512)])
def test_decode_range(orc, dev, regime, hidden, inter):
    """Decode step, 4-bit and 2-bit slots mixed (the per-CU MFMA kernel with
    16-group units at 4096/1024, with 8-group units at 2048/512); per-expert
    outputs and the combine."""
    import torch
    say("decode range", regime, hidden, inter)
    K = 6
    bl = [4, 2, 4, 2, 2, 4, 2]
    blobs = experts(range(5100, 5100 + K + 1), bl, hidden, inter)
    rng = synth.rng_for(42, REGIMES.index(regime), hidden)
    x = x_regime(rng, hidden, regime)
    w = orc.route(rng.normal(0, 1, 64).astype(np.float32), K)[1][0]
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, bl[i], hidden, inter) for i, db in enumerate(dblobs)]
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, hidden, inter), dev)
    eo = torch.zeros((K + 1, hidden), dtype=torch.float32, device=dev)
    fm.encode_experts_batched(ex, bl, T(x, dev), eo, ws, hidden, inter)
    out = torch.empty(hidden, dtype=torch.float32, device=dev)
    fm.moe_decode(ex[:K], bl[:K], w, T(x, dev), out, ws, hidden, inter, shared=ex[K], shared_bits=bl[K],
                  shared_score=0.7)
    torch.cuda.synchronize()
    eon = eo.cpu().numpy()
    for k in range(K + 1):
        assert norm_err(eon[k], orc.expert_forward(blobs[k], bl[k], hidden, inter, x)) <= TOL_F32, k
    ref = orc.moe_decode(blobs[:K], bl[:K], w, x, hidden, inter, shared_blob=blobs[K], shared_bits=bl[K],
                         shared_score=0.7)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("Tn", [4, 40])
def test_prefill_range(orc, dev, regime, Tn):
    """Prefill: T=4 runs the multi-token decode launch, T=40 the grouped GEMM."""
    import torch
    say("prefill range", regime, Tn)
    E, K = 16, 4
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(5200, 5200 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    rng = synth.rng_for(43, REGIMES.index(regime), Tn)
    idx, w = orc.route(rng.normal(0, 1, (Tn, E)).astype(np.float32), K)
    X = x_regime(rng, HIDDEN, regime, (Tn, HIDDEN))
    g = rng.normal(0, 1, Tn).astype(np.float32)
    shared_blob = synth.expert_blob((5300, 1), HIDDEN, INTER, 2)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 2, HIDDEN, INTER)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=2,
                   shared_scores=T(g, dev))
    torch.cuda.synchronize()
    ref = orc.prefill_moe(idx, w, blobs, bits, X, HIDDEN, INTER, shared_blob=shared_blob, shared_bits=2,
                          shared_scores=g)
    got = out.cpu().numpy()
    for t in range(Tn):  # per token: each row has its own magnitude
        assert norm_err(got[t], ref[t]) <= TOL_F32, t


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("bits", [4, 2])
def test_pfb_gemm_range(orc, dev, bits, regime):
    import torch
    say("pfb_gemm range", bits, regime)
    N, out_dim, in_dim = 24, 256, 4096
    W, s, b = matrix(600 + bits, out_dim, in_dim, bits)
    rng = synth.rng_for(44, bits, REGIMES.index(regime))
    X = x_regime(rng, in_dim, regime, (N, in_dim))
    X = X + rng.normal(0, 1e-3, X.shape).astype(np.float32) * np.abs(X)  # not bf16-exact
    Y = torch.empty((N, out_dim), dtype=torch.float32, device=dev)
    ws = torch.empty(fm.lib().fm_pfb_gemm_workspace_size(N, in_dim), dtype=torch.uint8, device=dev)
    fm.pfb_gemm(T(W, dev), T(s, dev), T(b, dev), T(X, dev), Y, bits, ws)
    torch.cuda.synchronize()
    ref = orc.gemm(bits, W, s, b, X)
    got = Y.cpu().numpy()
    for t in range(N):
        assert norm_err(got[t], ref[t]) <= TOL_F32, t
