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


@pytest.mark.parametrize("regime", REGIMES)
@pytest.mark.parametrize("K,bits", [(1, 4), (1, 2), (3, 4), (3, 2)])
def test_decode_few_slots_range(orc, dev, regime, K, bits):
    """One to three slots, no shared expert: the few-slot kernel (256
    workgroups, quarter partials handed off, down rows over all activations;
    with one slot its waves split the gate/up/down inputs), per-expert outputs
    and the combine."""
    import torch
    say("decode few slots range", regime, K, bits)
    bl = [bits] * K
    blobs = experts(range(5400 + 10 * K + bits, 5400 + 10 * K + bits + K), bl)
    rng = synth.rng_for(45, REGIMES.index(regime), K, bits)
    x = x_regime(rng, HIDDEN, regime)
    w = orc.route(rng.normal(0, 1, 16).astype(np.float32), K)[1][0]
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, bits, HIDDEN, INTER) for db in dblobs]
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    eo = torch.zeros((K, HIDDEN), dtype=torch.float32, device=dev)
    fm.encode_experts_batched(ex, bl, T(x, dev), eo, ws, HIDDEN, INTER)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode(ex, bl, w, T(x, dev), out, ws, HIDDEN, INTER)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    eon = eo.cpu().numpy()
    for k in range(K):
        assert norm_err(eon[k], orc.expert_forward(blobs[k], bits, HIDDEN, INTER, x)) <= TOL_F32, k
    ref = orc.moe_decode(blobs, bl, w, x, HIDDEN, INTER)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("regime", REGIMES)
def test_route_decode_range(orc, dev, regime):
    """The headline step: routing of 512 logits fused into the one-workgroup-
    per-CU launch (top-10 + shared, 4- and 2-bit slots)."""
    import torch
    say("route+decode range", regime)
    E, K, nb = 512, 10, 12
    bits8 = [4, 2, 4, 4, 2, 4, 2, 4, 4, 2, 4, 4]
    blobs = experts(range(5500, 5500 + nb), bits8)
    dp = fm.DevicePool(blobs, bits8, HIDDEN, INTER)
    dp.blob_table = T(np.array([dp.addrs[e % nb] for e in range(E)], np.int64), dev)
    dp.bits_table = T(np.array([bits8[e % nb] for e in range(E)], np.uint8), dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, HIDDEN, INTER, 64)
    rng = synth.rng_for(46, REGIMES.index(regime))
    lg = rng.normal(0, 1, E).astype(np.float32)
    x = x_regime(rng, HIDDEN, regime)
    hm = (x_regime(rng, HIDDEN, regime) * 0.5).astype(np.float32)
    g = np.array([0.3], np.float32)
    sh_blob = synth.expert_blob((5600, 1), HIDDEN, INTER, 4)
    dsh = T(sh_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    idx = torch.empty(K, dtype=torch.int32, device=dev)
    w = torch.empty(K, dtype=torch.float32, device=dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_route_decode_pool(dp, T(lg, dev), idx, w, T(x, dev), out, ws, shared=sh, shared_bits=4,
                             shared_score=T(g, dev), h_mid=T(hm, dev))
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    ri, rw = orc.route(lg[None, :], K)
    assert np.array_equal(idx.cpu().numpy(), ri[0])
    ref = orc.moe_decode([blobs[e % nb] for e in ri[0]], [bits8[e % nb] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                         shared_blob=sh_blob, shared_bits=4, shared_score=float(g[0]), h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32
