"""GPU parity of the prefill path (grouped MFMA dequant-GEMM) against the oracle.

Bars: fp32 outputs norm_err <= 1e-3, bf16 outputs <= 2e-2 (helpers.py).  At the
full config-3 size (512 tokens, 512 experts) the CPU oracle would take ~1 min for
every token, so there sampled tokens are checked against the oracle and against
the decode path on the same routing.
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_BF16, TOL_F32, bf16_out, experts, matrix, norm_err

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("bits,N,out_dim,in_dim", [
    (4, 1, 512, 4096), (4, 7, 300, 1024), (4, 16, 1024, 4096), (4, 33, 64, 512), (2, 20, 256, 1024),
    (4, 100, 512, 4096), (2, 5, 4096, 1024)])
def test_pfb_gemm(orc, dev, bits, N, out_dim, in_dim):
    import torch
    say("pfb_gemm", bits, N, out_dim, in_dim)
    W, s, b = matrix(77 + N + out_dim, out_dim, in_dim, bits)
    rng = synth.rng_for(8, N, in_dim)
    X = rng.normal(0, 1, (N, in_dim)).astype(np.float32)  # not bf16-exact: exercises the hi/lo split
    Y = torch.empty((N, out_dim), dtype=torch.float32, device=dev)
    ws = torch.empty(fm.lib().fm_pfb_gemm_workspace_size(N, in_dim), dtype=torch.uint8, device=dev)
    fm.pfb_gemm(T(W, dev), T(s, dev), T(b, dev), T(X, dev), Y, bits, ws)
    torch.cuda.synchronize()
    ref = orc.gemm(bits, W, s, b, X)
    assert norm_err(Y.cpu().numpy(), ref) <= TOL_F32


def _prefill_case(orc, dev, E, Tn, K, H, I, bits_of, seed, zipf=False, shared_bits=4):
    import torch
    bits = [bits_of(e) for e in range(E)]
    blobs = experts(range(seed * 1000, seed * 1000 + E), bits, H, I)
    pool = fm.DevicePool(blobs, bits, H, I)
    rng = synth.rng_for(9, seed)
    lg = synth.zipf_logits(rng, Tn, E) if zipf else rng.normal(0, 1, (Tn, E)).astype(np.float32)
    idx, w = orc.route(lg, K)
    X = synth.hidden_vec(rng, H, (Tn, H))
    hm = rng.normal(0, 1, (Tn, H)).astype(np.float32)
    g = rng.normal(0, 1, Tn).astype(np.float32)
    shared_blob = synth.expert_blob((seed, 99999), H, I, shared_bits)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, shared_bits, H, I)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    out = torch.empty((Tn, H), dtype=torch.float32, device=dev)
    ob = torch.empty((Tn, H), dtype=torch.int16, device=dev)
    fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=shared_bits,
                   shared_scores=T(g, dev), h_mid=T(hm, dev), out_bf16=ob)
    torch.cuda.synchronize()
    return dict(blobs=blobs, bits=bits, pool=pool, idx=idx, w=w, X=X, hm=hm, g=g, shared_blob=shared_blob,
                sh=sh, dsh=dsh, out=out.cpu().numpy(), ob=ob.cpu().numpy())


@pytest.mark.parametrize("E,Tn,K,H,I,mode", [(16, 40, 4, 1024, 512, "4"), (12, 23, 3, 1024, 512, "tiered"),
                                             (8, 5, 8, 2048, 256, "2"), (64, 12, 10, HIDDEN, INTER, "4"),
                                             # gate/up streamed (20 input groups: not whole 8-group
                                             # pieces), down resident with per-group scale loads
                                             (10, 30, 3, 1280, 768, "tiered"),
                                             # ~75 entries per expert: many 16-entry chunks per expert
                                             (16, 200, 6, 1024, 512, "4")])
def test_prefill_moe_vs_oracle(orc, dev, E, Tn, K, H, I, mode):
    say("prefill", E, Tn, K, H, I, mode)
    bits_of = (lambda e: 4) if mode == "4" else (lambda e: 2) if mode == "2" else (lambda e: 4 if e % 3 else 2)
    r = _prefill_case(orc, dev, E, Tn, K, H, I, bits_of, seed=E + Tn)
    ref = orc.prefill_moe(r["idx"], r["w"], r["blobs"], r["bits"], r["X"], H, I, shared_blob=r["shared_blob"],
                          shared_bits=4, shared_scores=r["g"], h_mid=r["hm"])
    assert norm_err(r["out"] - r["hm"], ref - r["hm"]) <= TOL_F32
    assert norm_err(bf16_out(r["ob"]), ref) <= TOL_BF16


@pytest.mark.parametrize("Tn,K", [(2, 10), (8, 16), (5, 7)])
def test_prefill_few_tokens_multi_pass(orc, dev, Tn, K):
    """2-8 tokens at the 4096 / 1024 shape: every token's slots in one
    multi-pass decode launch (8 x (16 + shared) = 136 slots: 17 passes of the
    512-workgroup grid, each pass loading the next one's gate/up rows)."""
    say("prefill few tokens", Tn, K)
    r = _prefill_case(orc, dev, 64, Tn, K, HIDDEN, INTER, lambda e: 4 if e % 4 == 0 else 2, seed=90 + Tn)
    ref = orc.prefill_moe(r["idx"], r["w"], r["blobs"], r["bits"], r["X"], HIDDEN, INTER,
                          shared_blob=r["shared_blob"], shared_bits=4, shared_scores=r["g"], h_mid=r["hm"])
    assert norm_err(r["out"] - r["hm"], ref - r["hm"]) <= TOL_F32
    assert norm_err(bf16_out(r["ob"]), ref) <= TOL_BF16


def test_prefill_config3_vs_decode(orc, dev):
    """Full config 3: 512 tokens, 512 experts, top-10 Zipf(1.1) routing + shared.
    Sampled tokens' prefill output must match the oracle (the reference's
    per-token arithmetic, batched_prefill.h:241-308) and the decode path on the
    same routing (a bug shared by both HIP paths would fail the first)."""
    import torch
    say("prefill config3")
    E, Tn, K = 512, 512, 10
    r = _prefill_case(orc, dev, E, Tn, K, HIDDEN, INTER, lambda e: 4, seed=3, zipf=True)
    counts = np.bincount(r["idx"].reshape(-1), minlength=E)
    assert counts.max() > 100  # skewed
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    for t in (0, 1, 77, 255, 511):
        ex = [r["pool"].expert(int(e)) for e in r["idx"][t]]
        fm.moe_decode(ex, [4] * K, r["w"][t], T(r["X"][t], dev), out, ws, HIDDEN, INTER, shared=r["sh"],
                      shared_bits=4, shared_score=float(r["g"][t]), h_mid=T(r["hm"][t], dev))
        torch.cuda.synchronize()
        d = out.cpu().numpy()
        assert norm_err(r["out"][t] - r["hm"][t], d - r["hm"][t]) <= TOL_F32, t
        ref = orc.moe_decode([r["blobs"][e] for e in r["idx"][t]], [4] * K, r["w"][t], r["X"][t], HIDDEN, INTER,
                             shared_blob=r["shared_blob"], shared_bits=4, shared_score=float(r["g"][t]),
                             h_mid=r["hm"][t])
        assert norm_err(r["out"][t] - r["hm"][t], ref - r["hm"][t]) <= TOL_F32, t


def test_moe_prefill_forward_layer(orc, dev):
    """Host C layer driver for prefill: router GEMM -> routing -> grouped experts."""
    import torch
    say("moe_prefill_forward")
    E, Tn, K, H, I = 32, 24, 4, 1024, 512
    bits = [4] * E
    blobs = experts(range(5000, 5000 + E), bits, H, I)
    pool = fm.DevicePool(blobs, bits, H, I)
    rng = synth.rng_for(15)
    Wr, sr, br = matrix(910, E, H, 4)
    Wg, sg, bg = matrix(911, 1, H, 4)
    shared_blob = synth.expert_blob((5001, 1), H, I, 4)
    dsh = T(shared_blob, dev)
    X = synth.hidden_vec(rng, H, (Tn, H))
    hm = rng.normal(0, 1, (Tn, H)).astype(np.float32)
    d = [T(a, dev) for a in (Wr, sr, br, Wg, sg, bg)]
    L = fm.MoeLayer()
    L.router_w, L.router_s, L.router_b = d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr()
    L.router_bits = 4
    L.seg_w, L.seg_s, L.seg_b = d[3].data_ptr(), d[4].data_ptr(), d[5].data_ptr()
    L.seg_bits = 4
    L.shared = fm.experts_from_blob(dsh, 4, H, I)
    L.shared_bits = 4
    L.has_shared = 1
    L.pool = pool.c
    ws = fm.workspace(fm.moe_prefill_workspace_bytes(L, K, Tn), dev)
    out = torch.empty((Tn, H), dtype=torch.float32, device=dev)
    fm.moe_prefill_forward(L, K, Tn, T(X, dev), T(hm, dev), out, ws)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    logits = orc.gemm(4, Wr, sr, br, X)
    scores = orc.gemm(4, Wg, sg, bg, X)[:, 0]
    idx, w = orc.route(logits, K)
    ref = orc.prefill_moe(idx, w, blobs, bits, X, H, I, shared_blob=shared_blob, shared_bits=4,
                          shared_scores=scores, h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


@pytest.mark.parametrize("E", [2048, 3000, 4096, 5000])
def test_prefill_large_expert_count(orc, dev, E):
    """Large pools (blob table cycling over 8 blobs) through the grouped GEMM
    path: 2048 (pool table staged in LDS by the lists kernel), 3000 and 4096
    (the staged table would not fit beside the lists: read from memory) and
    5000 (beyond the staging range)."""
    import torch
    say("prefill E", E)
    Tn, K = 40, 6
    bits8 = [4, 2, 4, 4, 2, 4, 2, 4]
    blobs8 = experts(range(3600, 3608), bits8)
    dp = fm.DevicePool(blobs8, bits8, HIDDEN, INTER)
    dp.blob_table = T(np.array([dp.addrs[e % 8] for e in range(E)], np.int64), dev)
    dp.bits_table = T(np.array([bits8[e % 8] for e in range(E)], np.uint8), dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, HIDDEN, INTER, 64)
    rng = synth.rng_for(42)
    idx, w = orc.route(rng.normal(0, 1, (Tn, E)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, dp), dev)
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.prefill_moe(dp, T(idx, dev), T(w, dev), T(X, dev), out, ws)
    torch.cuda.synchronize()
    ref = orc.prefill_moe(idx, w, [blobs8[e % 8] for e in range(E)], [bits8[e % 8] for e in range(E)], X, HIDDEN,
                          INTER)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


def test_prefill_status_bad_expert(orc, dev):
    import torch
    say("prefill status")
    E, Tn, K = 16, 24, 3
    bits = [4] * E
    blobs = experts(range(3700, 3700 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    rng = synth.rng_for(44)
    idx, w = orc.route(rng.normal(0, 1, (Tn, E)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.workspace_status(ws)
    fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws)
    assert fm.workspace_status(ws) == 0
    bad = idx.copy()
    bad[5, 1] = E + 3
    fm.prefill_moe(pool, T(bad, dev), T(w, dev), T(X, dev), out, ws)
    assert fm.workspace_status(ws) == fm.STATUS_BAD_EXPERT
