"""A shared expert with its own intermediate size (config.h:23 shared_intermediate,
layer_forward.h:1099-1137, 1265-1291) through every entry point that takes one:
fm_moe_decode, fm_moe_decode_pool(_norm, _noalloc), fm_prefill_moe (grouped and
few-token sizes) and the layer driver (fm_moe_forward / fm_moe_prefill_forward
with fm_moe_layer.shared_inter).  Bars as everywhere (helpers.py)."""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_F32, experts, matrix, norm_err

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("hidden,inter,shared_inter", [(HIDDEN, INTER, 512), (HIDDEN, INTER, 2048),
                                                       (2048, 512, 1024)])
def test_decode_shared_inter(orc, dev, hidden, inter, shared_inter):
    import torch
    say("decode shared_inter", hidden, inter, shared_inter)
    E, K = 24, 8
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(9000, 9000 + E), bits, hidden, inter)
    pool = fm.DevicePool(blobs, bits, hidden, inter)
    sb = synth.expert_blob((9100, shared_inter), hidden, shared_inter, 4)
    dsh = T(sb, dev)
    sh = fm.experts_from_blob(dsh, 4, hidden, shared_inter)
    rng = synth.rng_for(91, shared_inter)
    lg = rng.normal(0, 1, (1, E)).astype(np.float32)
    x = synth.hidden_vec(rng, hidden)
    hm = rng.normal(0, 1, hidden).astype(np.float32)
    g = np.array([0.35], np.float32)
    ri, rw = orc.route(lg, K)
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], x, hidden, inter,
                         shared_blob=sb, shared_bits=4, shared_score=float(g[0]), h_mid=hm, shared_inter=shared_inter)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    fm.route_topk(T(lg, dev), K, idx, w)
    ws = fm.workspace(fm.decode_workspace_bytes_ex(K, 1, hidden, inter, shared_inter), dev)
    out = torch.empty(hidden, dtype=torch.float32, device=dev)
    for rep in range(2):
        fm.moe_decode_pool(pool, idx, w, T(x, dev), out, ws, shared=sh, shared_bits=4, shared_score=T(g, dev),
                           h_mid=T(hm, dev), shared_inter=shared_inter)
        torch.cuda.synchronize()
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32, rep
    # host-routed form
    ex = [pool.expert(int(e)) for e in ri[0]]
    out2 = torch.empty(hidden, dtype=torch.float32, device=dev)
    fm.moe_decode(ex, [bits[e] for e in ri[0]], rw[0], T(x, dev), out2, ws, hidden, inter, shared=sh,
                  shared_bits=4, shared_score=float(g[0]), h_mid=T(hm, dev), shared_inter=shared_inter)
    torch.cuda.synchronize()
    assert norm_err(out2.cpu().numpy() - hm, ref - hm) <= TOL_F32
    # next-layer norm variant and the no-allocation entry point
    nw = synth.bf16_bits(rng.normal(1, 0.2, hidden).astype(np.float32))
    normed = torch.empty(hidden, dtype=torch.float32, device=dev)
    fm.moe_decode_pool_norm(pool, idx, w, T(x, dev), out, ws, T(nw.view(np.int16), dev), 1e-6, normed, shared=sh,
                            shared_bits=4, shared_score=T(g, dev), h_mid=T(hm, dev), shared_inter=shared_inter)
    torch.cuda.synchronize()
    assert norm_err(normed.cpu().numpy(), orc.rms_norm(ref, nw, 1e-6)) <= TOL_F32
    out3 = torch.empty(hidden, dtype=torch.float32, device=dev)
    fm.moe_decode_pool_noalloc(pool, idx, w, T(x, dev), out3, shared=sh, shared_bits=4, shared_score=T(g, dev),
                               h_mid=T(hm, dev), shared_inter=shared_inter)
    torch.cuda.synchronize()
    assert norm_err(out3.cpu().numpy() - hm, ref - hm) <= TOL_F32
    assert fm.workspace_status(ws) == 0


@pytest.mark.parametrize("Tn", [3, 40])
def test_prefill_shared_inter(orc, dev, Tn):
    import torch
    say("prefill shared_inter", Tn)
    E, K, Is = 16, 4, 512
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(9200, 9200 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    sb = synth.expert_blob((9300, Is), HIDDEN, Is, 4)
    dsh = T(sb, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, Is)
    rng = synth.rng_for(92, Tn)
    idx, w = orc.route(rng.normal(0, 1, (Tn, E)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    hm = rng.normal(0, 1, (Tn, HIDDEN)).astype(np.float32)
    g = rng.normal(0, 1, Tn).astype(np.float32)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool, Is), dev)
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=4,
                   shared_scores=T(g, dev), h_mid=T(hm, dev), shared_inter=Is)
    torch.cuda.synchronize()
    ref = orc.prefill_moe(idx, w, blobs, bits, X, HIDDEN, INTER, shared_blob=sb, shared_bits=4, shared_scores=g,
                          h_mid=hm, shared_inter=Is)
    got = out.cpu().numpy()
    for t in range(Tn):
        assert norm_err(got[t] - hm[t], ref[t] - hm[t]) <= TOL_F32, t


def test_layer_driver_shared_inter(orc, dev):
    """fm_moe_layer.shared_inter through the C layer driver, decode and prefill."""
    import torch
    say("layer shared_inter")
    E, K, Is = 32, 6, 512
    bits = [4] * E
    blobs = experts(range(9400, 9400 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    sb = synth.expert_blob((9500, Is), HIDDEN, Is, 4)
    dsh = T(sb, dev)
    Wr, sr, br = matrix(940, E, HIDDEN, 4)
    Wg, sg, bg = matrix(941, 1, HIDDEN, 4)
    d = [T(a, dev) for a in (Wr, sr, br, Wg, sg, bg)]
    L = fm.MoeLayer()
    L.router_w, L.router_s, L.router_b = d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr()
    L.router_bits = 4
    L.seg_w, L.seg_s, L.seg_b = d[3].data_ptr(), d[4].data_ptr(), d[5].data_ptr()
    L.seg_bits = 4
    L.shared = fm.experts_from_blob(dsh, 4, HIDDEN, Is)
    L.shared_bits = 4
    L.has_shared = 1
    L.pool = pool.c
    L.shared_inter = Is
    rng = synth.rng_for(94)
    hp = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    ws = fm.workspace(fm.moe_forward_workspace_bytes(L, K), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_forward(L, K, T(hp, dev), T(hm, dev), out, ws)
    torch.cuda.synchronize()
    ri, rw = orc.route(orc.matvec(4, Wr, sr, br, hp), K)
    score = orc.matvec(4, Wg, sg, bg, hp)[0]
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [4] * K, rw[0], hp, HIDDEN, INTER, shared_blob=sb,
                         shared_bits=4, shared_score=float(score), h_mid=hm, shared_inter=Is)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32
    Tn = 20
    HP = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    wsp = fm.workspace(fm.moe_prefill_workspace_bytes(L, K, Tn), dev)
    outp = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.moe_prefill_forward(L, K, Tn, T(HP, dev), None, outp, wsp)
    torch.cuda.synchronize()
    lg = orc.gemm(4, Wr, sr, br, HP)
    sc = orc.gemm(4, Wg, sg, bg, HP)[:, 0]
    pi, pw = orc.route(lg, K)
    refp = orc.prefill_moe(pi, pw, blobs, bits, HP, HIDDEN, INTER, shared_blob=sb, shared_bits=4, shared_scores=sc,
                           shared_inter=Is)
    assert norm_err(outp.cpu().numpy(), refp) <= TOL_F32


def test_alternating_shapes_one_workspace(orc, dev):
    """Calls alternating between a shared expert of the routed size and one of
    its own size (which runs as a sub-launch on the workspace tail), with
    different K, on ONE workspace and on the no-allocation path: the
    sub-launch tags from the workspace's own epoch, so no call can accept
    another's stale words; every output is checked against the oracle and the
    status words stay clean."""
    import torch
    say("alternating shared_inter / K on one workspace")
    E = 24
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(9600, 9600 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    shb = {si: synth.expert_blob((9700, si), HIDDEN, si, 4) for si in (INTER, 512, 2048)}
    dsh = {si: T(b, dev) for si, b in shb.items()}
    shw = {si: fm.experts_from_blob(dsh[si], 4, HIDDEN, si) for si in shb}
    ws = fm.workspace(max(fm.decode_workspace_bytes_ex(k, 1, HIDDEN, INTER, si)
                          for k in (3, 8, 12) for si in shb), dev)
    rng = synth.rng_for(97)
    fm.noalloc_status()  # clear what earlier tests left
    seq = [(8, 512), (12, INTER), (3, 2048), (8, INTER), (12, 512), (3, 512), (8, 2048), (12, INTER)]
    for i, (K, si) in enumerate(seq):
        lg = rng.normal(0, 1, (1, E)).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
        g = np.array([rng.normal()], np.float32)
        ri, rw = orc.route(lg, K)
        ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                             shared_blob=shb[si], shared_bits=4, shared_score=float(g[0]), h_mid=hm,
                             shared_inter=0 if si == INTER else si)
        idx, w = T(ri, dev), T(rw, dev)
        kw = dict(shared=shw[si], shared_bits=4, shared_score=T(g, dev), h_mid=T(hm, dev),
                  shared_inter=0 if si == INTER else si)
        out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
        out2 = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
        fm.moe_decode_pool(pool, idx, w, T(x, dev), out, ws, **kw)
        if fm.decode_workspace_bytes_ex(K, 1, HIDDEN, INTER, kw["shared_inter"]) <= fm.lib().fm_noalloc_workspace_bytes():
            fm.moe_decode_pool_noalloc(pool, idx, w, T(x, dev), out2, **kw)
        else:
            out2.copy_(out)
        torch.cuda.synchronize()
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32, (i, K, si)
        assert norm_err(out2.cpu().numpy() - hm, ref - hm) <= TOL_F32, (i, K, si)
    assert fm.workspace_status(ws) == 0
    assert fm.noalloc_status() == 0
