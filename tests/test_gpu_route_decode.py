"""GPU parity of fm_moe_route_decode_pool (routing + decode step in one launch)
against the oracle (cpu_softmax / cpu_topk / cpu_normalize_weights + the MoE
step) and against the two-launch path it replaces (fm_route_topk +
fm_moe_decode_pool).

Bars: routing indices bit-exact and in cpu_topk's slot order; routing weights
bit-equal to the oracle's (and so to fm_route_topk's); fp32 step output
norm_err <= 1e-3 from the oracle.
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_F32, experts, norm_err

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


def _cycled_pool(dev, E, blobs, bits, hidden, inter):
    """A pool of E experts whose blob table cycles over a few device blobs."""
    import torch
    n = len(blobs)
    dp = fm.DevicePool(blobs, bits, hidden, inter)
    dp.blob_table = torch.from_numpy(np.array([dp.addrs[e % n] for e in range(E)], np.int64)).to(dev)
    dp.bits_table = torch.from_numpy(np.array([bits[e % n] for e in range(E)], np.uint8)).to(dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, hidden, inter, 64)
    return dp


_POOLS = {}


def _pool(dev, hidden, inter, E):
    key = (hidden, inter, E)
    if key not in _POOLS:
        bits = [4, 2, 4, 4, 2, 4, 2, 4, 4, 2, 4]
        blobs = experts(range(7100, 7100 + len(bits)), bits, hidden, inter)
        _POOLS[key] = (blobs, bits, _cycled_pool(dev, E, blobs, bits, hidden, inter))
    return _POOLS[key]


def _logits(rng, E, K, kind):
    if kind == "zipf":
        return synth.zipf_logits(rng, 1, E)[0]
    if kind == "asc":
        return np.sort(rng.normal(0, 1, E)).astype(np.float32)
    if kind == "desc":
        return np.sort(rng.normal(0, 1, E))[::-1].astype(np.float32).copy()
    if kind == "dup":
        return np.round(rng.normal(0, 1, E), 1).astype(np.float32)
    lg = rng.normal(0, 1, E).astype(np.float32)
    if kind == "straddle":
        # equal logits at places K-2 .. K+2 of the descending order: a tie across
        # the K-th place, settled by cpu_topk's replacement history
        order = np.argsort(-lg, kind="stable")
        lg[order[K - 2:K + 3]] = lg[order[K - 2]]
    return lg


def _check(orc, dev, hidden, inter, E, K, kind, shared=True, shared_inter=0, seed=0):
    import torch
    blobs, bits, pool = _pool(dev, hidden, inter, E)
    n = len(blobs)
    rng = synth.rng_for(71, E, K, seed, sum(map(ord, kind)))
    lg = _logits(rng, E, K, kind)
    x = synth.hidden_vec(rng, hidden)
    hm = rng.normal(0, 1, hidden).astype(np.float32)
    g = np.array([rng.normal()], np.float32)
    si = shared_inter or inter
    sh_blob = synth.expert_blob((7200, K, si), hidden, si, 4) if shared else None
    dsh = T(sh_blob, dev) if shared else None
    sh = fm.experts_from_blob(dsh, 4, hidden, si) if shared else None
    ws_bytes = fm.decode_workspace_bytes_ex(K, 1 if shared else 0, hidden, inter, shared_inter)
    ws = fm.workspace(ws_bytes, dev)
    ws2 = fm.workspace(ws_bytes, dev)
    out = torch.empty(hidden, dtype=torch.float32, device=dev)
    out2 = torch.empty(hidden, dtype=torch.float32, device=dev)
    idx = torch.full((K,), -7, dtype=torch.int32, device=dev)
    w = torch.zeros(K, dtype=torch.float32, device=dev)
    idx2 = torch.empty((1, K), dtype=torch.int32, device=dev)
    w2 = torch.empty((1, K), dtype=torch.float32, device=dev)
    dlg, dx, dhm, dg = T(lg, dev), T(x, dev), T(hm, dev), T(g, dev)
    kw = dict(shared=sh, shared_bits=4, shared_score=dg if shared else None, h_mid=dhm, shared_inter=shared_inter)
    fm.moe_route_decode_pool(pool, dlg, idx, w, dx, out, ws, **kw)
    fm.route_topk(dlg.view(1, E), K, idx2, w2)
    fm.moe_decode_pool(pool, idx2[0], w2[0], dx, out2, ws2, **kw)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    ri, rw = orc.route(lg[None, :], K)
    gi, gw = idx.cpu().numpy(), w.cpu().numpy()
    assert np.array_equal(gi, ri[0]), (gi, ri[0])
    assert np.array_equal(gw.view(np.uint32), w2[0].cpu().numpy().view(np.uint32))
    assert np.array_equal(gw.view(np.uint32), rw[0].view(np.uint32)), (gw, rw[0])
    ref = orc.moe_decode([blobs[e % n] for e in ri[0]], [bits[e % n] for e in ri[0]], rw[0], x, hidden, inter,
                         shared_blob=sh_blob, shared_bits=4, shared_score=float(g[0]) if shared else 0.0, h_mid=hm,
                         shared_inter=shared_inter)
    got = out.cpu().numpy()
    assert norm_err(got - hm, ref - hm) <= TOL_F32
    # the two-launch path differs only by the order of the weighted sum
    assert norm_err(got - hm, out2.cpu().numpy() - hm) <= 1e-5


@pytest.mark.parametrize("E,K,kind", [
    (512, 10, "normal"), (512, 10, "zipf"), (512, 10, "straddle"), (512, 10, "dup"), (512, 10, "asc"),
    (512, 10, "desc"), (512, 1, "normal"), (512, 16, "normal"), (64, 10, "normal"), (20, 10, "normal"),
    (70, 10, "straddle"), (768, 16, "zipf"), (769, 10, "normal"), (2048, 10, "normal"), (12, 12, "normal")])
def test_route_decode_4096(orc, dev, E, K, kind):
    say("route+decode 4096/1024", E, K, kind)
    _check(orc, dev, HIDDEN, INTER, E, K, kind)


@pytest.mark.parametrize("E,K,kind,shared", [(256, 8, "normal", True), (256, 8, "straddle", True),
                                             (256, 8, "normal", False), (128, 16, "zipf", True)])
def test_route_decode_2048(orc, dev, E, K, kind, shared):
    say("route+decode 2048/512", E, K, kind, shared)
    _check(orc, dev, 2048, 512, E, K, kind, shared=shared)


def test_route_decode_no_shared_and_shared_inter(orc, dev):
    say("route+decode: no shared expert; shared expert of its own size")
    _check(orc, dev, HIDDEN, INTER, 512, 10, "normal", shared=False)
    _check(orc, dev, HIDDEN, INTER, 512, 10, "normal", shared=True, shared_inter=512)


def test_route_decode_graph_replay(orc, dev):
    """One fused step recorded into a HIP graph, replayed over new logits and
    inputs written in place: each replay matches the oracle (the hand-off tag
    lives in the workspace, so replays are not confused by earlier ones)."""
    import torch
    say("route+decode graph replay")
    blobs, bits, pool = _pool(dev, HIDDEN, INTER, 512)
    n = len(blobs)
    E, K = 512, 10
    rng = synth.rng_for(72)
    dlg = torch.zeros(E, dtype=torch.float32, device=dev)
    dx = torch.zeros(HIDDEN, dtype=torch.float32, device=dev)
    idx = torch.empty(K, dtype=torch.int32, device=dev)
    w = torch.empty(K, dtype=torch.float32, device=dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        fm.moe_route_decode_pool(pool, dlg, idx, w, dx, out, ws, stream=s)  # warm-up outside capture
        with torch.cuda.graph(g, stream=s):
            fm.moe_route_decode_pool(pool, dlg, idx, w, dx, out, ws, stream=s)
    torch.cuda.synchronize()
    for rep in range(4):
        lg = rng.normal(0, 1, E).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        dlg.copy_(T(lg, dev))
        dx.copy_(T(x, dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ri, rw = orc.route(lg[None, :], K)
        assert np.array_equal(idx.cpu().numpy(), ri[0]), rep
        ref = orc.moe_decode([blobs[e % n] for e in ri[0]], [bits[e % n] for e in ri[0]], rw[0], x, HIDDEN, INTER)
        assert norm_err(out.cpu().numpy(), ref) <= TOL_F32, rep
    assert fm.workspace_status(ws) == 0


def test_route_decode_rejects_bad_arguments(dev):
    import torch
    say("route+decode argument checks")
    _, _, pool = _pool(dev, HIDDEN, INTER, 64)
    ws = fm.workspace(fm.decode_workspace_bytes(10, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    x = torch.zeros(HIDDEN, dtype=torch.float32, device=dev)
    idx = torch.empty(10, dtype=torch.int32, device=dev)
    w = torch.empty(10, dtype=torch.float32, device=dev)
    with pytest.raises(fm.FmError):  # more logits than pool experts
        fm.moe_route_decode_pool(pool, torch.zeros(65, device=dev), idx, w, x, out, ws)
    with pytest.raises(fm.FmError):  # E < K
        fm.moe_route_decode_pool(pool, torch.zeros(9, device=dev), idx, w, x, out, ws)
