"""Workspace contract of the decode hand-off (epoch tags kept on the device).

Workgroups of one decode launch hand activations and per-slot outputs to each
other as 64-bit (value, tag) words; the tag of a call is the workspace header's
epoch + 1, advanced on the device by the launch's last workgroup.  These tests
check the three ways that could go wrong:
  * a workspace whose memory held data with small integers in every high half
    (the tags a fresh sequence of calls uses) -- after fm_workspace_init the
    results must still match the oracle;
  * a decode step recorded into a HIP graph and replayed with new inputs -- each
    replay must tag its words anew (a host-side tag would be frozen in the graph);
  * one prefill workspace used alternately by the grouped GEMM (untagged
    arrays) and the few-token decode launch (tagged words): the two regions
    must not overlap.
Bars as everywhere (helpers.py): fp32 outputs norm_err <= 1e-3.
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


@pytest.fixture(scope="module")
def pool32(dev):
    E = 32
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(7000, 7000 + E), bits)
    shared_blob = synth.expert_blob((7100, 1), HIDDEN, INTER, 4)
    return blobs, bits, fm.DevicePool(blobs, bits, HIDDEN, INTER), shared_blob


def _ref(orc, blobs, bits, idx, w, x, shared_blob, score, hm=None):
    return orc.moe_decode([blobs[e] for e in idx], [bits[e] for e in idx], w, x, HIDDEN, INTER,
                          shared_blob=shared_blob, shared_bits=4, shared_score=score, h_mid=hm)


def test_poisoned_workspace_after_init(orc, dev, pool32):
    import torch
    say("poisoned workspace")
    blobs, bits, pool, shared_blob = pool32
    K = 10
    nbytes = fm.decode_workspace_bytes(K + 1, HIDDEN, INTER)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    w32 = ws.view(torch.int32)
    # every 64-bit word: low half garbage, high half 1, 2, 3, ... (the first tags)
    w32[0::2] = torch.randint(-2**31, 2**31 - 1, (w32.numel() // 2,), dtype=torch.int32, device=dev)
    w32[1::2] = (torch.arange(w32.numel() // 2, device=dev, dtype=torch.int32) % 7) + 1
    fm.workspace_init(ws)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    rng = synth.rng_for(71)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    for call in range(4):
        lg = rng.normal(0, 1, (1, 32)).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        idx = torch.empty((1, K), dtype=torch.int32, device=dev)
        w = torch.empty((1, K), dtype=torch.float32, device=dev)
        fm.route_topk(T(lg, dev), K, idx, w)
        fm.moe_decode_pool(pool, idx, w, T(x, dev), out, ws, shared=sh, shared_bits=4,
                           shared_score=T(np.array([0.1 * call], np.float32), dev))
        torch.cuda.synchronize()
        ri, rw = orc.route(lg, K)
        ref = _ref(orc, blobs, bits, ri[0], rw[0], x, shared_blob, 0.1 * call)
        assert norm_err(out.cpu().numpy(), ref) <= TOL_F32, call
    assert fm.workspace_status(ws) == 0
    # the header epoch counted the four calls (each call tags with epoch + 1)
    assert int(ws[64:68].view(torch.int32).item()) == 4


def test_graph_replay_decode_step(orc, dev, pool32):
    """Routing + decode recorded into one graph, replayed with new logits and x."""
    import torch
    say("graph replay")
    blobs, bits, pool, shared_blob = pool32
    K = 8
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    lg_in = torch.zeros((1, 32), dtype=torch.float32, device=dev)
    x_in = torch.zeros(HIDDEN, dtype=torch.float32, device=dev)
    g_in = torch.zeros(1, dtype=torch.float32, device=dev)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)

    def step():
        fm.route_topk(lg_in, K, idx, w)
        fm.moe_decode_pool(pool, idx, w, x_in, out, ws, shared=sh, shared_bits=4, shared_score=g_in)

    rng = synth.rng_for(72)
    step()  # eager warm-up (occupancy queries are cached before capture)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            step()
    torch.cuda.synchronize()
    for rep in range(4):
        lg = rng.normal(0, 1, (1, 32)).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        g = np.array([rng.normal()], np.float32)
        lg_in.copy_(T(lg, dev))
        x_in.copy_(T(x, dev))
        g_in.copy_(T(g, dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ri, rw = orc.route(lg, K)
        assert np.array_equal(idx.cpu().numpy(), ri), rep
        ref = _ref(orc, blobs, bits, ri[0], rw[0], x, shared_blob, float(g[0]))
        assert norm_err(out.cpu().numpy(), ref) <= TOL_F32, rep
        if rep == 1:  # eager work on the same workspace between replays
            step()
            torch.cuda.synchronize()
            assert norm_err(out.cpu().numpy(), ref) <= TOL_F32
    assert fm.workspace_status(ws) == 0


def test_prefill_workspace_alternating_paths(orc, dev, pool32):
    """One prefill workspace: grouped GEMM (T=40), few-token decode (T=4), and
    again, each call checked against the oracle."""
    import torch
    say("prefill alternating paths")
    blobs, bits, pool, shared_blob = pool32
    K = 6
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    ws = fm.workspace(fm.prefill_workspace_bytes(40, K, pool), dev)
    rng = synth.rng_for(73)
    for Tn in (40, 4, 40, 3, 4):
        lg = rng.normal(0, 1, (Tn, 32)).astype(np.float32)
        idx, w = orc.route(lg, K)
        X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
        g = rng.normal(0, 1, Tn).astype(np.float32)
        out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
        fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=4,
                       shared_scores=T(g, dev))
        torch.cuda.synchronize()
        ref = orc.prefill_moe(idx, w, blobs, bits, X, HIDDEN, INTER, shared_blob=shared_blob, shared_bits=4,
                              shared_scores=g)
        assert norm_err(out.cpu().numpy(), ref) <= TOL_F32, Tn
    assert fm.workspace_status(ws) == 0
