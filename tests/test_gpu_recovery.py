"""Recovery from a bounded-wait timeout of the one-launch decode step.

fm_moe_decode_pool_stepwise computes the step with independent launches
(no workgroup waits on another) and must match the oracle like the fused
step; fm_moe_forward_checked reads the step's status word and, on
FM_STATUS_WAIT_TIMEOUT, recomputes the step that way.  The timeout itself is
forced from the host (FMOE_FORCE_STEP_RECOVERY=1): no kernel is made to wait
or fail.  Bars as everywhere (helpers.py)."""
import os

import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_F32, experts, matrix, norm_err

pytestmark = pytest.mark.gpu

FM_STATUS_BAD_EXPERT, FM_STATUS_RECOVERED = 2, 16


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("K,shared_inter,bad", [(10, 0, False), (6, 512, False), (8, 0, True), (1, 0, False)])
def test_stepwise_decode_vs_oracle(orc, dev, K, shared_inter, bad):
    import torch
    say("stepwise decode", K, shared_inter, bad)
    E = 24
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(9800, 9800 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    si = shared_inter or INTER
    sb = synth.expert_blob((9900, si), HIDDEN, si, 4)
    dsh = T(sb, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, si)
    rng = synth.rng_for(98, K, shared_inter)
    ri, rw = orc.route(rng.normal(0, 1, (1, E)).astype(np.float32), K)
    if bad:
        ri = ri.copy()
        ri[0, 3] = E + 5  # skipped, like the one-launch step skips it
    x = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    g = np.array([-0.4], np.float32)
    ws = fm.workspace(fm.decode_workspace_bytes_ex(K, 1, HIDDEN, INTER, shared_inter), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    kw = dict(shared=sh, shared_bits=4, shared_score=T(g, dev), h_mid=T(hm, dev), shared_inter=shared_inter)
    fm.moe_decode_pool_stepwise(pool, T(ri[0], dev), T(rw[0], dev), T(x, dev), out, ws, **kw)
    torch.cuda.synchronize()
    keep = [k for k in range(K) if 0 <= ri[0, k] < E]
    ref = orc.moe_decode([blobs[ri[0, k]] for k in keep], [bits[ri[0, k]] for k in keep], rw[0][keep], x, HIDDEN,
                         INTER, shared_blob=sb, shared_bits=4, shared_score=float(g[0]), h_mid=hm,
                         shared_inter=shared_inter)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32
    # the workspace is left initialised: the one-launch step runs on it next
    out2 = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode_pool(pool, T(ri[0], dev), T(rw[0], dev), T(x, dev), out2, ws, **kw)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == (FM_STATUS_BAD_EXPERT if bad else 0)
    assert norm_err(out2.cpu().numpy() - hm, ref - hm) <= TOL_F32


def test_moe_forward_checked_recovers(orc, dev, monkeypatch):
    import torch
    say("moe_forward_checked: clean call, then a forced timeout")
    E, K = 64, 8
    bits = [4 if e % 4 else 2 for e in range(E)]
    blobs = experts(range(9950, 9950 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    Wr, sr, br = matrix(990, E, HIDDEN, 4)
    Wg, sg, bg = matrix(991, 1, HIDDEN, 4)
    shared_blob = synth.expert_blob((9990, 2), HIDDEN, INTER, 4)
    dsh = T(shared_blob, dev)
    d = [T(a, dev) for a in (Wr, sr, br, Wg, sg, bg)]
    L = fm.MoeLayer()
    L.router_w, L.router_s, L.router_b = d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr()
    L.router_bits = 4
    L.seg_w, L.seg_s, L.seg_b = d[3].data_ptr(), d[4].data_ptr(), d[5].data_ptr()
    L.seg_bits = 4
    L.shared = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    L.shared_bits = 4
    L.has_shared = 1
    L.pool = pool.c
    ws = fm.workspace(fm.moe_forward_workspace_bytes(L, K), dev)
    rng = synth.rng_for(99)
    for rep, force in enumerate([False, True, False, True]):
        hp = synth.hidden_vec(rng, HIDDEN)
        hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
        if force:
            monkeypatch.setenv("FMOE_FORCE_STEP_RECOVERY", "1")
        else:
            monkeypatch.delenv("FMOE_FORCE_STEP_RECOVERY", raising=False)
        out = torch.full((HIDDEN,), float("nan"), dtype=torch.float32, device=dev)
        st = fm.moe_forward_checked(L, K, T(hp, dev), T(hm, dev), out, ws)
        assert st == (FM_STATUS_RECOVERED | 1 if force else 0), (rep, st)
        logits = orc.matvec(4, Wr, sr, br, hp)
        score = orc.matvec(4, Wg, sg, bg, hp)[0]
        ri, rw = orc.route(logits, K)
        ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], hp, HIDDEN, INTER,
                             shared_blob=shared_blob, shared_bits=4, shared_score=float(score), h_mid=hm)
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32, rep
    assert os.environ.get("FMOE_FORCE_STEP_RECOVERY") == "1"
