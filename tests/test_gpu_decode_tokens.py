"""GPU checks of the decode kernel's multi-pass form: several tokens' decode
steps in ONE launch (fm_prefill_moe with a few tokens), and single-token steps
with more slots than one pass of resident workgroups holds (K = 16 + shared).

Bars: against the oracle, fp32 norm_err <= 1e-3 and bf16 <= 2e-2 (helpers.py);
against one fm_moe_decode_pool launch per token, bit-equal (same per-slot
arithmetic and combine order, only the work distribution differs).
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_BF16, TOL_F32, bf16_out, experts, norm_err

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def pool64():
    E = 64
    bits = [4 if e % 3 else 2 for e in range(E)]  # tiered
    blobs = experts(range(8800, 8800 + E), bits, HIDDEN, INTER)
    return blobs, bits, fm.DevicePool(blobs, bits, HIDDEN, INTER)


def _per_token(pool, idx, w, X, hm, g, sh, dev, K):
    import torch
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    outs = []
    for t in range(idx.shape[0]):
        o = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
        fm.moe_decode_pool(pool, T(idx[t], dev), T(w[t], dev), T(X[t], dev), o, ws, shared=sh, shared_bits=4,
                           shared_score=T(g[t:t + 1], dev), h_mid=T(hm[t], dev))
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
    return np.stack(outs)


# up to 8 tokens x 17 slots in one launch; 9 tokens take the grouped GEMM
@pytest.mark.parametrize("Tn,K", [(2, 10), (4, 10), (5, 10), (8, 10), (3, 16), (8, 16), (9, 10)])
def test_few_tokens_one_launch(orc, dev, pool64, Tn, K):
    import torch
    blobs, bits, pool = pool64
    say("few tokens", Tn, K)
    rng = synth.rng_for(8801, Tn, K)
    idx, w = orc.route(rng.normal(0, 1, (Tn, 64)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    hm = rng.normal(0, 1, (Tn, HIDDEN)).astype(np.float32)
    g = rng.normal(0, 1, Tn).astype(np.float32)
    sh_blob = synth.expert_blob((8802, 0), HIDDEN, INTER, 4)
    dsh = T(sh_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    fm.workspace_status(ws)  # clears the status word of the fresh workspace
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    ob = torch.empty((Tn, HIDDEN), dtype=torch.int16, device=dev)
    for rep in range(2):  # a second call reuses the workspace (new epoch)
        out.fill_(float("nan"))
        fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=4,
                       shared_scores=T(g, dev), h_mid=T(hm, dev), out_bf16=ob)
        torch.cuda.synchronize()
        assert fm.workspace_status(ws) == 0
        got = out.cpu().numpy()
        per = _per_token(pool, idx, w, X, hm, g, sh, dev, K)
        if Tn <= 8:  # one decode launch: bit-equal to one launch per token
            assert np.array_equal(got, per), rep
        else:  # grouped GEMM: same sums, other rounding
            assert norm_err(got - hm, per - hm) <= TOL_F32, rep
    ref = orc.prefill_moe(idx, w, blobs, bits, X, HIDDEN, INTER, shared_blob=sh_blob, shared_bits=4,
                          shared_scores=g, h_mid=hm)
    assert norm_err(got - hm, ref - hm) <= TOL_F32
    assert norm_err(bf16_out(ob.cpu().numpy()), ref) <= TOL_BF16


def test_few_tokens_bad_expert_skipped(orc, dev, pool64):
    """An out-of-range index in one token's row is skipped and flagged; the other
    tokens' outputs are unaffected."""
    import torch
    blobs, bits, pool = pool64
    say("few tokens bad expert")
    Tn, K = 4, 10
    rng = synth.rng_for(8803)
    idx, w = orc.route(rng.normal(0, 1, (Tn, 64)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    bad = idx.copy()
    bad[2, 3] = 64
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    fm.workspace_status(ws)  # clears the status word of the fresh workspace
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.prefill_moe(pool, T(bad, dev), T(w, dev), T(X, dev), out, ws)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == fm.api.STATUS_BAD_EXPERT
    got = out.cpu().numpy()
    wv = w.copy()
    wv[2, 3] = 0.0  # the skipped slot contributes nothing
    ref = orc.prefill_moe(idx, wv, blobs, bits, X, HIDDEN, INTER)
    assert norm_err(got, ref) <= TOL_F32


def test_single_token_17_slots(orc, dev, pool64):
    """K = 16 routed + shared = 17 slots x 64 tiles exceed one pass of resident
    workgroups: the multi-pass instance runs the step."""
    import torch
    blobs, bits, pool = pool64
    say("single token 17 slots")
    K = 16
    rng = synth.rng_for(8804)
    idx, w = orc.route(rng.normal(0, 1, (1, 64)).astype(np.float32), K)
    x = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    sh_blob = synth.expert_blob((8805, 0), HIDDEN, INTER, 2)
    dsh = T(sh_blob, dev)
    sh = fm.experts_from_blob(dsh, 2, HIDDEN, INTER)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode_pool(pool, T(idx[0], dev), T(w[0], dev), T(x, dev), out, ws, shared=sh, shared_bits=2,
                       shared_score=T(np.array([0.3], np.float32), dev), h_mid=T(hm, dev))
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    ref = orc.moe_decode([blobs[e] for e in idx[0]], [bits[e] for e in idx[0]], w[0], x, HIDDEN, INTER,
                         shared_blob=sh_blob, shared_bits=2, shared_score=0.3, h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


@pytest.mark.parametrize("Tn,K,shared_bits,with_hmid", [(3, 8, None, False), (4, 10, 2, True), (7, 6, 4, False)])
def test_few_tokens_optional_args(orc, dev, pool64, Tn, K, shared_bits, with_hmid):
    """No shared expert (slots per token = K), a 2-bit shared expert, no h_mid:
    bit-equal to one fm_moe_decode_pool launch per token, and oracle-checked."""
    import torch
    blobs, bits, pool = pool64
    say("few tokens optional", Tn, K, shared_bits, with_hmid)
    rng = synth.rng_for(8806, Tn, K)
    idx, w = orc.route(rng.normal(0, 1, (Tn, 64)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    hm = rng.normal(0, 1, (Tn, HIDDEN)).astype(np.float32) if with_hmid else None
    g = rng.normal(0, 1, Tn).astype(np.float32)
    sh = sh_blob = dsh = None
    if shared_bits:
        sh_blob = synth.expert_blob((8807, shared_bits), HIDDEN, INTER, shared_bits)
        dsh = T(sh_blob, dev)
        sh = fm.experts_from_blob(dsh, shared_bits, HIDDEN, INTER)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    fm.workspace_status(ws)
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=shared_bits or 4,
                   shared_scores=T(g, dev) if sh is not None else None, h_mid=T(hm, dev) if with_hmid else None)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    got = out.cpu().numpy()
    dws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    o = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    for t in range(Tn):
        fm.moe_decode_pool(pool, T(idx[t], dev), T(w[t], dev), T(X[t], dev), o, dws, shared=sh,
                           shared_bits=shared_bits or 4, shared_score=T(g[t:t + 1], dev) if sh is not None else None,
                           h_mid=T(hm[t], dev) if with_hmid else None)
        torch.cuda.synchronize()
        assert np.array_equal(got[t], o.cpu().numpy()), t
    ref = orc.prefill_moe(idx, w, blobs, bits, X, HIDDEN, INTER, shared_blob=sh_blob, shared_bits=shared_bits or 4,
                          shared_scores=g if sh is not None else None, h_mid=hm)
    assert norm_err(got, ref) <= TOL_F32
