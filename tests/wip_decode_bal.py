"""GPU parity of the row-split decode kernel (fm_decode_bal.hip: every CU owns
4 intermediate rows and 16 output rows of every slot; one activation hand-off
per CU, combine local to the CU).

It is the kernel of a one-token step at hidden 4096 / inter 1024 with 2 to 11
slots; FMOE_DECODE_NO_BAL=1 selects the per-CU item kernel instead.  Bars:
fp32 output norm_err <= 1e-3 from the oracle; the two kernels within 1e-5 of
each other (they differ only in the rounding of the activation group sums);
bf16 output <= 2e-2.  Covers 4-bit, 2-bit and mixed-width gate/up tiles,
steps with and without a shared expert, invalid routed slots, and the two
kernels alternating on one workspace (one epoch shared by both).
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import HIDDEN, INTER, TOL_BF16, TOL_F32, bf16_out, experts, norm_err

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["flag", "tagged"])
def _bal_on(monkeypatch, request):
    """Both activation hand-offs: one flag word per CU, or tagged activations."""
    monkeypatch.setenv("FMOE_DECODE_BAL", "1")
    monkeypatch.setenv("FMOE_BAL_TAGGED", "1" if request.param == "tagged" else "0")


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


def _bits(mode, n):
    if mode in ("4", "2"):
        return [int(mode)] * n
    return [4 if i % 3 else 2 for i in range(n)]  # mixed: tiles of two widths


def _step(orc, dev, K, mode, shared, seed, monkeypatch, valid=None, hidden=HIDDEN, inter=INTER):
    import torch
    HIDDEN, INTER = hidden, inter  # noqa: N806 (the step's shape)
    n = K + (1 if shared else 0)
    bl = _bits(mode, n)
    blobs = experts(range(9100 + 20 * seed, 9100 + 20 * seed + n), bl, HIDDEN, INTER)
    rng = synth.rng_for(91, K, seed, sum(map(ord, mode)))
    x = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    w = rng.random(K).astype(np.float32)
    w /= w.sum()
    score = float(rng.normal())
    dbl = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(d, bl[i], HIDDEN, INTER) for i, d in enumerate(dbl)]
    ws = fm.workspace(fm.decode_workspace_bytes(n, HIDDEN, INTER), dev)
    outs = {}
    for kern in ("bal", "cu"):
        if kern == "cu":
            monkeypatch.setenv("FMOE_DECODE_NO_BAL", "1")
        else:
            monkeypatch.delenv("FMOE_DECODE_NO_BAL", raising=False)
        out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
        ob = torch.empty(HIDDEN, dtype=torch.int16, device=dev)
        fm.moe_decode(ex[:K], bl[:K], w, T(x, dev), out, ws, HIDDEN, INTER, valid=valid,
                      shared=ex[K] if shared else None, shared_bits=bl[K] if shared else 4, shared_score=score,
                      h_mid=T(hm, dev), out_bf16=ob)
        torch.cuda.synchronize()
        outs[kern] = (out.cpu().numpy(), bf16_out(ob.cpu().numpy()))
    monkeypatch.delenv("FMOE_DECODE_NO_BAL", raising=False)
    assert fm.workspace_status(ws) == 0
    keep = [k for k in range(K) if valid is None or valid[k]]
    ref = orc.moe_decode([blobs[k] for k in keep], [bl[k] for k in keep], w[keep], x, HIDDEN, INTER,
                         shared_blob=blobs[K] if shared else None, shared_bits=bl[K] if shared else 4,
                         shared_score=score if shared else 0.0, h_mid=hm)
    got, gotb = outs["bal"]
    assert norm_err(got - hm, ref - hm) <= TOL_F32
    assert norm_err(gotb, ref) <= TOL_BF16
    assert norm_err(got - hm, outs["cu"][0] - hm) <= 1e-5


@pytest.mark.parametrize("mode", ["4", "2", "mixed"])
@pytest.mark.parametrize("K,shared", [(10, True), (10, False), (7, True), (4, True), (1, True), (11, False)])
def test_bal_step(orc, dev, monkeypatch, K, shared, mode):
    say("bal decode", K, shared, mode)
    _step(orc, dev, K, mode, shared, 0, monkeypatch)


@pytest.mark.parametrize("mode", ["4", "mixed"])
@pytest.mark.parametrize("K,shared", [(8, True), (5, False), (11, False)])
def test_bal_step_2048(orc, dev, monkeypatch, K, shared, mode):
    """The hidden 2048 / inter 512 shape (Qwen3.5-35B-A3B experts): 2
    intermediate and 8 output rows of every slot per CU, 4 slots a gate/up tile."""
    say("bal decode 2048/512", K, shared, mode)
    _step(orc, dev, K, mode, shared, 2, monkeypatch, hidden=2048, inter=512)


def test_bal_invalid_slots(orc, dev, monkeypatch):
    say("bal decode: invalid routed slots")
    _step(orc, dev, 10, "mixed", True, 1, monkeypatch, valid=[1, 0, 1, 1, 0, 1, 1, 1, 1, 0])


def test_bal_and_cu_alternate_on_one_workspace(orc, dev, monkeypatch):
    """Pool steps that alternate the row-split kernel, the per-CU item kernel
    and the fused-routing row-split kernel on one workspace: each is checked
    against the oracle, so a stale hand-off word from another kernel's call
    would show."""
    import torch
    say("bal / cu alternating on one workspace")
    E, K = 64, 10
    bits = [4, 2, 4, 4, 2, 4, 4, 2]
    blobs = experts(range(9300, 9300 + len(bits)), bits)
    n = len(blobs)
    dp = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    dp.blob_table = torch.from_numpy(np.array([dp.addrs[e % n] for e in range(E)], np.int64)).to(dev)
    dp.bits_table = torch.from_numpy(np.array([bits[e % n] for e in range(E)], np.uint8)).to(dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, HIDDEN, INTER, 64)
    sh_blob = synth.expert_blob((9400, 1), HIDDEN, INTER, 4)
    dsh = T(sh_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    ridx = torch.empty(K, dtype=torch.int32, device=dev)
    rw = torch.empty(K, dtype=torch.float32, device=dev)
    rng = synth.rng_for(93)
    for step, kern in enumerate(["bal", "cu", "bal", "fused", "cu", "fused", "bal", "bal"]):
        lg = rng.normal(0, 1, E).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        g = np.array([rng.normal()], np.float32)
        if kern == "cu":
            monkeypatch.setenv("FMOE_DECODE_NO_BAL", "1")
        else:
            monkeypatch.delenv("FMOE_DECODE_NO_BAL", raising=False)
        kw = dict(shared=sh, shared_bits=4, shared_score=T(g, dev))
        if kern == "fused":
            fm.moe_route_decode_pool(dp, T(lg, dev), ridx, rw, T(x, dev), out, ws, **kw)
        else:
            fm.route_topk(T(lg, dev).view(1, E), K, idx, w)
            fm.moe_decode_pool(dp, idx[0], w[0], T(x, dev), out, ws, **kw)
        torch.cuda.synchronize()
        ri, rwt = orc.route(lg[None, :], K)
        ref = orc.moe_decode([blobs[e % n] for e in ri[0]], [bits[e % n] for e in ri[0]], rwt[0], x, HIDDEN, INTER,
                             shared_blob=sh_blob, shared_bits=4, shared_score=float(g[0]))
        assert norm_err(out.cpu().numpy(), ref) <= TOL_F32, (step, kern)
        if kern == "fused":
            assert np.array_equal(ridx.cpu().numpy(), ri[0]), step
            assert np.array_equal(rw.cpu().numpy().view(np.uint32), rwt[0].view(np.uint32)), step
    monkeypatch.delenv("FMOE_DECODE_NO_BAL", raising=False)
    assert fm.workspace_status(ws) == 0


@pytest.mark.parametrize("regime", ["1e-3", "1e2", "outliers", "mixed"])
def test_bal_range(orc, dev, regime):
    """Inputs outside N(0,1) (the regimes of test_gpu_range.py) through the
    row-split kernel: the combined step and the per-expert outputs (mode 1),
    mixed bit widths, 10 routed slots + shared."""
    import torch
    from test_gpu_range import REGIMES, x_regime
    say("bal range", regime)
    K = 10
    bl = [4, 2, 4, 4, 2, 4, 2, 4, 4, 2, 4]
    blobs = experts(range(9500, 9500 + K + 1), bl)
    rng = synth.rng_for(95, REGIMES.index(regime))
    x = x_regime(rng, HIDDEN, regime)
    w = orc.route(rng.normal(0, 1, 64).astype(np.float32), K)[1][0]
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, bl[i], HIDDEN, INTER) for i, db in enumerate(dblobs)]
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    eo = torch.zeros((K + 1, HIDDEN), dtype=torch.float32, device=dev)
    fm.encode_experts_batched(ex, bl, T(x, dev), eo, ws, HIDDEN, INTER)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode(ex[:K], bl[:K], w, T(x, dev), out, ws, HIDDEN, INTER, shared=ex[K], shared_bits=bl[K],
                  shared_score=0.7)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    eon = eo.cpu().numpy()
    for k in range(K + 1):
        assert norm_err(eon[k], orc.expert_forward(blobs[k], bl[k], HIDDEN, INTER, x)) <= TOL_F32, k
    ref = orc.moe_decode(blobs[:K], bl[:K], w, x, HIDDEN, INTER, shared_blob=blobs[K], shared_bits=bl[K],
                         shared_score=0.7)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


def test_bal_norm(orc, dev):
    """The step with the next layer's RMS norm fused (a second round of tagged
    per-CU partial sums), pool-routed, tiered pool, 2-bit shared expert, three
    calls on one workspace."""
    import torch
    say("bal decode + fused norm")
    E, K = 64, 10
    bits = [4, 2, 4, 4, 2, 4, 4, 2]
    blobs = experts(range(9600, 9600 + len(bits)), bits)
    n = len(blobs)
    dp = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    dp.blob_table = torch.from_numpy(np.array([dp.addrs[e % n] for e in range(E)], np.int64)).to(dev)
    dp.bits_table = torch.from_numpy(np.array([bits[e % n] for e in range(E)], np.uint8)).to(dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, HIDDEN, INTER, 64)
    rng = synth.rng_for(96)
    shared_blob = synth.expert_blob((9700, 1), HIDDEN, INTER, 2)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 2, HIDDEN, INTER)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    normed = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    for rep in range(3):
        lg = rng.normal(0, 1, (1, E)).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
        nw = synth.bf16_bits(rng.normal(1, 0.2, HIDDEN).astype(np.float32))
        g = T(np.array([-0.4], np.float32), dev)
        fm.route_topk(T(lg, dev), K, idx, w)
        fm.moe_decode_pool_norm(dp, idx, w, T(x, dev), out, ws, T(nw.view(np.int16), dev), 1e-6, normed, shared=sh,
                                shared_bits=2, shared_score=g, h_mid=T(hm, dev))
        torch.cuda.synchronize()
        ri, rw = orc.route(lg, K)
        ref = orc.moe_decode([blobs[e % n] for e in ri[0]], [bits[e % n] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                             shared_blob=shared_blob, shared_bits=2, shared_score=-0.4, h_mid=hm)
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32, rep
        assert norm_err(normed.cpu().numpy(), orc.rms_norm(ref, nw, 1e-6)) <= TOL_F32, rep
    assert fm.workspace_status(ws) == 0


@pytest.mark.parametrize("Tn,K", [(2, 10), (4, 10), (8, 10), (3, 16)])
def test_bal_few_tokens(orc, dev, Tn, K):
    """A few tokens (fm_prefill_moe with T <= 8 runs decode steps): with the
    row-split kernel one launch per token (K = 16 + shared is beyond its 11
    slots and takes the multi-pass kernel); bit-equal to one fm_moe_decode_pool
    call per token and within the bars of the oracle."""
    import torch
    say("bal few tokens", Tn, K)
    E = 64
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(9800, 9800 + E), bits)
    pool = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    rng = synth.rng_for(98, Tn, K)
    idx, w = orc.route(rng.normal(0, 1, (Tn, E)).astype(np.float32), K)
    X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
    hm = rng.normal(0, 1, (Tn, HIDDEN)).astype(np.float32)
    g = rng.normal(0, 1, Tn).astype(np.float32)
    sh_blob = synth.expert_blob((9801, 0), HIDDEN, INTER, 4)
    dsh = T(sh_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    fm.workspace_status(ws)
    out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
    fm.prefill_moe(pool, T(idx, dev), T(w, dev), T(X, dev), out, ws, shared=sh, shared_bits=4,
                   shared_scores=T(g, dev), h_mid=T(hm, dev))
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    got = out.cpu().numpy()
    ws1 = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    for t in range(Tn):
        o = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
        fm.moe_decode_pool(pool, T(idx[t], dev), T(w[t], dev), T(X[t], dev), o, ws1, shared=sh, shared_bits=4,
                           shared_score=T(g[t:t + 1], dev), h_mid=T(hm[t], dev))
        torch.cuda.synchronize()
        assert np.array_equal(got[t], o.cpu().numpy()), t
    ref = orc.prefill_moe(idx, w, blobs, bits, X, HIDDEN, INTER, shared_blob=sh_blob, shared_bits=4,
                          shared_scores=g, h_mid=hm)
    assert norm_err(got - hm, ref - hm) <= TOL_F32
