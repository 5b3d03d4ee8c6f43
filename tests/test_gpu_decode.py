"""GPU parity of the decode path through the libfmoe C ABI against the oracle.

Bars: routing indices bit-exact; fp32 outputs norm_err <= 1e-3; bf16 outputs
norm_err <= 2e-2 (norm_err = max|g - r| / max|r|, see helpers.py).
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import GS, HIDDEN, INTER, TOL_BF16, TOL_F32, bf16_out, experts, matrix, norm_err

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("bits,out_dim,in_dim", [
    (4, 4096, 4096), (4, 1024, 4096), (4, 4096, 1024), (4, 1000, 2048), (4, 7, 512), (4, 300, 8192),
    (4, 33, 3072), (2, 4096, 4096), (2, 4096, 1024), (2, 129, 8192), (4, 64, 16384)])
def test_matvec(orc, dev, bits, out_dim, in_dim):
    import torch
    say("matvec", bits, out_dim, in_dim)
    W, s, b = matrix(out_dim * 7 + in_dim, out_dim, in_dim, bits)
    x = synth.hidden_vec(synth.rng_for(3, in_dim), in_dim)
    out = torch.empty(out_dim, dtype=torch.float32, device=dev)
    fm.dequant_matvec(T(W, dev), T(s, dev), T(b, dev), T(x, dev), out, bits)
    torch.cuda.synchronize()
    ref = orc.matvec(bits, W, s, b, x)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


def test_batch_matvec_mixed(orc, dev):
    import torch
    say("batch_matvec")
    x = synth.hidden_vec(synth.rng_for(4), HIDDEN)
    specs, refs = [], []
    for i, (rows, bits) in enumerate([(512, 4), (1024, 4), (1024, 2), (1, 4), (77, 2)]):
        W, s, b = matrix(50 + i, rows, HIDDEN, bits)
        out = torch.full((rows,), float("nan"), dtype=torch.float32, device=dev)
        specs.append((T(W, dev), T(s, dev), T(b, dev), out, bits))
        refs.append(orc.matvec(bits, W, s, b, x))
    fm.batch_matvec(T(x, dev), specs)
    torch.cuda.synchronize()
    for sp, r in zip(specs, refs):
        assert norm_err(sp[3].cpu().numpy(), r) <= TOL_F32


@pytest.mark.parametrize("Tn,E,K,kind", [(1, 512, 10, "normal"), (512, 512, 10, "zipf"), (64, 512, 1, "normal"),
                                         (16, 64, 64, "normal"), (8, 10, 10, "normal"), (32, 128, 16, "dup"),
                                         (4, 4096, 8, "normal"), (3, 512, 20, "normal"),
                                         (64, 512, 10, "normal"), (4, 512, 10, "asc"), (4, 300, 16, "asc"),
                                         (4, 512, 10, "desc"), (8, 4096, 64, "normal"), (16, 70, 7, "dup"),
                                         (32, 1024, 16, "normal"), (16, 1000, 10, "normal"),
                                         (16, 1025, 10, "normal"), (4, 1024, 10, "asc"), (64, 512, 32, "normal"),
                                         (16, 65, 10, "normal"), (16, 960, 40, "zipf"), (16, 1024, 4, "dup")])
def test_route_topk(orc, dev, Tn, E, K, kind):
    import torch
    say("route", Tn, E, K, kind)
    rng = synth.rng_for(5, Tn, E, K)
    if kind == "zipf":
        lg = synth.zipf_logits(rng, Tn, E)
    elif kind in ("asc", "desc"):
        # ascending: every element is inserted (long eviction chains / overflow path); descending: none
        lg = np.sort(rng.normal(0, 1, (Tn, E)), axis=1).astype(np.float32)
        lg = lg if kind == "asc" else np.ascontiguousarray(lg[:, ::-1])
    elif kind == "dup":
        lg = np.round(rng.normal(0, 1, (Tn, E)), 1).astype(np.float32)
    else:
        lg = rng.normal(0, 1, (Tn, E)).astype(np.float32)
    idx = torch.empty((Tn, K), dtype=torch.int32, device=dev)
    w = torch.empty((Tn, K), dtype=torch.float32, device=dev)
    fm.route_topk(T(lg, dev), K, idx, w)
    torch.cuda.synchronize()
    ri, rw = orc.route(lg, K)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert norm_err(w.cpu().numpy(), rw) <= 1e-5


def _decode_inputs(seed, K, bits_list, hidden=HIDDEN, inter=INTER):
    rng = synth.rng_for(6, seed)
    blobs = experts(range(seed * 100, seed * 100 + K + 1), bits_list, hidden, inter)
    x = synth.hidden_vec(rng, hidden)
    hm = rng.normal(0, 1, hidden).astype(np.float32)
    lg = rng.normal(0, 1, 512).astype(np.float32)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    w = np.sort(p)[-K:][::-1].astype(np.float32)
    w /= w.sum()
    return blobs, x, hm, w, float(rng.normal())


@pytest.mark.parametrize("K,bitmode,hidden,inter", [(10, "4", HIDDEN, INTER), (10, "tiered", HIDDEN, INTER),
                                                     (1, "4", HIDDEN, INTER), (16, "2", HIDDEN, INTER),
                                                     (4, "4", 2048, 512), (3, "tiered", 1024, 2048),
                                                     (8, "tiered", 2048, 512), (16, "2", 2048, 512),
                                                     (1, "4", 2048, 512)])
def test_moe_decode_host_routed(orc, dev, K, bitmode, hidden, inter):
    import torch
    say("moe_decode", K, bitmode, hidden, inter)
    bl = [4 if bitmode == "4" else 2 if bitmode == "2" else (4 if i % 3 == 0 else 2) for i in range(K + 1)]
    blobs, x, hm, w, score = _decode_inputs(K + hidden // 512, K, bl, hidden, inter)
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, bl[i], hidden, inter) for i, db in enumerate(dblobs)]
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, hidden, inter), dev)
    out = torch.empty(hidden, dtype=torch.float32, device=dev)
    ob = torch.empty(hidden, dtype=torch.int16, device=dev)
    fm.moe_decode(ex[:K], bl[:K], w, T(x, dev), out, ws, hidden, inter, shared=ex[K], shared_bits=bl[K],
                  shared_score=score, h_mid=T(hm, dev), out_bf16=ob)
    torch.cuda.synchronize()
    ref = orc.moe_decode(blobs[:K], bl[:K], w, x, hidden, inter, shared_blob=blobs[K], shared_bits=bl[K],
                         shared_score=score, h_mid=hm)
    # compare the MoE contribution (out - h_mid) so the residual does not mask errors
    got = out.cpu().numpy()
    assert norm_err(got - hm, ref - hm) <= TOL_F32
    assert norm_err(bf16_out(ob.cpu().numpy()), ref) <= TOL_BF16


def test_moe_decode_valid_mask_and_no_shared(orc, dev):
    import torch
    say("moe_decode valid mask")
    K = 6
    bl = [4] * (K + 1)
    blobs, x, hm, w, _ = _decode_inputs(77, K, bl)
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, 4, HIDDEN, INTER) for db in dblobs]
    valid = [1, 0, 1, 1, 0, 1]
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode(ex[:K], bl[:K], w, T(x, dev), out, ws, HIDDEN, INTER, valid=valid)
    torch.cuda.synchronize()
    ref = orc.moe_decode(blobs[:K], bl[:K], w, x, HIDDEN, INTER, valid=valid)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("solo", [True, False])
@pytest.mark.parametrize("bits", [4, 2])
def test_moe_decode_single_expert(orc, dev, bits, solo, monkeypatch):
    """Config 1: one expert x router weight, no shared expert.  One slot runs
    on fm_decode_solo_kernel (each workgroup computes whole gate/up rows, one
    hand-off); with FMOE_DECODE_NO_SOLO=1 on the few-slot kernel's one-slot
    path (gate and up rows split over the waves).  Three calls on one
    workspace, new inputs each time, plus the per-expert output mode
    (encode_experts_batched)."""
    import torch
    if solo:
        monkeypatch.delenv("FMOE_DECODE_NO_SOLO", raising=False)
    else:
        monkeypatch.setenv("FMOE_DECODE_NO_SOLO", "1")
    say("moe_decode single expert", bits, "solo" if solo else "few-slot kernel")
    ws = fm.workspace(fm.decode_workspace_bytes(1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    ob = torch.empty(HIDDEN, dtype=torch.int16, device=dev)
    for rep in range(3):
        blobs, x, hm, w, _ = _decode_inputs(300 + 10 * bits + rep, 1, [bits, bits])
        ex = fm.experts_from_blob(T(blobs[0], dev), bits, HIDDEN, INTER)
        hmd = T(hm, dev) if rep != 1 else None
        fm.moe_decode([ex], [bits], np.array([0.37], np.float32), T(x, dev), out, ws, HIDDEN, INTER, h_mid=hmd,
                      out_bf16=ob)
        torch.cuda.synchronize()
        ref = orc.moe_decode(blobs[:1], [bits], np.array([0.37], np.float32), x, HIDDEN, INTER,
                             h_mid=hm if rep != 1 else None)
        base = hm if rep != 1 else 0.0
        assert norm_err(out.cpu().numpy() - base, ref - base) <= TOL_F32, rep
        assert norm_err(bf16_out(ob.cpu().numpy()), ref) <= TOL_BF16, rep
    assert fm.workspace_status(ws) == 0
    eo = torch.zeros((1, HIDDEN), dtype=torch.float32, device=dev)
    fm.encode_experts_batched([ex], [bits], T(x, dev), eo, ws, HIDDEN, INTER)
    torch.cuda.synchronize()
    r = orc.expert_forward(blobs[0], bits, HIDDEN, INTER, x)
    assert norm_err(eo.cpu().numpy()[0], r) <= TOL_F32


def test_encode_experts_batched_and_combine(orc, dev):
    import torch
    say("encode_experts_batched + combine")
    K = 4
    bl = [4, 2, 4, 4, 2]
    blobs, x, hm, w, score = _decode_inputs(12, K, bl)
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, bl[i], HIDDEN, INTER) for i, db in enumerate(dblobs)]
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    eo = torch.zeros((K + 1, HIDDEN), dtype=torch.float32, device=dev)
    fm.encode_experts_batched(ex, bl, T(x, dev), eo, ws, HIDDEN, INTER)
    torch.cuda.synchronize()
    eon = eo.cpu().numpy()
    for k in range(K + 1):
        r = orc.expert_forward(blobs[k], bl[k], HIDDEN, INTER, x)
        assert norm_err(eon[k], r) <= TOL_F32, k
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    sc = torch.tensor([score], dtype=torch.float32, device=dev)
    fm.moe_combine(eo, T(w, dev), out, K, h_mid=T(hm, dev), shared_out=eo[K], shared_score=sc)
    torch.cuda.synchronize()
    ref = orc.moe_decode(blobs[:K], bl[:K], w, x, HIDDEN, INTER, shared_blob=blobs[K], shared_bits=bl[K],
                         shared_score=score, h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


@pytest.mark.parametrize("bitmode", ["4", "mixed"])
def test_encode_experts_batched_eleven(orc, dev, bitmode):
    """Per-expert outputs (mode 1) with 11 experts: 704 tiles on 256 CUs, so
    192 CUs hold a third item, whose 4-bit down rows are split with item 0's
    waves; "mixed" gives third items of both widths."""
    import torch
    say("encode_experts_batched, 11 experts", bitmode)
    n = 11
    bl = [4] * n if bitmode == "4" else [4 if i % 2 == 0 else 2 for i in range(n)]
    blobs, x, _, _, _ = _decode_inputs(17, n - 1, bl)
    dblobs = [T(b, dev) for b in blobs]
    ex = [fm.experts_from_blob(db, bl[i], HIDDEN, INTER) for i, db in enumerate(dblobs)]
    ws = fm.workspace(fm.decode_workspace_bytes(n, HIDDEN, INTER), dev)
    eo = torch.full((n, HIDDEN), float("nan"), dtype=torch.float32, device=dev)
    for rep in range(2):  # the second call reuses the workspace (next epoch)
        fm.encode_experts_batched(ex, bl, T(x, dev), eo, ws, HIDDEN, INTER)
        torch.cuda.synchronize()
        eon = eo.cpu().numpy()
        for k in range(n):
            r = orc.expert_forward(blobs[k], bl[k], HIDDEN, INTER, x)
            assert norm_err(eon[k], r) <= TOL_F32, (rep, k)
    assert fm.workspace_status(ws) == 0


@pytest.fixture(scope="module")
def pool64(dev):
    """64 experts, tiered 4/2-bit (every fourth expert 4-bit), plus a shared expert."""
    E = 64
    bits = [4 if e % 4 == 0 else 2 for e in range(E)]
    blobs = experts(range(3000, 3000 + E), bits)
    return blobs, bits, fm.DevicePool(blobs, bits, HIDDEN, INTER)


def test_moe_decode_pool_device_routing(orc, dev, pool64):
    import torch
    say("moe_decode_pool")
    blobs, bits, pool = pool64
    K = 10
    rng = synth.rng_for(13)
    lg = rng.normal(0, 1, (1, 64)).astype(np.float32)
    x = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    shared_blob = synth.expert_blob((4000, 1), HIDDEN, INTER, 4)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, HIDDEN, INTER)
    g = np.float32(0.3)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    fm.route_topk(T(lg, dev), K, idx, w)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode_pool(pool, idx, w, T(x, dev), out, ws, shared=sh, shared_bits=4,
                       shared_score=T(np.array([g]), dev), h_mid=T(hm, dev))
    torch.cuda.synchronize()
    ri, rw = orc.route(lg, K)
    assert np.array_equal(idx.cpu().numpy(), ri)
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                         shared_blob=shared_blob, shared_bits=4, shared_score=float(g), h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


def test_moe_forward_layer(orc, dev, pool64):
    """Host C layer driver: router matvec -> device routing -> fused experts."""
    import torch
    say("moe_forward")
    blobs, bits, pool = pool64
    K = 8
    rng = synth.rng_for(14)
    Wr, sr, br = matrix(900, 64, HIDDEN, 4)
    Wg, sg, bg = matrix(901, 1, HIDDEN, 4)
    shared_blob = synth.expert_blob((4000, 2), HIDDEN, INTER, 4)
    dsh = T(shared_blob, dev)
    hp = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
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
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_forward(L, K, T(hp, dev), T(hm, dev), out, ws)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0  # the step's status word sits at the start of the layer workspace
    logits = orc.matvec(4, Wr, sr, br, hp)
    score = orc.matvec(4, Wg, sg, bg, hp)[0]
    ri, rw = orc.route(logits, K)
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], hp, HIDDEN, INTER,
                         shared_blob=shared_blob, shared_bits=4, shared_score=float(score), h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


@pytest.mark.parametrize("dim", [4096, 777, 1, 16384])
def test_rms_norm_vs_oracle(orc, dev, dim):
    """fm_rms_norm vs cpu_rms_norm (cpu_kernels.h:235-246); the device sums squares
    as a tree, so results agree to fp32 rounding (bar 1e-5), bf16 outputs to 2e-2."""
    import torch
    say("rms_norm", dim)
    rng = synth.rng_for(21, dim)
    x = rng.normal(0, 2, dim).astype(np.float32)
    w = synth.bf16_bits(rng.normal(1, 0.2, dim).astype(np.float32))
    out = torch.empty(dim, dtype=torch.float32, device=dev)
    ob = torch.empty(dim, dtype=torch.int16, device=dev)
    fm.rms_norm(T(x, dev), T(w.view(np.int16), dev), 1e-6, out, ob)
    torch.cuda.synchronize()
    ref = orc.rms_norm(x, w, 1e-6)
    assert norm_err(out.cpu().numpy(), ref) <= 1e-5
    assert norm_err(bf16_out(ob.cpu().numpy()), ref) <= TOL_BF16


@pytest.mark.parametrize("hidden,inter", [(HIDDEN, INTER), (2048, 512)])
def test_moe_decode_pool_norm(orc, dev, hidden, inter):
    """Decode step + the next layer's input RMS norm (fused into the combine for
    the 4096/1024 shape, a separate launch otherwise)."""
    import torch
    say("moe_decode_pool_norm", hidden, inter)
    E, K = 16, 6
    bits = [4 if e % 2 else 2 for e in range(E)]
    blobs = experts(range(6000, 6000 + E), bits, hidden, inter)
    pool = fm.DevicePool(blobs, bits, hidden, inter)
    rng = synth.rng_for(22, hidden)
    lg = rng.normal(0, 1, (1, E)).astype(np.float32)
    x = synth.hidden_vec(rng, hidden)
    hm = rng.normal(0, 1, hidden).astype(np.float32)
    w = synth.bf16_bits(rng.normal(1, 0.2, hidden).astype(np.float32))
    shared_blob = synth.expert_blob((6000, 99), hidden, inter, 4)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, hidden, inter)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    wt = torch.empty((1, K), dtype=torch.float32, device=dev)
    fm.route_topk(T(lg, dev), K, idx, wt)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, hidden, inter), dev)
    out = torch.empty(hidden, dtype=torch.float32, device=dev)
    normed = torch.empty(hidden, dtype=torch.float32, device=dev)
    for rep in range(2):  # a second call on the same workspace (stale tags must not leak)
        fm.moe_decode_pool_norm(pool, idx, wt, T(x, dev), out, ws, T(w.view(np.int16), dev), 1e-6, normed,
                                shared=sh, shared_bits=4, shared_score=T(np.array([0.2], np.float32), dev),
                                h_mid=T(hm, dev))
        torch.cuda.synchronize()
        got_out = out.cpu().numpy()
        assert norm_err(normed.cpu().numpy(), orc.rms_norm(got_out, w, 1e-6)) <= 1e-5
    ri, rw = orc.route(lg, K)
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], x, hidden, inter,
                         shared_blob=shared_blob, shared_bits=4, shared_score=0.2, h_mid=hm)
    assert norm_err(got_out - hm, ref - hm) <= TOL_F32
    assert norm_err(normed.cpu().numpy(), orc.rms_norm(ref, w, 1e-6)) <= TOL_F32


def test_moe_decode_repeated_calls_one_workspace(orc, dev):
    """Back-to-back decode steps on one workspace: each call's activation
    hand-off must only see its own words (epoch tags), never the previous
    call's, including when the slot count and bit widths change."""
    import torch
    say("moe_decode repeated calls")
    ws = fm.workspace(fm.decode_workspace_bytes(11, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    for rep, (K, bl) in enumerate([(10, [4] * 11), (10, [2, 4] * 5 + [4]), (5, [4, 2, 2, 4, 4, 2]), (10, [4] * 11)]):
        blobs, x, hm, w, score = _decode_inputs(500 + rep, K, bl)
        dblobs = [T(b, dev) for b in blobs]
        ex = [fm.experts_from_blob(db, bl[i], HIDDEN, INTER) for i, db in enumerate(dblobs)]
        fm.moe_decode(ex[:K], bl[:K], w, T(x, dev), out, ws, HIDDEN, INTER, shared=ex[K], shared_bits=bl[K],
                      shared_score=score, h_mid=T(hm, dev))
        torch.cuda.synchronize()
        ref = orc.moe_decode(blobs[:K], bl[:K], w, x, HIDDEN, INTER, shared_blob=blobs[K], shared_bits=bl[K],
                             shared_score=score, h_mid=hm)
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32, rep


def _cycled_pool(dev, E, blobs, bits):
    """A pool of E experts whose blob table cycles over the given device pool's blobs."""
    import torch
    n = len(blobs)
    dp = fm.DevicePool(blobs, bits, HIDDEN, INTER)
    dp.blob_table = torch.from_numpy(np.array([dp.addrs[e % n] for e in range(E)], np.int64)).to(dev)
    dp.bits_table = torch.from_numpy(np.array([bits[e % n] for e in range(E)], np.uint8)).to(dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, HIDDEN, INTER, 64)
    return dp


def test_moe_decode_pool_large_expert_count(orc, dev):
    """2048 experts: past the LDS-staged pool tables (1024), the slot lookup reads the
    device tables directly."""
    import torch
    say("moe_decode_pool E=2048")
    bits = [4, 2, 4, 4, 2, 4, 2, 4]
    blobs = experts(range(3500, 3508), bits)
    pool = _cycled_pool(dev, 2048, blobs, bits)
    K = 10
    rng = synth.rng_for(41)
    lg = rng.normal(0, 1, (1, 2048)).astype(np.float32)
    ri, rw = orc.route(lg, K)
    x = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.moe_decode_pool(pool, T(ri[0].astype(np.int32), dev), T(rw[0], dev), T(x, dev), out, ws, h_mid=T(hm, dev))
    torch.cuda.synchronize()
    ref = orc.moe_decode([blobs[e % 8] for e in ri[0]], [bits[e % 8] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                         h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


def test_workspace_status_bad_expert(orc, dev, pool64):
    """An expert index outside the pool is skipped and reported (FM_STATUS_BAD_EXPERT);
    a clean call reports nothing."""
    import torch
    say("workspace status")
    blobs, bits, pool = pool64
    K = 4
    rng = synth.rng_for(43)
    x = synth.hidden_vec(rng, HIDDEN)
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    fm.workspace_status(ws)  # a fresh workspace holds arbitrary bits
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    fm.moe_decode_pool(pool, T(np.array([3, 7, 11, 19], np.int32), dev), T(w, dev), T(x, dev), out, ws)
    assert fm.workspace_status(ws) == 0
    fm.moe_decode_pool(pool, T(np.array([3, 64, 11, -1], np.int32), dev), T(w, dev), T(x, dev), out, ws)
    assert fm.workspace_status(ws) == fm.STATUS_BAD_EXPERT
    ref = orc.moe_decode([blobs[3], blobs[11]], [bits[3], bits[11]], w[[0, 2]], x, HIDDEN, INTER)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32
    assert fm.workspace_status(ws) == 0  # cleared by the previous read


@pytest.mark.parametrize("bits", [4, 2])
def test_unpacked_codes_bit_exact_one_hot(orc, dev, bits):
    """With a one-hot x the dequant product is exactly one code:
    out[r] = c[r,i] * s + b, and c * s is exact in fp32, so the GPU result must
    equal the oracle's bit for bit -- for every field position of a packed word
    (all 64 positions of one group, plus a few in other groups).  Checked
    through the matvec kernel and the MFMA GEMM (one token per position)."""
    import torch
    say("one-hot codes", bits)
    out_dim, in_dim = 96, 512
    W, s, b = matrix(700 + bits, out_dim, in_dim, bits)
    pos = list(range(64, 128)) + [0, 7, 200, 333, 511]
    X = np.zeros((len(pos), in_dim), np.float32)
    for t, i in enumerate(pos):
        X[t, i] = 1.0
    Y = torch.empty((len(pos), out_dim), dtype=torch.float32, device=dev)
    ws = torch.empty(fm.lib().fm_pfb_gemm_workspace_size(len(pos), in_dim), dtype=torch.uint8, device=dev)
    fm.pfb_gemm(T(W, dev), T(s, dev), T(b, dev), T(X, dev), Y, bits, ws)
    out = torch.empty((len(pos), out_dim), dtype=torch.float32, device=dev)
    dW, ds, db = T(W, dev), T(s, dev), T(b, dev)
    for t in range(len(pos)):
        fm.dequant_matvec(dW, ds, db, T(X[t], dev), out[t], bits)
    torch.cuda.synchronize()
    ref = orc.gemm(bits, W, s, b, X)
    # the oracle itself: c * s + b of the unpacked code, element by element
    codes = orc.unpack(bits, W).reshape(out_dim, in_dim).astype(np.float32)
    sf, bf = synth.bf16_to_f32(s), synth.bf16_to_f32(b)
    want = np.stack([codes[:, i] * sf[:, i // 64] + bf[:, i // 64] for i in pos]).astype(np.float32)
    assert np.array_equal(ref.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(Y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kernel", ["cu", "three_per_cu"])
def test_decode_pool_both_mfma_kernels(orc, dev, pool64, kernel, monkeypatch):
    """The one-workgroup-per-CU decode kernel and the three-workgroups-per-CU one
    (FMOE_DECODE_NO_CU) on the same step, each against the oracle, with the
    fused next-layer norm and a tiered pool."""
    import torch
    say("decode kernel", kernel)
    if kernel == "three_per_cu":
        monkeypatch.setenv("FMOE_DECODE_NO_CU", "1")
    blobs, bits, pool = pool64
    K = 10
    rng = synth.rng_for(15, kernel == "cu")
    lg = rng.normal(0, 1, (1, 64)).astype(np.float32)
    x = synth.hidden_vec(rng, HIDDEN)
    hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
    nw = synth.bf16_bits(rng.normal(1, 0.2, HIDDEN).astype(np.float32))
    shared_blob = synth.expert_blob((4000, 3), HIDDEN, INTER, 2)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 2, HIDDEN, INTER)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    fm.route_topk(T(lg, dev), K, idx, w)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    normed = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    g = T(np.array([-0.4], np.float32), dev)
    for rep in range(3):
        fm.moe_decode_pool_norm(pool, idx, w, T(x, dev), out, ws, T(nw.view(np.int16), dev), 1e-6, normed, shared=sh,
                                shared_bits=2, shared_score=g, h_mid=T(hm, dev))
    torch.cuda.synchronize()
    ri, rw = orc.route(lg, K)
    ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                         shared_blob=shared_blob, shared_bits=2, shared_score=-0.4, h_mid=hm)
    assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32
    assert norm_err(normed.cpu().numpy(), orc.rms_norm(ref, nw, 1e-6)) <= TOL_F32
    assert fm.workspace_status(ws) == 0


@pytest.mark.parametrize("K", [8, 16])
@pytest.mark.parametrize("kernel", ["mfma", "eager"])
def test_decode_2048_512_kernels(orc, dev, monkeypatch, K, kernel):
    """The hidden 2048 / inter 512 shape (Qwen3.5-35B-A3B experts): the MFMA
    one-workgroup-per-CU kernel with 8-group units, and the v_dot2 kernel it
    replaces (FMOE_DECODE_KERNEL=eager), on a tiered pool with the fused norm,
    three calls on one workspace, each against the oracle."""
    import torch
    say("decode 2048/512", K, kernel)
    if kernel == "eager":
        monkeypatch.setenv("FMOE_DECODE_KERNEL", "eager")
    H2, I2, E = 2048, 512, 48
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(8800, 8800 + E), bits, H2, I2)
    pool = fm.DevicePool(blobs, bits, H2, I2)
    shared_blob = synth.expert_blob((8900, K), H2, I2, 4)
    dsh = T(shared_blob, dev)
    sh = fm.experts_from_blob(dsh, 4, H2, I2)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, H2, I2), dev)
    out = torch.empty(H2, dtype=torch.float32, device=dev)
    normed = torch.empty(H2, dtype=torch.float32, device=dev)
    rng = synth.rng_for(88, K, kernel == "mfma")
    nw = synth.bf16_bits(rng.normal(1, 0.2, H2).astype(np.float32))
    for rep in range(3):
        lg = rng.normal(0, 1, (1, E)).astype(np.float32)
        x = synth.hidden_vec(rng, H2)
        hm = rng.normal(0, 1, H2).astype(np.float32)
        g = np.array([rng.normal()], np.float32)
        idx = torch.empty((1, K), dtype=torch.int32, device=dev)
        w = torch.empty((1, K), dtype=torch.float32, device=dev)
        fm.route_topk(T(lg, dev), K, idx, w)
        fm.moe_decode_pool_norm(pool, idx, w, T(x, dev), out, ws, T(nw.view(np.int16), dev), 1e-6, normed,
                                shared=sh, shared_bits=4, shared_score=T(g, dev), h_mid=T(hm, dev))
        torch.cuda.synchronize()
        ri, rw = orc.route(lg, K)
        ref = orc.moe_decode([blobs[e] for e in ri[0]], [bits[e] for e in ri[0]], rw[0], x, H2, I2,
                             shared_blob=shared_blob, shared_bits=4, shared_score=float(g[0]), h_mid=hm)
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32, rep
        assert norm_err(normed.cpu().numpy(), orc.rms_norm(ref, nw, 1e-6)) <= TOL_F32, rep
    assert fm.workspace_status(ws) == 0
