"""GPU checks of expert staging (fm_expert_io.h): experts read from layer files in
the reference's format land in HBM byte-exact, and the decode/prefill kernels
fed from them match the oracle (fp32 norm_err <= 1e-3)."""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from fmoe_amd.expert_io import STORE_TIERED, ExpertStore, write_layer_files
from helpers import HIDDEN, INTER, TOL_F32, norm_err

pytestmark = pytest.mark.gpu

E = 24


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def tiered_model(tmp_path_factory):
    """Two layers of 24 full-size experts, 4-bit when (e + l) % 3 == 0 else 2-bit."""
    d = tmp_path_factory.mktemp("model")
    s4, s2 = fm.layout_of(HIDDEN, INTER, 64, 4).size, fm.layout_of(HIDDEN, INTER, 64, 2).size
    m = [[(synth.expert_blob((6000, l, e), HIDDEN, INTER, 4 if (e + l) % 3 == 0 else 2),
           4 if (e + l) % 3 == 0 else 2) for e in range(E)] for l in range(2)]
    write_layer_files(d, m, "tiered", s4, s2)
    return d, m


def test_load_layer_bytes_and_decode(orc, dev, tiered_model):
    import torch
    d, m = tiered_model
    say("load_layer + moe_decode_pool")
    with ExpertStore(d, 2, E, HIDDEN, INTER, mode=STORE_TIERED) as st:
        lp = st.load_layer(1)
        torch.cuda.synchronize()
        # every blob at its manifest offset, byte-exact; tables point there
        host = lp.storage.cpu().numpy()
        off0 = lp.base - lp.storage.data_ptr()
        tab = lp.blob_table.cpu().numpy()
        bits = lp.bits_table.cpu().numpy()
        for e in range(E):
            o, sz, b = st.extent(1, e)
            assert np.array_equal(host[off0 + o: off0 + o + sz], m[1][e][0])
            assert tab[e] == lp.base + o and bits[e] == b == m[1][e][1]
        K = 8
        rng = synth.rng_for(21)
        lg = rng.normal(0, 1, (1, E)).astype(np.float32)
        x = synth.hidden_vec(rng, HIDDEN)
        hm = rng.normal(0, 1, HIDDEN).astype(np.float32)
        ri, rw = orc.route(lg, K)
        ws = fm.workspace(fm.decode_workspace_bytes(K + 1, HIDDEN, INTER), dev)
        out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
        fm.moe_decode_pool(lp, T(ri.astype(np.int32), dev), T(rw, dev), T(x, dev), out, ws, h_mid=T(hm, dev))
        torch.cuda.synchronize()
        ref = orc.moe_decode([m[1][e][0] for e in ri[0]], [m[1][e][1] for e in ri[0]], rw[0], x, HIDDEN, INTER,
                             h_mid=hm)
        assert norm_err(out.cpu().numpy() - hm, ref - hm) <= TOL_F32


def test_load_layer_prefill(orc, dev, tiered_model):
    import torch
    d, m = tiered_model
    say("load_layer + prefill_moe")
    with ExpertStore(d, 2, E, HIDDEN, INTER) as st:
        lp = st.load_layer(0)
        Tn, K = 20, 4
        rng = synth.rng_for(22)
        idx, w = orc.route(rng.normal(0, 1, (Tn, E)).astype(np.float32), K)
        X = synth.hidden_vec(rng, HIDDEN, (Tn, HIDDEN))
        ws = fm.workspace(fm.lib().fm_prefill_moe_workspace_size(Tn, K, lp.c, 0), dev)
        out = torch.empty((Tn, HIDDEN), dtype=torch.float32, device=dev)
        fm.prefill_moe(lp, T(idx, dev), T(w, dev), T(X, dev), out, ws)
        torch.cuda.synchronize()
        ref = orc.prefill_moe(idx, w, [b for b, _ in m[0]], [b for _, b in m[0]], X, HIDDEN, INTER)
        assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


def test_stage_per_token_then_decode(orc, dev, tiered_model):
    """Three staging rounds in a row (the two pinned sets alternate and are reused),
    each followed by a decode from the staged slot buffers."""
    import torch
    d, m = tiered_model
    K = 10
    slot = fm.layout_of(HIDDEN, INTER, 64, 4).size
    bufs = torch.empty((K, slot), dtype=torch.uint8, device=dev)
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    with ExpertStore(d, 2, E, HIDDEN, INTER, io_threads=8) as st:
        for it, layer in enumerate((0, 1, 0)):
            say("stage round", it, "layer", layer)
            rng = synth.rng_for(23, it)
            ids = [int(e) for e in rng.permutation(E)[:K]]
            loaded, valid = st.stage(layer, ids, [bufs[k].data_ptr() for k in range(K)])
            assert loaded == K and valid == [1] * K
            x = synth.hidden_vec(rng, HIDDEN)
            w = rng.dirichlet(np.ones(K)).astype(np.float32)
            bl = [m[layer][e][1] for e in ids]
            ex = [fm.experts_from_blob(bufs[k], bl[k], HIDDEN, INTER) for k in range(K)]
            fm.moe_decode(ex, bl, w, T(x, dev), out, ws, HIDDEN, INTER)
            torch.cuda.synchronize()
            got = bufs.cpu().numpy()
            for k, e in enumerate(ids):
                assert np.array_equal(got[k, : m[layer][e][0].size], m[layer][e][0])
            ref = orc.moe_decode([m[layer][e][0] for e in ids], bl, w, x, HIDDEN, INTER)
            assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


def test_stage_invalid_expert_is_skipped(orc, dev, tmp_path):
    """A blob cut short on disk stages as valid = 0 and the decode skips it
    through the valid mask (gpu_encode_experts_batched, gpu_dispatch.h:461-609)."""
    import os
    import torch
    s4, s2 = fm.layout_of(HIDDEN, INTER, 64, 4).size, fm.layout_of(HIDDEN, INTER, 64, 2).size
    blobs = [synth.expert_blob((6100, e), HIDDEN, INTER, 4) for e in range(4)]
    write_layer_files(tmp_path, [[(b, 4) for b in blobs]], "4bit", s4, s2)
    f = tmp_path / "packed_experts" / "layer_00.bin"
    os.truncate(f, f.stat().st_size - 4096)
    say("stage invalid")
    K = 3
    ids = [3, 0, 1]
    bufs = torch.zeros((K, s4), dtype=torch.uint8, device=dev)
    with ExpertStore(tmp_path, 1, 4, HIDDEN, INTER) as st:
        loaded, valid = st.stage(0, ids, [bufs[k].data_ptr() for k in range(K)])
    assert loaded == 2 and valid == [0, 1, 1]
    rng = synth.rng_for(24)
    x = synth.hidden_vec(rng, HIDDEN)
    w = np.array([0.5, 0.3, 0.2], np.float32)
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    ex = [fm.experts_from_blob(bufs[k], 4, HIDDEN, INTER) for k in range(K)]
    fm.moe_decode(ex, [4] * K, w, T(x, dev), out, ws, HIDDEN, INTER, valid=valid)
    torch.cuda.synchronize()
    ref = orc.moe_decode([blobs[e] for e in ids], [4] * K, w, x, HIDDEN, INTER, valid=valid)
    assert norm_err(out.cpu().numpy(), ref) <= TOL_F32


def test_deferred_decode_overlaps_next_staging(orc, dev, tiered_model):
    """Deferred completion (layer_forward.h:1587-1602, 1658, 4033): the decode of
    token t is enqueued and NOT waited for; the expert I/O of token t+1 (preads
    + host->device copies on a second stream) runs meanwhile; then both are
    joined and checked -- decode t against the oracle, token t+1's staged bytes
    byte-exact.  Two slot-buffer sets alternate so staging never overwrites
    what an in-flight decode reads."""
    import torch
    d, m = tiered_model
    K, NT, layer = 8, 4, 0
    slot = fm.layout_of(HIDDEN, INTER, 64, 4).size
    sets = [torch.zeros((K, slot), dtype=torch.uint8, device=dev) for _ in range(2)]
    s_dec, s_io = torch.cuda.Stream(), torch.cuda.Stream()
    ws = fm.workspace(fm.decode_workspace_bytes(K, HIDDEN, INTER), dev)
    torch.cuda.synchronize()
    rng = synth.rng_for(25)
    ids = [[int(e) for e in rng.permutation(E)[:K]] for _ in range(NT)]
    xs = [synth.hidden_vec(rng, HIDDEN) for _ in range(NT)]
    ws_k = [rng.dirichlet(np.ones(K)).astype(np.float32) for _ in range(NT)]
    outs = [torch.empty(HIDDEN, dtype=torch.float32, device=dev) for _ in range(NT)]
    dec_done = [None] * NT
    with ExpertStore(d, 2, E, HIDDEN, INTER, io_threads=4) as st:
        st.stage(layer, ids[0], [sets[0][k].data_ptr() for k in range(K)], stream=s_io)
        staged = torch.cuda.Event()
        staged.record(s_io)
        for t in range(NT):
            say("deferred token", t)
            bl = [m[layer][e][1] for e in ids[t]]
            ex = [fm.experts_from_blob(sets[t % 2][k], bl[k], HIDDEN, INTER) for k in range(K)]
            s_dec.wait_event(staged)  # token t's experts are in HBM
            fm.moe_decode(ex, bl, ws_k[t], T(xs[t], dev), outs[t], ws, HIDDEN, INTER, stream=s_dec)
            dec_done[t] = torch.cuda.Event()
            dec_done[t].record(s_dec)
            if t + 1 < NT:  # next token's I/O while the decode may still run
                if t >= 1:
                    s_io.wait_event(dec_done[t - 1])  # that set was read by decode t-1
                st.stage_start(layer, ids[t + 1], [sets[(t + 1) % 2][k].data_ptr() for k in range(K)], stream=s_io)
                loaded, valid = st.stage_wait()
                assert loaded == K and valid == [1] * K
                staged = torch.cuda.Event()
                staged.record(s_io)
            # complete_deferred_experts: join, then check both results
            dec_done[t].synchronize()
            ref = orc.moe_decode([m[layer][e][0] for e in ids[t]], bl, ws_k[t], xs[t], HIDDEN, INTER)
            assert norm_err(outs[t].cpu().numpy(), ref) <= TOL_F32, t
            if t + 1 < NT:
                staged.synchronize()
                got = sets[(t + 1) % 2].cpu().numpy()
                for k, e in enumerate(ids[t + 1]):
                    assert np.array_equal(got[k, : m[layer][e][0].size], m[layer][e][0]), (t + 1, k)
    assert fm.workspace_status(ws) == 0
