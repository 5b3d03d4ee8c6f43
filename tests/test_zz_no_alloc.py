"""The no-allocation decode entry point (fm_moe_decode_pool_noalloc) against
the workspace entry point (fm_moe_decode_pool): same kernels, so the outputs
must be bit-identical; two calls in a row, the second with a smaller input
(fewer slots, smaller expert shape), then the first shape again.  Its shape
limit is checked on the host (no GPU call is made for a rejected shape)."""
import ctypes

import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from helpers import experts

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(dev, seed, E, K, H, I, with_shared):
    import torch
    bits = [4 if e % 3 else 2 for e in range(E)]
    blobs = experts(range(seed, seed + E), bits, H, I)
    pool = fm.DevicePool(blobs, bits, H, I)
    rng = synth.rng_for(seed)
    idx = torch.empty((1, K), dtype=torch.int32, device=dev)
    w = torch.empty((1, K), dtype=torch.float32, device=dev)
    fm.route_topk(T(rng.normal(0, 1, (1, E)).astype(np.float32), dev), K, idx, w)
    x = T(synth.hidden_vec(rng, H), dev)
    hm = T(rng.normal(0, 1, H).astype(np.float32), dev)
    sh = dsh = g = None
    if with_shared:
        dsh = T(synth.expert_blob((seed, 999), H, I, 4), dev)
        sh = fm.experts_from_blob(dsh, 4, H, I)
        g = T(np.array([0.4], np.float32), dev)
    return dict(pool=pool, idx=idx, w=w, x=x, hm=hm, sh=sh, dsh=dsh, g=g, H=H, I=I, K=K)


def _run_both(dev, c):
    import torch
    H = c["H"]
    ws = fm.workspace(fm.decode_workspace_bytes(c["K"] + 1, H, c["I"]), dev)
    ref = torch.empty(H, dtype=torch.float32, device=dev)
    got = torch.full((H,), float("nan"), dtype=torch.float32, device=dev)
    rb = torch.empty(H, dtype=torch.int16, device=dev)
    gb = torch.empty(H, dtype=torch.int16, device=dev)
    fm.moe_decode_pool(c["pool"], c["idx"], c["w"], c["x"], ref, ws, shared=c["sh"], shared_bits=4,
                       shared_score=c["g"], h_mid=c["hm"], out_bf16=rb)
    fm.moe_decode_pool_noalloc(c["pool"], c["idx"], c["w"], c["x"], got, shared=c["sh"], shared_bits=4,
                               shared_score=c["g"], h_mid=c["hm"], out_bf16=gb)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
    assert torch.equal(gb, rb)


def test_noalloc_matches_workspace_entry_point(dev):
    print("[case] noalloc decode", flush=True)
    big = _case(dev, 8100, 64, 10, 4096, 1024, True)
    small = _case(dev, 8200, 16, 4, 2048, 512, False)
    _run_both(dev, big)
    _run_both(dev, small)
    _run_both(dev, big)


def test_noalloc_status_reports_bad_expert(dev):
    """An out-of-range expert index is skipped by the step and reported through
    fm_noalloc_status (read and cleared); a clean call reads 0 afterwards."""
    import torch
    print("[case] noalloc status: out-of-range expert", flush=True)
    c = _case(dev, 8300, 32, 6, 4096, 1024, True)
    assert fm.noalloc_status() == 0  # earlier calls of this process were clean
    bad = c["idx"].clone()
    bad[0, 2] = 40  # pool of 32 experts
    out = torch.empty(c["H"], dtype=torch.float32, device=dev)
    fm.moe_decode_pool_noalloc(c["pool"], bad, c["w"], c["x"], out, shared=c["sh"], shared_bits=4,
                               shared_score=c["g"], h_mid=c["hm"])
    st = fm.noalloc_status()
    assert st & 2, st  # FM_STATUS_BAD_EXPERT
    assert not st & 1, st  # no wait timed out
    # the step skipped that slot: equal to the workspace entry point with the slot skipped too
    ws = fm.workspace(fm.decode_workspace_bytes(c["K"] + 1, c["H"], c["I"]), dev)
    ref = torch.empty(c["H"], dtype=torch.float32, device=dev)
    fm.moe_decode_pool(c["pool"], bad, c["w"], c["x"], ref, ws, shared=c["sh"], shared_bits=4,
                       shared_score=c["g"], h_mid=c["hm"])
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    assert fm.noalloc_status() == 0  # cleared by the read
    _run_both(dev, c)
    assert fm.noalloc_status() == 0


def test_noalloc_rejects_oversized_shape():
    assert fm.lib().fm_noalloc_workspace_bytes() == 2 << 20
    dummy = (ctypes.c_void_p * 1)(1)
    pool = fm.ExpertPool(ctypes.cast(dummy, ctypes.c_void_p).value, 1, 1, 16384, 4096, 64)
    rc = fm.lib().fm_moe_decode_pool_noalloc(ctypes.byref(pool), 16, 1, 1, None, 4, 0, None, 1, None, 1, None, None)
    assert rc == -4  # FM_ERR_UNSUPPORTED
    assert "static one holds" in fm.lib().fm_last_error().decode()
