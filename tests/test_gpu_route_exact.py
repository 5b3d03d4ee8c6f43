"""Routing on the device is bit-exact against the reference's CPU routing.

cpu_softmax / cpu_topk / cpu_normalize_weights (cpu_kernels.h:263-309) as the
oracle runs them (the reference's own code compiled here, libm expf) against:
  * fm_route_topk (the routing kernel of the two-launch step and of prefill);
  * fm_moe_route_decode_pool (routing fused into the decode step's launch),
    whose route_idx / route_w outputs are the caller's routing.
The device computes exp with the libm algorithm (fm_expf_ref, checked over
every float input by tests/test_expf.py) and the softmax sum in index order,
so indices AND weights must be bit-equal; the mismatch counts are printed.

The 10^4 seeded 512-logit vectors mix N(0,1), Zipf-skewed, rounded (equal
logits), K-th-place-straddling ties and near ties (the logits at places K-1
and K one to three ulps apart, so their exponentials are equal or adjacent
floats and the fused kernel takes its exact-probability path).
"""
import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth

pytestmark = pytest.mark.gpu

E, K, NV = 512, 10, 10000


def say(*a):
    print("[case]", *a, flush=True)


def _vectors():
    rng = synth.rng_for(8100, E, K)
    lg = rng.normal(0, 1, (NV, E)).astype(np.float32)
    kinds = np.arange(NV) % 10
    for t in range(NV):
        k = kinds[t]
        if k == 6:
            lg[t] = synth.zipf_logits(rng, 1, E)[0]
        elif k == 7:
            lg[t] = np.round(lg[t], 1)
        elif k == 8:
            order = np.argsort(-lg[t], kind="stable")
            lg[t, order[K - 2:K + 3]] = lg[t, order[K - 2]]
        elif k == 9:
            order = np.argsort(-lg[t], kind="stable")
            a = lg[t, order[K - 1]]
            steps = 1 + t % 3
            b = a
            for _ in range(steps):
                b = np.nextafter(b, np.float32(-np.inf))
            lg[t, order[K]] = b
            if t % 7 == 0:  # also near the top: p of the largest values close too
                lg[t, order[1]] = np.nextafter(lg[t, order[0]], np.float32(-np.inf))
    return lg


_VEC = {}


def _data(orc):
    if "v" not in _VEC:
        lg = _vectors()
        ri, rw = orc.route(lg, K)
        _VEC["v"] = (lg, ri, rw)
    return _VEC["v"]


def _report(name, gi, gw, ri, rw):
    idx_bad = int(np.sum(np.any(gi != ri, axis=1)))
    w_bad = int(np.sum(np.any(gw.view(np.uint32) != rw.view(np.uint32), axis=1)))
    print(f"{name}: {len(ri)} vectors, index mismatches {idx_bad}, weight bit mismatches {w_bad}", flush=True)
    return idx_bad, w_bad


def test_route_topk_bitexact_10k(orc, dev):
    import torch
    say("fm_route_topk vs oracle, 10^4 vectors of 512 logits")
    lg, ri, rw = _data(orc)
    idx = torch.empty((NV, K), dtype=torch.int32, device=dev)
    w = torch.empty((NV, K), dtype=torch.float32, device=dev)
    fm.route_topk(torch.from_numpy(lg).to(dev), K, idx, w)
    torch.cuda.synchronize()
    assert _report("fm_route_topk", idx.cpu().numpy(), w.cpu().numpy(), ri, rw) == (0, 0)


def test_fused_route_bitexact_10k(orc, dev):
    import torch
    say("fm_moe_route_decode_pool routing outputs vs oracle, 10^4 vectors of 512 logits")
    lg, ri, rw = _data(orc)
    H, I = 2048, 512  # routing does not depend on the expert shape; the smaller step is faster
    nb = 8
    blobs = [synth.expert_blob((8200, e), H, I, 4) for e in range(nb)]
    dp = fm.DevicePool(blobs, [4] * nb, H, I)
    dp.blob_table = torch.from_numpy(np.array([dp.addrs[e % nb] for e in range(E)], np.int64)).to(dev)
    dp.bits_table = torch.from_numpy(np.full(E, 4, np.uint8)).to(dev)
    dp.c = fm.ExpertPool(dp.blob_table.data_ptr(), dp.bits_table.data_ptr(), E, H, I, 64)
    rng = synth.rng_for(8101)
    x = torch.from_numpy(synth.hidden_vec(rng, H)).to(dev)
    out = torch.empty(H, dtype=torch.float32, device=dev)
    ws = fm.workspace(fm.decode_workspace_bytes_ex(K, 0, H, I, 0), dev)
    dlg = torch.from_numpy(lg).to(dev)
    idx = torch.empty((NV, K), dtype=torch.int32, device=dev)
    w = torch.empty((NV, K), dtype=torch.float32, device=dev)
    for t in range(NV):
        fm.moe_route_decode_pool(dp, dlg[t], idx[t], w[t], x, out, ws)
    torch.cuda.synchronize()
    assert fm.workspace_status(ws) == 0
    assert _report("fused routing", idx.cpu().numpy(), w.cpu().numpy(), ri, rw) == (0, 0)
