"""Pins the CPU oracle (oracle/fm_oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the reference's own compiled CPU
kernels through the committed golden vectors (tests/golden/ref_kernels.npz,
written by tests/golden/make_golden.py from oracle/_ref), (b) the live
compiled reference when oracle/_ref is present, and (c) what the mathematics
fixes: closed forms, one-hot inputs, brute force in float64, invariants.
"""
import os

import numpy as np
import pytest

from fmoe_amd import synth
from fmoe_amd.layout import expert_offsets
from helpers import norm_err

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_kernels.npz"))


def bits_eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


# ---------------------------------------------------------------- golden ----
@pytest.mark.parametrize("name", ["mv_a", "mv_b", "mv_c"])
def test_matvec4_golden(orc, name):
    g = {k: GOLD[f"{name}_{k}"] for k in "Wsbxy"}
    assert bits_eq(orc.matvec(4, g["W"], g["s"], g["b"], g["x"]), g["y"])


def test_swiglu_golden(orc):
    assert bits_eq(orc.swiglu(GOLD["sw_g"], GOLD["sw_u"]), GOLD["sw_y"])


@pytest.mark.parametrize("name", ["sm", "sm2"])
def test_softmax_golden(orc, name):
    assert bits_eq(orc.softmax(GOLD[f"{name}_x"]), GOLD[f"{name}_y"])


@pytest.mark.parametrize("name", ["tk_a", "tk_b", "tk_c", "tk_d", "tk_e"])
def test_topk_golden(orc, name):
    idx, val = orc.topk(GOLD[f"{name}_s"], int(GOLD[f"{name}_K"]))
    assert np.array_equal(idx, GOLD[f"{name}_idx"])
    assert bits_eq(val, GOLD[f"{name}_val"])


def test_normalize_madd_bf16_golden(orc):
    assert bits_eq(orc.normalize(GOLD["nw_x"]), GOLD["nw_y"])
    d = GOLD["ma_d"].copy()
    orc.L.fmo_vec_madd(d.ctypes.data, GOLD["ma_s"].ctypes.data, float(GOLD["ma_c"]), d.size)
    assert bits_eq(d, GOLD["ma_y"])
    got = np.array([orc.L.fmo_bf16_to_f32(int(v)) for v in GOLD["bf_in"]], np.float32)
    assert bits_eq(got, GOLD["bf_f32"])
    tr = np.array([orc.L.fmo_f32_to_bf16_trunc(float(v)) for v in GOLD["tr_in"]], np.uint16)
    assert np.array_equal(tr, GOLD["tr_out"])


def test_rms_norm_golden(orc):
    assert bits_eq(orc.rms_norm(GOLD["rn_x"], GOLD["rn_w"], float(GOLD["rn_eps"])), GOLD["rn_y"])


def test_rms_norm_closed_form(orc):
    """Constant x = c with unit weights: out = c / sqrt(c^2 + eps) (float64 check);
    x and -x give mirrored outputs; scaling the weights scales the output."""
    from fmoe_amd import synth
    n, c, eps = 256, 3.0, 1e-5
    x = np.full(n, c, np.float32)
    w1 = synth.bf16_bits(np.ones(n, np.float32))
    y = orc.rms_norm(x, w1, eps)
    assert np.allclose(y, c / np.sqrt(c * c + eps), rtol=1e-6)
    rng = synth.rng_for(77)
    x = rng.normal(0, 1, n).astype(np.float32)
    w = synth.bf16_bits(rng.normal(1, 0.3, n).astype(np.float32))
    assert bits_eq(orc.rms_norm(-x, w, eps), -orc.rms_norm(x, w, eps))
    w2 = synth.bf16_bits(2 * synth.bf16_to_f32(w))  # exact doubling in bf16
    assert bits_eq(orc.rms_norm(x, w2, eps), 2 * orc.rms_norm(x, w, eps))
    ref64 = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * synth.bf16_to_f32(w)
    assert np.max(np.abs(orc.rms_norm(x, w, eps) - ref64)) < 1e-5


# ------------------------------------------------ live compiled reference ---
def test_matvec4_vs_live_reference(orc, ref):
    rng = synth.rng_for(7)
    for r, n in ((17, 64), (33, 4096), (9, 1024), (4, 8192)):
        W, s, b = synth.quant_matrix(rng, r, n, 4)
        x = synth.hidden_vec(rng, n)
        assert bits_eq(orc.matvec(4, W, s, b, x), ref.matvec4(W, s, b, x))


def test_routing_vs_live_reference(orc, ref):
    rng = synth.rng_for(8)
    for E, K in ((512, 10), (64, 8), (128, 64), (10, 10)):
        lg = rng.normal(0, 1, E).astype(np.float32)
        p = ref.softmax(lg)
        assert bits_eq(orc.softmax(lg), p)
        i1, v1 = orc.topk(p, K)
        i2, v2 = ref.topk(p, K)
        assert np.array_equal(i1, i2) and bits_eq(v1, v2)
        assert bits_eq(orc.normalize(v1), ref.normalize(v2))


# ------------------------------------------------------- mathematics -------
def test_unpack_pack_bruteforce(orc):
    for bits in (2, 4):
        per = 32 // bits
        codes = np.tile(np.arange(2 ** bits, dtype=np.uint8), per * 4)[: per * 16]
        rng = np.random.default_rng(bits)
        rng.shuffle(codes)
        packed = orc.pack(bits, codes)
        # independent LSB-first packing in numpy
        want = np.zeros(codes.size // per, dtype=np.uint64)
        for n in range(per):
            want |= codes[n::per].astype(np.uint64) << np.uint64(bits * n)
        assert np.array_equal(packed, want.astype(np.uint32))
        assert np.array_equal(orc.unpack(bits, packed), codes)
    # single-code words: code c at position n  <=>  word == c << (bits*n)
    for bits in (2, 4):
        for n in range(32 // bits):
            for c in range(2 ** bits):
                u = orc.unpack(bits, np.array([c << (bits * n)], np.uint32))
                assert u[n] == c and u.sum() == c


def test_matvec_closed_form_constant_codes(orc):
    # every code == c: out[r] = sum_g (c*s_g + b_g) * sum(x_g)
    rng = synth.rng_for(9)
    for bits in (2, 4):
        for c in range(2 ** bits):
            per = 32 // bits
            word = 0
            for n in range(per):
                word |= c << (bits * n)
            W = np.full((6, 256 // per), word, np.uint32)
            _, s, b = synth.quant_matrix(rng, 6, 256, bits)
            x = synth.hidden_vec(rng, 256)
            sf, bf = synth.bf16_to_f32(s).astype(np.float64), synth.bf16_to_f32(b).astype(np.float64)
            xs = x.astype(np.float64).reshape(4, 64).sum(1)
            want = ((c * sf + bf) * xs[None, :]).sum(1)
            assert norm_err(orc.matvec(bits, W, s, b, x), want) < 1e-5


def test_matvec_one_hot_picks_column(orc):
    rng = synth.rng_for(10)
    for bits in (2, 4):
        W, s, b = synth.quant_matrix(rng, 8, 512, bits)
        codes = orc.unpack(bits, W).reshape(8, 512).astype(np.float32)
        sf, bf = synth.bf16_to_f32(s), synth.bf16_to_f32(b)
        for j in (0, 1, 7, 8, 63, 64, 200, 511):
            x = np.zeros(512, np.float32)
            x[j] = 1.0
            want = (codes[:, j] * sf[:, j // 64] + bf[:, j // 64]).astype(np.float32)
            assert bits_eq(orc.matvec(bits, W, s, b, x), want)


def test_matvec_bruteforce_float64(orc):
    rng = synth.rng_for(11)
    for bits in (2, 4):
        W, s, b = synth.quant_matrix(rng, 2, 64, bits)
        x = synth.hidden_vec(rng, 64)
        codes = np.zeros((2, 64))
        per = 32 // bits
        for r in range(2):
            for i in range(64):
                codes[r, i] = (int(W[r, i // per]) >> (bits * (i % per))) & (2 ** bits - 1)
        w = codes * synth.bf16_to_f32(s)[:, :1] + synth.bf16_to_f32(b)[:, :1]
        want = w @ x.astype(np.float64)
        assert norm_err(orc.matvec(bits, W, s, b, x), want) < 1e-5


def test_2bit_equals_4bit_on_widened_codes(orc):
    # 2-bit codes re-packed as 4-bit nibbles: same elements, same order -> bit-identical
    rng = synth.rng_for(12)
    W2, s, b = synth.quant_matrix(rng, 16, 1024, 2)
    codes = orc.unpack(2, W2)
    W4 = orc.pack(4, codes).reshape(16, 128)
    x = synth.hidden_vec(rng, 1024)
    assert bits_eq(orc.matvec(2, W2, s, b, x), orc.matvec(4, W4, s, b, x))


def test_swiglu_closed_form(orc):
    g = np.array([0.0, 30.0, -30.0, 1.0], np.float32)
    u = np.array([5.0, 2.0, 2.0, 1.0], np.float32)
    y = orc.swiglu(g, u)
    assert y[0] == 0.0 and abs(y[1] - 60.0) < 1e-4 and abs(y[2]) < 1e-10
    assert abs(y[3] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7


def test_topk_known_answers(orc):
    idx, val = orc.topk(np.array([.1, .5, .3, .5], np.float32), 2)
    assert list(idx) == [3, 1]  # slot order, not sorted
    # ties keep the earlier index; equal later values are not inserted
    idx, _ = orc.topk(np.array([.2, .2, .2, .2], np.float32), 2)
    assert list(idx) == [0, 1]
    # K == E keeps every element in scan order
    idx, _ = orc.topk(np.array([3, 1, 2], np.float32), 3)
    assert list(idx) == [0, 1, 2]
    # the selected set is the top-K set
    rng = np.random.default_rng(0)
    s = rng.random(512).astype(np.float32)
    idx, val = orc.topk(s, 10)
    assert set(idx) == set(np.argsort(-s)[:10])


def test_route_softmax_invariants(orc):
    rng = np.random.default_rng(1)
    lg = rng.normal(0, 1, (4, 512)).astype(np.float32)
    idx, w = orc.route(lg, 10)
    for t in range(4):
        assert abs(w[t].sum() - 1.0) < 1e-6
        assert set(idx[t]) == set(np.argsort(-lg[t])[:10])
        p = np.exp(lg[t].astype(np.float64) - lg[t].max())
        p /= p.sum()
        assert norm_err(w[t], p[idx[t]] / p[idx[t]].sum()) < 1e-6


def test_expert_layout_matches_reference_constants(orc):
    # main.m:57-78 constants for the 4-bit 4096/1024/64 expert
    off, size = orc.expert_offsets(4096, 1024, 64, 4)
    assert off == [0, 2097152, 2228224, 2359296, 4456448, 4587520, 4718592, 6815744, 6946816]
    assert size == 7077888
    assert orc.expert_offsets(4096, 1024, 64, 2)[1] == 3932160
    for bits in (2, 4):
        po, ps = expert_offsets(4096, 1024, 64, bits)
        o, s = orc.expert_offsets(4096, 1024, 64, bits)
        assert list(po.values()) == o and ps == s


def test_expert_forward_composition(orc, ref):
    # gate/up/down through the reference's own matvec + SwiGLU give the same bits
    blob = synth.expert_blob((5, 1), 256, 128, 4)
    off, _ = expert_offsets(256, 128, 64, 4)
    x = synth.hidden_vec(synth.rng_for(5), 256)

    def mat(name, rows, cols):
        w = blob[off[name + "_w"]: off[name + "_w"] + rows * cols // 2].view(np.uint32).reshape(rows, cols // 8)
        s = blob[off[name + "_s"]: off[name + "_s"] + rows * cols // 32].view(np.uint16).reshape(rows, -1)
        b = blob[off[name + "_b"]: off[name + "_b"] + rows * cols // 32].view(np.uint16).reshape(rows, -1)
        return w, s, b

    g = ref.matvec4(*mat("gate", 128, 256), x)
    u = ref.matvec4(*mat("up", 128, 256), x)
    y = ref.matvec4(*mat("down", 256, 128), ref.swiglu(g, u))
    assert bits_eq(orc.expert_forward(blob, 4, 256, 128, x), y)


def test_moe_decode_reductions(orc):
    H, I = 256, 128
    blobs = [synth.expert_blob((6, e), H, I, 4) for e in range(3)]
    x = synth.hidden_vec(synth.rng_for(6), H)
    e0 = orc.expert_forward(blobs[0], 4, H, I, x)
    # all weight on one expert reduces to that expert
    assert bits_eq(orc.moe_decode(blobs[:1], [4], [1.0], x, H, I), e0)
    # invalid experts are skipped
    full = orc.moe_decode(blobs, [4, 4, 4], [0.5, 0.3, 0.2], x, H, I, valid=[1, 0, 1])
    part = orc.moe_decode([blobs[0], blobs[2]], [4, 4], [0.5, 0.2], x, H, I)
    assert bits_eq(full, part)
    # linearity in the weights and the shared term
    sh = blobs[1]
    a = orc.moe_decode(blobs[:1], [4], [1.0], x, H, I, shared_blob=sh, shared_score=0.7)
    es = orc.expert_forward(sh, 4, H, I, x)
    sg = 1.0 / (1.0 + np.exp(-0.7))
    assert norm_err(a, e0.astype(np.float64) + sg * es) < 1e-6


def test_prefill_equals_per_token_decode(orc):
    H, I, E, K, T = 256, 128, 6, 2, 3
    blobs = [synth.expert_blob((7, e), H, I, 4 if e % 2 else 2) for e in range(E)]
    bits = [4 if e % 2 else 2 for e in range(E)]
    rng = synth.rng_for(7)
    X = synth.hidden_vec(rng, H, (T, H))
    idx, w = orc.route(rng.normal(0, 1, (T, E)).astype(np.float32), K)
    g = rng.normal(0, 1, T).astype(np.float32)
    hm = rng.normal(0, 1, (T, H)).astype(np.float32)
    out = orc.prefill_moe(idx, w, blobs, bits, X, H, I, shared_blob=blobs[0], shared_bits=2,
                          shared_scores=g, h_mid=hm)
    for t in range(T):
        d = orc.moe_decode([blobs[e] for e in idx[t]], [bits[e] for e in idx[t]], w[t], X[t], H, I,
                           shared_blob=blobs[0], shared_bits=2, shared_score=g[t], h_mid=hm[t])
        assert bits_eq(out[t], d)


# ------------------------------------------- dequant GEMM (prefill checker) ---
@pytest.mark.parametrize("name", ["mv_a", "mv_b", "mv_c"])
def test_gemm_rows_equal_golden_matvec(orc, name):
    # shaders.metal:2140-2216 computes, per token column, the matvec of that
    # token: each output row of the GEMM must be the reference's matvec of its
    # token, bit for bit.  Token 1 is the golden x itself; the others are
    # derived tokens checked against the matvec oracle pinned above.
    g = {k: GOLD[f"{name}_{k}"] for k in "Wsbxy"}
    x = g["x"]
    X = np.stack([x[::-1].copy(), x, np.zeros_like(x), (x * 0.5).astype(np.float32)])
    Y = orc.gemm(4, g["W"], g["s"], g["b"], X)
    assert bits_eq(Y[1], g["y"])
    for t in range(X.shape[0]):
        assert bits_eq(Y[t], orc.matvec(4, g["W"], g["s"], g["b"], X[t]))
    # the zero token reduces to nothing: every product is (c*s + b) * 0
    assert np.all(Y[2] == 0.0)


def test_gemm_vs_live_reference_and_2bit(orc, ref):
    rng = synth.rng_for(31)
    W, s, b = synth.quant_matrix(rng, 24, 1024, 4)
    X = synth.hidden_vec(rng, 1024, (5, 1024))
    Y = orc.gemm(4, W, s, b, X)
    for t in range(5):
        assert bits_eq(Y[t], ref.matvec4(W, s, b, X[t]))
    # 2-bit: the same elements widened into nibbles give the same GEMM
    W2, s2, b2 = synth.quant_matrix(rng, 16, 1024, 2)
    W4 = orc.pack(4, orc.unpack(2, W2)).reshape(16, 128)
    assert bits_eq(orc.gemm(2, W2, s2, b2, X), orc.gemm(4, W4, s2, b2, X))
    for t in range(5):
        assert bits_eq(orc.gemm(2, W2, s2, b2, X)[t], ref.matvec4(W4, s2, b2, X[t]))


# --------------------------------------------------- f32 -> bf16 (RNE) ------
def _rne_f64(f):
    """Round-to-nearest-even onto bf16 by exhaustive choice between the two
    neighbouring bf16 values, distances measured in float64."""
    u = int(np.float32(f).view(np.uint32))
    if (u & 0x7F800000) == 0x7F800000:
        return (u >> 16) | (0x40 if (u & 0x7FFFFF) else 0)
    lo = u >> 16
    hi = lo + 1
    f64 = float(np.float32(f))
    v_lo = float(np.uint32(lo << 16).view(np.float32))
    v_hi = float(np.uint32((hi & 0xFFFF) << 16).view(np.float32)) if (hi & 0x7F80) != 0x7F80 or (hi & 0x7F) else None
    if v_hi is None:  # the next bf16 up is infinity: the value beyond the largest bf16
        v_hi = np.inf if f64 > 0 else -np.inf
    d_lo, d_hi = abs(f64 - v_lo), abs(f64 - v_hi)
    if d_lo < d_hi:
        return lo
    if d_hi < d_lo:
        return hi & 0xFFFF
    return lo if (lo & 1) == 0 else hi & 0xFFFF


def test_f32_to_bf16_rne_cases(orc):
    f = orc.L.fmo_f32_to_bf16_rne
    cases = [
        (1.0, 0x3F80),
        (-2.0, 0xC000),
        (0.0, 0x0000),
        (-0.0, 0x8000),
        (float(np.uint32(0x3F808000).view(np.float32)), 0x3F80),  # halfway, even below: stays
        (float(np.uint32(0x3F818000).view(np.float32)), 0x3F82),  # halfway, odd below: rounds up
        (float(np.uint32(0x3F808001).view(np.float32)), 0x3F81),  # just above halfway
        (float(np.uint32(0x3F807FFF).view(np.float32)), 0x3F80),  # just below halfway
        (float(np.uint32(0x3FFF8000).view(np.float32)), 0x4000),  # carry into the exponent
        (float(np.uint32(0x7F7FFFFF).view(np.float32)), 0x7F80),  # largest float rounds to inf
        (float("inf"), 0x7F80),
        (float("-inf"), 0xFF80),
        (float(np.uint32(0x00008000).view(np.float32)), 0x0000),  # subnormal halfway, even
        (float(np.uint32(0x00018000).view(np.float32)), 0x0002),  # subnormal halfway, odd
    ]
    for x, want in cases:
        assert f(x) == want, (hex(int(np.float32(x).view(np.uint32))), hex(f(x)), hex(want))
    # NaN stays NaN (quiet), sign kept
    for nan_bits in (0x7FC00000, 0x7F800001, 0xFF800001, 0x7F810000):
        r = f(float(np.uint32(nan_bits).view(np.float32)))
        assert (r & 0x7F80) == 0x7F80 and (r & 0x7F) != 0 and (r >> 15) == (nan_bits >> 31)


def test_f32_to_bf16_rne_vs_float64_brute(orc):
    rng = np.random.default_rng(5)
    u = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    u = u[(u & 0x7F800000) != 0x7F800000]
    # plus every low-half pattern near the rounding boundary of one value
    u = np.concatenate([u, 0x40490000 + np.arange(0x7F00, 0x8100, dtype=np.uint32),
                        0x40480000 + np.arange(0x7F00, 0x8100, dtype=np.uint32)])
    for v in u.view(np.float32):
        assert orc.L.fmo_f32_to_bf16_rne(float(v)) == _rne_f64(v), hex(int(np.float32(v).view(np.uint32)))
    # agrees with truncation whenever the dropped half is below halfway
    low = u[(u & 0xFFFF) < 0x8000]
    for v in low[:2000].view(np.float32):
        assert orc.L.fmo_f32_to_bf16_rne(float(v)) == orc.L.fmo_f32_to_bf16_trunc(float(v))


def test_shared_expert_own_intermediate_size(orc):
    # layer_forward.h:1099-1137 sizes the shared expert by cfg.shared_intermediate:
    # with no routed experts the step is h_mid + sigmoid(g) * shared(x) at that size
    rng = synth.rng_for(32)
    H, Is = 1024, 768
    sb = synth.expert_blob((32, 1), H, Is, 4)
    x = synth.hidden_vec(rng, H)
    hm = rng.normal(0, 1, H).astype(np.float32)
    got = orc.moe_decode([], [], np.zeros(0, np.float32), x, H, 512, shared_blob=sb, shared_bits=4,
                         shared_score=0.3, h_mid=hm, shared_inter=Is)
    so = orc.expert_forward(sb, 4, H, Is, x)
    want = hm + np.float32(orc.sigmoid(0.3)) * so
    assert norm_err(got, want) < 1e-6
    # prefill per token agrees with decode per token at the shared expert's own size
    blobs = [synth.expert_blob((32, 10 + e), H, 512, 4) for e in range(4)]
    idx, w = orc.route(rng.normal(0, 1, (3, 4)).astype(np.float32), 2)
    X = synth.hidden_vec(rng, H, (3, H))
    g = rng.normal(0, 1, 3).astype(np.float32)
    P = orc.prefill_moe(idx, w, blobs, [4] * 4, X, H, 512, shared_blob=sb, shared_bits=4, shared_scores=g,
                        shared_inter=Is)
    for t in range(3):
        d = orc.moe_decode([blobs[e] for e in idx[t]], [4, 4], w[t], X[t], H, 512, shared_blob=sb, shared_bits=4,
                           shared_score=float(g[t]), shared_inter=Is)
        assert norm_err(P[t], d) < 1e-6
