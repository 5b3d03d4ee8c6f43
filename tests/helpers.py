"""Shared test helpers: seeded config data and the parity metric.

Parity metric (fixed for every floating-point check):
  norm_err(g, r) = max_i |g_i - r_i| / max_i |r_i|
fp32 outputs pass at <= 1e-3; bf16-rounded outputs at <= 2e-2.
"""
import numpy as np

from fmoe_amd import synth

TOL_F32 = 1e-3
TOL_BF16 = 2e-2

HIDDEN, INTER, GS = 4096, 1024, 64


def norm_err(g, r):
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(g - r)) / (den if den > 0 else 1.0))


def bf16_out(bits_u16):
    return synth.bf16_to_f32(np.asarray(bits_u16).view(np.uint16))


def matrix(seed, out_dim, in_dim, bits):
    rng = synth.rng_for(1000, seed)
    W, s, b = synth.quant_matrix(rng, out_dim, in_dim, bits)
    return W, s, b


def experts(seeds, bits_list, hidden=HIDDEN, inter=INTER):
    return [synth.expert_blob((2000, int(s)), hidden, inter, int(b)) for s, b in zip(seeds, bits_list)]
