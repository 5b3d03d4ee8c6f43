"""Seeded synthetic inputs in the shapes and distributions of the benchmark
configurations (no checkpoints are available offline).

Generation (numpy PCG64; one SeedSequence per (config, expert id)):
  codes   uniform over 0..2^bits-1  -> every packed uint32 word is uniform
  4-bit   scale bf16(|N(0, 0.02)|), bias bf16(-8*scale + N(0, 0.002))
  2-bit   scale bf16(|N(0, 0.05)|), bias bf16(-1.5*scale)
  x       bf16(N(0, 1)), carried as fp32 values
bf16 rounding is round-to-nearest-even.
"""
import numpy as np

from .layout import expert_offsets


def bf16_bits(f32):
    """fp32 array -> uint16 bf16 bit patterns (round to nearest even)."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(f32):
    return bf16_to_f32(bf16_bits(f32))


def rng_for(*key):
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence(list(key))))


def quant_matrix(rng, out_dim, in_dim, bits, group_size=64):
    """(W u32 [out, in*bits/32], scales u16 [out, G], biases u16 [out, G])."""
    G = in_dim // group_size
    W = rng.integers(0, 2 ** 32, size=(out_dim, in_dim * bits // 32), dtype=np.uint32)
    if bits == 4:
        s = bf16_bits(np.abs(rng.normal(0.0, 0.02, size=(out_dim, G))).astype(np.float32))
        sf = bf16_to_f32(s)
        b = bf16_bits((-8.0 * sf + rng.normal(0.0, 0.002, size=(out_dim, G))).astype(np.float32))
    else:
        s = bf16_bits(np.abs(rng.normal(0.0, 0.05, size=(out_dim, G))).astype(np.float32))
        sf = bf16_to_f32(s)
        b = bf16_bits((-1.5 * sf).astype(np.float32))
    return W, s, b


def expert_blob(seed_key, hidden, inter, bits, group_size=64):
    """One packed expert (config.h:94-137 layout) as a uint8 array."""
    rng = rng_for(*seed_key)
    off, size = expert_offsets(hidden, inter, group_size, bits)
    blob = np.empty(size, dtype=np.uint8)
    for proj, (o, i) in (("gate", (inter, hidden)), ("up", (inter, hidden)), ("down", (hidden, inter))):
        W, s, b = quant_matrix(rng, o, i, bits, group_size)
        for suffix, arr in (("_w", W), ("_s", s), ("_b", b)):
            a = arr.reshape(-1).view(np.uint8)
            blob[off[proj + suffix]: off[proj + suffix] + a.size] = a
    return blob


def hidden_vec(rng, n, shape=None):
    """bf16-valued N(0,1) activations as fp32."""
    shape = (n,) if shape is None else shape
    return bf16_round(rng.normal(0.0, 1.0, size=shape).astype(np.float32))


def zipf_logits(rng, T, E, s=1.1):
    """logit[t,e] = ln p_{pi(e)} + Gumbel(0,1), p_r ~ r^-s: top-K of these is
    sampling without replacement proportional to a Zipf(s) law over experts."""
    ranks = np.arange(1, E + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    perm = rng.permutation(E)
    base = np.log(p)[perm]
    g = rng.gumbel(0.0, 1.0, size=(T, E))
    return (base[None, :] + g).astype(np.float32)
