"""Seeded synthetic workloads for the benchmark configurations (no datasets or
checkpoints: the weights are generated directly in packed form).

Distributions (per config):
  nibbles/bytes uniform over 0..2^bits-1 packed LSB-first into uint32 words;
  scales ~ U(0.002, 0.02) rounded to T; biases = RNE_T(-2^(bits-1) * scale)
  (exact), plus N(0, bias_noise) for the CPU-plumbing config;
  activations ~ N(0, 1) rounded to T.
16-bit floats are returned as raw uint16 bit patterns.
"""
from __future__ import annotations

import numpy as np

__all__ = ["to_bits", "from_bits", "make_weight", "make_x", "make_routing", "pack_rows"]


def to_bits(a, dtype: str) -> np.ndarray:
    """float32 -> T bit patterns, round-to-nearest-even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == "f16":
        return a.astype(np.float16).view(np.uint16)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def from_bits(b, dtype: str) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    if dtype == "bf16":
        return (b.astype(np.uint32) << 16).view(np.float32)
    return b.view(np.float16).astype(np.float32)


def pack_rows(q: np.ndarray, bits: int) -> np.ndarray:
    """[rows, K] values < 2^bits -> [rows, K*bits/32] uint32, element i at bits
    [bits*i, bits*(i+1)) of the row's little-endian bit stream."""
    q = np.ascontiguousarray(q, dtype=np.uint32)
    rows, k = q.shape
    if 32 % bits == 0:
        per = 32 // bits
        q = q.reshape(rows, k // per, per)
        shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
        return np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)
    # bits 3/5/6: assemble the bit stream explicitly
    bitpos = np.arange(k, dtype=np.int64) * bits
    words = np.zeros((rows, k * bits // 32), np.uint64)
    for j in range(bits):
        bit = (q >> j) & 1
        p = bitpos + j
        np.add.at(words, (slice(None), p // 32), (bit.astype(np.uint64) << (p % 32).astype(np.uint64)))
    return words.astype(np.uint32)


def make_weight(rng: np.random.Generator, n: int, k: int, gs: int, bits: int, dtype: str,
                bias_noise: float = 0.0):
    """Packed weight [n, k*bits/32] u32, scales/biases [n, k/gs] as T bits."""
    q = rng.integers(0, 1 << bits, size=(n, k), dtype=np.uint32)
    w_q = pack_rows(q, bits)
    s = to_bits(rng.uniform(0.002, 0.02, size=(n, k // gs)).astype(np.float32), dtype)
    sf = from_bits(s, dtype)
    bias = -float(1 << (bits - 1)) * sf
    if bias_noise:
        bias = bias + rng.normal(0.0, bias_noise, size=bias.shape).astype(np.float32)
    b = to_bits(bias.astype(np.float32), dtype)
    return w_q, s.reshape(n, k // gs), b.reshape(n, k // gs)


def make_x(rng: np.random.Generator, m: int, k: int, dtype: str) -> np.ndarray:
    return to_bits(rng.standard_normal(size=(m, k)).astype(np.float32), dtype)


def make_routing(rng: np.random.Generator, tokens: int, top_k: int, n_experts: int) -> np.ndarray:
    """[tokens, top_k] expert ids, drawn uniformly without replacement per token."""
    out = np.empty((tokens, top_k), np.uint32)
    for t in range(tokens):
        out[t] = rng.choice(n_experts, size=top_k, replace=False)
    return out
