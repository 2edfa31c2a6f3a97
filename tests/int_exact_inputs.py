"""Inputs on which every fp32 operation of the matrix path is exact.

The integer stage of the path (quant_primitives.cuh:28-32: int32 group dots
seeded with sum8) is only visible through fp16 outputs.  With ordinary
inputs those outputs carry fp32 rounding in an order that differs between
the GPU and the CPU golden, so parity is a tolerance and a group dot that is
off by one can hide inside it.  The inputs built here remove all rounding:

* activations are fp16 values q * 2^-k with integer |q| <= 127 and, in every
  128-group, one element of magnitude exactly 127 * 2^-k, so the Q8_1
  quantizer (quant_primitives.cuh:37-89) yields d = 2^-k, q8 = q, exactly;
* weight scales are powers of two, so dequantized weights and every product
  dot * (w_s * x_s) are exact in fp32;
* the sum of |terms| of every output stays below 2^24 units of the smallest
  term granularity, so fp32 accumulation in any order is exact.

Every output is then RNE(exact value) on both sides, and the GPU must match
the oracle bit for bit.  In the sparse variant most outputs are below 2048
granularity units, so a change of one in any group dot changes the fp16
output: `visible_fraction` measures that.
"""
from __future__ import annotations

import numpy as np

GROUP = 128


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """q[N, K] in [0, 15] -> uint32[N, K/8] in the exporter's order
    (tools/export_qwen25.py:59-72: element 8w+j at bits j=0:0, 4:4, 1:8, 5:12,
    2:16, 6:20, 3:24, 7:28)."""
    N, K = q.shape
    q = q.astype(np.uint32).reshape(N, K // 8, 8)
    return (q[..., 0] | (q[..., 4] << 4) | (q[..., 1] << 8) | (q[..., 5] << 12)
            | (q[..., 2] << 16) | (q[..., 6] << 20) | (q[..., 3] << 24) | (q[..., 7] << 28))


def activation(rng, K: int, sparse: bool, exps=(0, 1), main=None):
    """fp16[K] with Q8_1 scale 2^-k per group (k drawn from `exps`) and
    integer q8 values; returns (x, main) where main[g] is the position of the
    group's |q| = 127 element (drawn, or the given one: rows of a prefill
    activation share them so that the sparse weights keep every row small)."""
    G = K // GROUP
    q = np.zeros(K, np.int64)
    if sparse:
        nz = rng.random(K) < 0.25
        q[nz] = rng.integers(-3, 4, nz.sum())
    else:
        q[:] = rng.integers(-127, 128, K)
    if main is None:
        main = rng.integers(0, GROUP, G) + np.arange(G) * GROUP
    q[main] = np.where(rng.random(G) < 0.5, -127, 127)
    k = rng.choice(np.asarray(exps), G)
    x = q.astype(np.float64) * (2.0 ** -np.repeat(k, GROUP))
    x16 = x.astype(np.float16)
    assert np.array_equal(x16.astype(np.float64), x)
    return x16, main


def weights(rng, N: int, K: int, sparse_main=None, exps=(0, 1, 2)):
    """Nibbles uniform in [0, 15] and fp16 scales 2^-e per (row, group).
    With `sparse_main` (positions of the activation's 127 elements) those
    columns get nibbles 7..9 only, which keeps sparse-variant outputs small."""
    q = rng.integers(0, 16, (N, K))
    if sparse_main is not None:
        q[:, sparse_main] = rng.integers(7, 10, (N, len(sparse_main)))
    e = rng.choice(np.asarray(exps), (N, K // GROUP))
    sc = (2.0 ** -e).astype(np.float16)
    return pack_nibbles(q), sc, q


def swiglu_weights(rng, I: int, K: int, x16: np.ndarray, main):
    """Interleaved gate/up rows (row 2i gate, 2i+1 up; scales 1) such that
    every gate value g is 127 * 2^-k0 plus a few non-negative terms (so
    silu(g) == g in fp32 and double: exp(-g) < 2^-60) and every up value has
    |u| <= 12, so |g * u| <= 154 * 12 < 2048 and every output is an exact fp16."""
    K_ = x16.size
    xq = x16.astype(np.float64)
    q = np.full((2 * I, K_), 8, np.int64)
    small = np.nonzero((xq != 0) & (np.abs(xq) <= 3))[0]
    for i in range(I):
        q[2 * i, main[0]] = 8 + int(np.sign(xq[main[0]]))
        extra = rng.choice(small, 3, replace=False)
        q[2 * i, extra] = 8 + np.sign(xq[extra]).astype(np.int64) * rng.integers(0, 4, 3)
        up = rng.choice(small, 2, replace=False)
        q[2 * i + 1, up] = 8 + rng.integers(-2, 3, 2)
    sc = np.ones((2 * I, K_ // GROUP), np.float16)
    return pack_nibbles(q), sc


def exact_in_fp32(bound: np.ndarray, granularity: float) -> bool:
    """Every partial sum of terms that are multiples of `granularity` and whose
    |terms| sum to at most `bound` is exact in fp32 if bound < 2^24 units."""
    return bool(np.all(np.asarray(bound) < 2.0 ** 24 * granularity))


def visible_fraction(exact: np.ndarray, granularity: float) -> float:
    """Fraction of outputs whose fp16 spacing is at most `granularity`: there a
    change of one unit in any group dot changes the fp16 output."""
    ax = np.abs(np.asarray(exact, np.float64))
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -14)))
    return float(np.mean(2.0 ** (e - 10) <= granularity))
