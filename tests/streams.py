"""The reference tests' input streams, reproduced: the LCG of tests/int8-check.ts:116-117 and
tests/ternary-check.ts:80-81 (`seed = imul(seed, 1103515245) + 12345 >>> 0; next = seed >>> 8`), and the
value rules their cases use.  Test-side helpers only."""
import numpy as np


class LCG:
    def __init__(self, seed):
        self.seed = seed & 0xFFFFFFFF

    def next(self):
        self.seed = (self.seed * 1103515245 + 12345) & 0xFFFFFFFF
        return self.seed >> 8


def f32(v):
    return np.float32(v)


def scale_rule(rng, i):
    """tests/int8-check.ts:119: every size, a subnormal every 11 and a zero every 13."""
    if i % 11 == 7:
        return f32(2.0 ** -130 * (1 + (rng.next() % 1000)))
    if i % 13 == 5:
        return f32(0.0)
    return f32(1e-3 * (1 + (rng.next() % 1000)))


def pack6(values):
    """src/python/engine/packing.py:56-62's layout (tests/int8-check.ts:56-63): int8 multiples of 4, groups of 32 ->
    24 bytes a group: low nibble of value j and of j + 16 in byte j, the top two bits of k, k+8, k+16, k+24 at bits
    0, 2, 4, 6 of byte 16 + k."""
    v = (np.asarray(values, np.int8).reshape(-1, 32).view(np.uint8) >> 2) & 63
    out = np.zeros((v.shape[0], 24), np.uint8)
    out[:, :16] = (v[:, :16] & 15) | ((v[:, 16:] & 15) << 4)
    top = v >> 4
    out[:, 16:] = top[:, 0:8] | (top[:, 8:16] << 2) | (top[:, 16:24] << 4) | (top[:, 24:32] << 6)
    return out.reshape(-1)


def pack_ternary(codes):
    """src/python/engine/packing.py:106-109's layout: code j of a row in byte j >> 2 at bits 2 (j & 3)."""
    c = np.asarray(codes, np.uint8).reshape(-1, 4)
    return (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)


def uninterleave_index(n):
    """tests/ternary-check.ts:96: byte `at` of the interleaved activations is activation
    (at & ~63) + 4 (at & 15) + ((at >> 4) & 3)."""
    at = np.arange(n)
    return (at & ~63) + 4 * (at & 15) + ((at >> 4) & 3)


def pack_binary(bits, n):
    """kernels/binary.ts:1-4 (the layout of packing.py's pack_binary), as tests/ternary-check.ts:303-305 writes it:
    bit i of a row (1 for +1) at byte (group) 16 + ((i >> 2) & 15), bit ((i >> 6) & 1) * 4 + (i & 3)."""
    b = np.asarray(bits, np.uint8).reshape(-1, n)
    rows = b.shape[0]
    out = np.zeros((rows, n // 8), np.uint8)
    i = np.arange(n)
    at = ((i >> 7) << 4) + ((i >> 2) & 15)
    shift = (((i >> 6) & 1) << 2) | (i & 3)
    for r in range(rows):
        np.bitwise_or.at(out[r], at, (b[r] << shift).astype(np.uint8))
    return out.reshape(-1)
