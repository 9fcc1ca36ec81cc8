"""oracle.py — TEST INFRASTRUCTURE ONLY.

ctypes bindings of liboracle.so (oracle.c: a scalar C restatement of the reference's quantized-matmul arithmetic,
in the reference's float32 order) for the tests, the smoke check and bench.py's CPU baseline.  Nothing on the
product path imports this module.

Every function takes NumPy arrays (C-contiguous, of the dtype the reference's memory holds) and returns NumPy
arrays; byte strides follow the reference (os, frame in bytes).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "liboracle.so")


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            build()
        L = ctypes.CDLL(LIBRARY)
        p, i32 = ctypes.c_void_p, ctypes.c_int32
        sigs = {
            "o_quantize_x": [p, p, p, i32, i32],
            "o_int8_sums": [p, p, i32],
            "o_six_sums": [p, p, i32],
            "o_six_unpack": [p, p],
            "o_interleave": [p, p, i32],
            "o_matmul_q8r": [p, p, p, p, p, p, i32, i32, i32],
            "o_matmul_q8": [p, p, p, p, p, i32, i32, i32],
            "o_matmul_q8r_tile": [p, p, p, p, p, p, i32, i32, i32, i32, i32, i32],
            "o_matmul_q6r": [p, p, p, p, p, p, i32, i32, i32],
            "o_matmul_q6": [p, p, p, p, p, i32, i32, i32],
            "o_matmul_t2r": [p, p, p, p, p, i32, i32, i32, i32],
            "o_matmul_t2r_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32],
            "o_matmul_b1r": [p, p, p, p, p, i32, i32, i32, i32],
            "o_matmul_b1r_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32],
            "o_sums_x": [p, p, i32],
            "o_matmul_sbr": [p, p, p, p, p, i32, i32, i32, i32],
            "o_matmul_sbr_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32],
            "o_sb_row": [p, p, p, i32, i32],
            "o_add_columns": [p, p, p, i32, i32],
        }
        for name, argtypes in sigs.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = argtypes, None
        L.o_half.argtypes, L.o_half.restype = [ctypes.c_uint16], ctypes.c_float
        L.o_binary_x.argtypes, L.o_binary_x.restype = [p, p, p, i32], i32
        L.o_quantize6_x.argtypes, L.o_quantize6_x.restype = [p, p, p, i32], None
        L.o_ternary_x.argtypes, L.o_ternary_x.restype = [p, p, p, i32], i32
        L.o_sb_bytes.argtypes, L.o_sb_bytes.restype = [i32], i32
        L.o_sb_tables.argtypes, L.o_sb_tables.restype = [p, p], i32
        L.o_time_gemv.argtypes = [i32, p, p, p, p, p, p, i32, i32, i32, i32]
        L.o_time_gemv.restype = ctypes.c_double
        L.f_matmul_q8r.argtypes, L.f_matmul_q8r.restype = [p, p, p, p, p, p, i32, i32, i32], None
        L.f_matmul_q8r_tile.argtypes = [p, p, p, p, p, p, i32, i32, i32, i32, i32, i32]
        L.f_matmul_q8r_tile.restype = None
        L.f_time_q8r.argtypes = [p, p, p, p, p, p, i32, i32, i32, i32, i32, i32]
        L.f_time_q8r.restype = ctypes.c_double
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


def quantize_x(x, bias):
    """kernels/kernel/quantize.ts:124-151: float32 x (n) -> (uint8 xq (n), float32 xs (n/32))."""
    x = _c(x, np.float32)
    n = x.shape[-1]
    xq, xs = np.zeros(n, np.uint8), np.zeros(n // 32, np.float32)
    lib().o_quantize_x(_p(xq), _p(xs), _p(x), n, bias)
    return xq, xs


def int8_sums(w):
    w = _c(w, np.int8).reshape(-1)
    out = np.zeros(w.size // 32, np.int32)
    lib().o_int8_sums(_p(out), _p(w), out.size)
    return out


def six_sums(w):
    w = _c(w, np.uint8).reshape(-1)
    out = np.zeros(w.size // 24, np.int32)
    lib().o_six_sums(_p(out), _p(w), out.size)
    return out


def six_unpack(packed):
    """24 bytes a group -> the groups' int8 values (flattened)."""
    packed = _c(packed, np.uint8).reshape(-1, 24)
    out = np.zeros((packed.shape[0], 32), np.int8)
    for g in range(packed.shape[0]):
        lib().o_six_unpack(out[g].ctypes.data, packed[g].ctypes.data)
    return out.reshape(-1)


def interleave(xq, xs):
    """kernels/kernel/matmul.ts:134-146: returns (permuted int8 xq, the 8 bytes a group of xs: scales then sums)."""
    xq = _c(xq, np.int8).copy()
    n = xq.size
    area = np.zeros(2 * (n // 32), np.float32)
    area[: n // 32] = np.asarray(xs, np.float32)
    lib().o_interleave(_p(xq), _p(area), n)
    return xq, area


def half(bits):
    return lib().o_half(int(bits) & 0xFFFF)


def matmul_q8r(xq, xs, wq, ws, wc, n, r0=0, r1=None):
    rows = wq.size // n
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_q8r(_p(out), _p(_c(xq, np.uint8)), _p(_c(xs, np.float32)), _p(_c(wq, np.int8)),
                       _p(_c(ws, np.float32)), _p(_c(wc, np.int32)), n, r0, r1)
    return out


def matmul_q8(xq, xs, wq, ws, n, r0=0, r1=None):
    rows = wq.size // n
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_q8(_p(out), _p(_c(xq, np.int8)), _p(_c(xs, np.float32)), _p(_c(wq, np.int8)),
                      _p(_c(ws, np.float32)), n, r0, r1)
    return out


def matmul_q6r(xq, xs, wq, ws, wc, n, r0=0, r1=None):
    rows = wq.size // (n // 32 * 24)
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_q6r(_p(out), _p(_c(xq, np.uint8)), _p(_c(xs, np.float32)), _p(_c(wq, np.uint8)),
                       _p(_c(ws, np.float32)), _p(_c(wc, np.int32)), n, r0, r1)
    return out


def matmul_q6(xq, xs, wq, ws, n, r0=0, r1=None):
    rows = wq.size // (n // 32 * 24)
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_q6(_p(out), _p(_c(xq, np.int8)), _p(_c(xs, np.float32)), _p(_c(wq, np.uint8)),
                      _p(_c(ws, np.float32)), n, r0, r1)
    return out


def matmul_t2r(xq, area, wq, ws_bits, n, r0=0, r1=None, three=3):
    """xq: interleaved int8 activations; area: xs then the int32 sums (interleave's 8 bytes a group)."""
    rows = wq.size // (n // 4)
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_t2r(_p(out), _p(_c(xq, np.int8)), _p(_c(area, np.float32)), _p(_c(wq, np.uint8)),
                       _p(_c(ws_bits, np.uint16)), n, r0, r1, three)
    return out


def matmul_b1r(xq, area, wq, ws_bits, n, r0=0, r1=None, two=2):
    """binary weights (16 bytes a group of 128); xq, area as matmul_t2r's."""
    rows = wq.size // (n // 8)
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_b1r(_p(out), _p(_c(xq, np.int8)), _p(_c(area, np.float32)), _p(_c(wq, np.uint8)),
                       _p(_c(ws_bits, np.uint16)), n, r0, r1, two)
    return out


def binary_x(x):
    """kernels/kernel/quantize.ts:232-247: float32 x (groups of 128) -> (uint8 bits (n/8), float32 scales (n/128),
    the refusal flag)."""
    x = _c(x, np.float32)
    n = x.size
    out, xs = np.zeros(n // 8, np.uint8), np.zeros(n // 128, np.float32)
    bad = lib().o_binary_x(_p(out), _p(xs), _p(x), n)
    return out, xs, bad


def quantize6_x(x):
    """kernels/kernel/quantize.ts:161-182: float32 x (groups of 32) -> (uint8 24 bytes a group, float32 scale / 4 a
    group)."""
    x = _c(x, np.float32)
    n = x.size
    out, xs = np.zeros(n // 32 * 24, np.uint8), np.zeros(n // 32, np.float32)
    lib().o_quantize6_x(_p(out), _p(xs), _p(x), n)
    return out, xs


def ternary_x(x):
    """kernels/kernel/quantize.ts:197-225: float32 x (groups of 128) -> (uint8 codes (n/4), float32 scales (n/128),
    the refusal flag)."""
    x = _c(x, np.float32)
    n = x.size
    out, xs = np.zeros(n // 4, np.uint8), np.zeros(n // 128, np.float32)
    bad = lib().o_ternary_x(_p(out), _p(xs), _p(x), n)
    return out, xs, bad


SB_TYPES = {"Q2_K": 10, "Q4_K": 12, "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21,
            "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29}
SB_TABLES = 34992
SB_CODEBOOKS = 33808  # the codebooks row (src/python/engine/dtypes.py CODEBOOKS)


def sb_bytes(type_):
    return lib().o_sb_bytes(type_)


def sb_tables(codebooks):
    """kernels/blocks/types.ts:323-348: the tables (uint8, 34992) from the codebooks row (uint8, 33808)."""
    area = np.zeros(SB_TABLES, np.uint8)
    lib().o_sb_tables(_p(area), _p(_c(codebooks, np.uint8)))
    return area


def sums_x(xq, xs):
    """quantize_x(.., 0)'s int8 xq (n) and scales xs (n/32) -> the area kernels/blocks/token.ts reads: the scales,
    then n/16 and n/8 int16 sums, as one uint8 array"""
    xq = _c(xq, np.int8)
    n = xq.size
    area = np.zeros(4 * (n // 32) + 2 * (n // 16) + 2 * (n // 8), np.uint8)
    area[:4 * (n // 32)] = _c(xs, np.float32).view(np.uint8)
    lib().o_sums_x(_p(area), _p(xq), n)
    return area


def matmul_sbr(xq, area, w, tab, n, type_, r0=0, r1=None):
    rows = w.size // ((n // 256) * sb_bytes(type_))
    r1 = rows if r1 is None else r1
    out = np.zeros(rows, np.float32)
    lib().o_matmul_sbr(_p(out), _p(_c(xq, np.int8)), _p(_c(area, np.uint8)), _p(_c(w, np.uint8)),
                       _p(_c(tab, np.uint8)), n, r0, r1, type_)
    return out


def sb_row(w, tab, n, type_):
    out = np.zeros(n, np.float32)
    lib().o_sb_row(_p(out), _p(_c(w, np.uint8)), _p(_c(tab, np.uint8)), n, type_)
    return out


def matmul_q8r_tokens(xq, xs, wq, ws, wc, n):
    """matmul_q8r for each token (rows of xq / xs): (count, rows) outputs."""
    return np.stack([matmul_q8r(xq[t], xs[t], wq, ws, wc, n) for t in range(xq.shape[0])])


def matmul_t2r_tokens(xq, area, wq, ws_bits, n):
    return np.stack([matmul_t2r(xq[t], area[t], wq, ws_bits, n) for t in range(xq.shape[0])])


KINDS = {"matmul_q8r": 0, "matmul_q8": 1, "matmul_q6r": 2, "matmul_q6": 3, "matmul_t2r": 4}


def time_gemv(kind, xq, xs, wq, ws, wc, n, rows, threads, reps):
    """The oracle's GEMV over all rows on `threads` host threads (phase()-style chunks); fastest of reps, seconds."""
    out = np.zeros(rows, np.float32)
    return lib().o_time_gemv(KINDS[kind], _p(out), _p(xq), _p(xs), _p(wq), _p(ws), _p(wc), n, rows, threads, reps)


def fast_matmul_q8r(xq, xs, wq, ws, wc, n, r0=0, r1=None):
    """fast.c's vectorised matmul_q8r (the CPU baseline's kernel): the oracle's numbers to the bit."""
    wq = _c(wq, np.int8).reshape(-1)
    r1 = wq.size // n if r1 is None else r1
    out = np.zeros(wq.size // n, np.float32)
    lib().f_matmul_q8r(_p(out), _p(_c(xq, np.uint8)), _p(_c(xs, np.float32)), _p(wq), _p(_c(ws, np.float32)),
                       _p(_c(wc, np.int32)), n, r0, r1)
    return out


def fast_matmul_q8r_tile(xq, xs, wq, ws, wc, n, count, r0=0, r1=None):
    """fast.c's vectorised matmul_q8r_tile: xq (count, n) uint8, xs (count, n/32); returns (count, rows)."""
    wq = _c(wq, np.int8).reshape(-1)
    rows = wq.size // n
    r1 = rows if r1 is None else r1
    frame = n + 4 * (n // 32)
    buf = np.zeros((count, frame), np.uint8)
    buf[:, :n] = np.asarray(xq, np.uint8).reshape(count, n)
    buf[:, n:] = np.asarray(xs, np.float32).reshape(count, n // 32).view(np.uint8)
    out = np.zeros((count, rows), np.float32)
    lib().f_matmul_q8r_tile(_p(out), _p(buf), buf.ctypes.data + n, _p(wq), _p(_c(ws, np.float32)),
                            _p(_c(wc, np.int32)), n, r0, r1, count, 4 * rows, frame)
    return out


def time_fast_q8r(xq, xs, wq, ws, wc, n, rows, threads, count=0, frame=0):
    """Seconds one call of fast.c's matmul_q8r (count 0: xq (n), xs (n/32)) or matmul_q8r_tile (count tokens a frame
    apart in xq, their scales in xs at the same frame) takes over all rows on `threads` host threads."""
    out = np.zeros(max(count, 1) * rows, np.float32)
    return lib().f_time_q8r(_p(out), _p(xq), _p(xs), _p(wq), _p(ws), _p(wc), n, rows, count, 4 * rows, frame,
                            threads)


def add_columns(y, rows, a):
    """kernels/kernel/matmul.ts:248-266: y (n) plus the products of a (count) and rows (count, n), in order"""
    y = np.array(y, np.float32)
    rows = _c(rows, np.float32).reshape(-1, y.size)
    a = _c(a, np.float32)
    lib().o_add_columns(_p(y), _p(rows), _p(a), a.size, y.size)
    return y


def packed_values(packing, raw, count):
    """jobs.ts:398-433 (each packing's value()): the first `count` weights of a packed tensor as int32 —
    int8 the bytes; int6 (six.ts:1-11) 4 v from its 24 bytes a group of 32; ternary (ternary.ts:25-34) code - 1;
    binary (binary.ts:1-4) +1 where bit 4 h + p of byte c of a group is set for weight 64 h + 4 c + p, else -1"""
    u = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    i = np.arange(count, dtype=np.int64)
    if packing == "int8":
        return u[:count].view(np.int8).astype(np.int32)
    if packing == "int6":
        g, j = (i >> 5) * 24, i & 31
        low = np.where(j < 16, u[g + np.minimum(j, 15)] & 15, u[g + np.maximum(j - 16, 0)] >> 4).astype(np.int32)
        top = (u[g + 16 + (j & 7)].astype(np.int32) >> (2 * (j >> 3))) & 3
        return ((low | (top << 4)) << 2).astype(np.uint8).view(np.int8).astype(np.int32)
    if packing == "ternary":
        return ((u[i >> 2].astype(np.int32) >> (2 * (i & 3))) & 3) - 1
    if packing == "binary":
        byte = u[((i >> 7) << 4) + ((i >> 2) & 15)].astype(np.int32)
        return (((byte >> ((((i >> 6) & 1) << 2) | (i & 3))) & 1) << 1) - 1
    raise ValueError(packing)


def outlier_columns(packing, values, scales, channels, vocab, dim, group):
    """src/runtime/forward/tensors.ts:175-186: columns[i][w] = f(value(w dim + c_i) scale(w groups + c_i / group))
    (float32 scales, or float16 ones for ternary and binary, widened exactly), as (len(channels), vocab) float32"""
    v = packed_values(packing, values, vocab * dim).reshape(vocab, dim)
    if packing in ("ternary", "binary"):
        s = np.ascontiguousarray(scales).reshape(-1).view(np.uint16)[:vocab * (dim // group)]
        s = np.array([half(h) for h in s], np.float32)
    else:
        s = np.ascontiguousarray(scales).reshape(-1).view(np.float32)[:vocab * (dim // group)]
    s = s.reshape(vocab, dim // group)
    out = np.zeros((len(channels), vocab), np.float32)
    for i, c in enumerate(channels):
        out[i] = v[:, c].astype(np.float32) * s[:, c // group]
    return out


def take_channels(x, channels):
    """src/runtime/forward/engine.ts:461-464: (picked, x with those channels set to 0), channel by channel"""
    x = np.array(x, np.float32)
    picked = np.zeros(len(channels), np.float32)
    for i, c in enumerate(channels):
        picked[i] = x[c]
        x[c] = 0.0
    return picked, x
