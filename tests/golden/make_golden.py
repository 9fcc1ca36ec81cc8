"""Writes tests/golden/golden.npz: small input / output vectors of every kernel on the path, computed by the oracle
(oracle/, the C restatement of the reference arithmetic; binary and llama.cpp's blocks included) from the reference
tests' LCG streams (tests/int8-check.ts:116-117, seed 644; tests/ternary-check.ts:80-81, seed 231; the blocks' stream
seed 363) and the stories15M shape of the first benchmark config (n = 288,
24 of its 768 rows).  Arrays only (numpy.load with allow_pickle=False reads it).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import oracle  # noqa: E402
from streams import LCG, pack6, pack_binary, pack_ternary, scale_rule  # noqa: E402

F = np.float32
ROWS, N, TOKENS = 24, 288, 6
TN = 384  # ternary: 3 groups of 128
SB_ROWS, SB_N = 3, 512  # llama.cpp's blocks: 3 rows of 2 blocks
# where each block type keeps a float16 scale (kernels/blocks/types.ts:60-79; IQ1_M's is spread over four words and
# stays the stream's bytes)
SB_SCALES = {10: (80, 82), 12: (0, 2), 16: (0,), 17: (0,), 18: (0,), 19: (0,), 21: (0,), 22: (0,), 23: (0,)}


def frames(qs, ss, n, area):
    """tokens' bytes and their scale area in one buffer, a frame (16-byte multiple) a token"""
    frame = (n + area + 15) // 16 * 16
    buf = np.zeros((len(qs), frame), np.uint8)
    for t, (q, s) in enumerate(zip(qs, ss)):
        buf[t, :n] = np.asarray(q).view(np.uint8)
        buf[t, n:n + s.nbytes] = s.view(np.uint8)
    return buf, frame


def make():
    g = {}
    rng = LCG(644)
    x = np.array([((rng.next() % 20001) - 10000) * 3e-4 for _ in range(N)], F)
    x[5], x[40] = F(0.0), F(-2.5)
    g["x"] = x
    for bias in (0, 64):
        q, s = oracle.quantize_x(x, bias)
        g[f"xq{bias}"], g[f"xs{bias}"] = q.view(np.uint8), s
    w = np.array([(rng.next() & 255) - 128 for _ in range(ROWS * N)], np.int8)
    w[:N] = -128
    ws = np.array([scale_rule(rng, i) for i in range(ROWS * N // 32)], F)
    g["w"], g["ws"] = w, ws
    g["wc"] = oracle.int8_sums(w)
    g["q8r"] = oracle.matmul_q8r(g["xq64"], g["xs64"], w, ws, g["wc"], N)
    g["q8"] = oracle.matmul_q8(g["xq0"].view(np.int8), g["xs0"], w, ws, N)
    # int6: 4 v, v in -32..31
    v6 = np.array([4 * ((rng.next() & 63) - 32) for _ in range(ROWS * N)], np.int8)
    p6 = pack6(v6)
    g["w6"], g["wc6"] = p6, oracle.six_sums(p6)
    g["q6r"] = oracle.matmul_q6r(g["xq64"], g["xs64"], p6, ws, g["wc6"], N)
    g["q6"] = oracle.matmul_q6(g["xq0"].view(np.int8), g["xs0"], p6, ws, N)
    # a prompt of TOKENS tokens for the tile: 7-bit bytes, scales by the rule
    qs = [np.array([rng.next() & 127 for _ in range(N)], np.uint8) for _ in range(TOKENS)]
    ss = [np.array([scale_rule(rng, j + t) for j in range(N // 32)], F) for t in range(TOKENS)]
    buf, frame = frames(qs, ss, N, 4 * (N // 32))
    g["tile_x"], g["tile_frame"] = buf, np.array([frame], np.int32)
    g["tile_q8r"] = np.stack([oracle.matmul_q8r(q, s, w, ws, g["wc"], N) for q, s in zip(qs, ss)])
    # ternary (seed 231): codes 0..2, float16 scales a group of 128, activations quantize_x(bias 0) + interleave
    rt = LCG(231)
    codes = np.array([rt.next() % 3 for _ in range(ROWS * TN)], np.uint8)
    g["wt"] = pack_ternary(codes)
    g["wst"] = np.array([(1e-3 * (1 + rt.next() % 1000)) for _ in range(ROWS * TN // 128)], np.float16).view(np.uint16)
    xt = np.array([((rt.next() % 20001) - 10000) * 2e-4 for _ in range(TN)], F)
    q, s = oracle.quantize_x(xt, 0)
    tq, tarea = oracle.interleave(q.view(np.int8), s)
    g["xt"], g["xtq"], g["xtarea"] = xt, tq.view(np.uint8), tarea
    g["t2r"] = oracle.matmul_t2r(tq, tarea, g["wt"], g["wst"], TN)
    tqs, tss = [], []
    for t in range(TOKENS):
        xx = np.array([((rt.next() % 20001) - 10000) * 2e-4 for _ in range(TN)], F)
        q, s = oracle.quantize_x(xx, 0)
        a, b = oracle.interleave(q.view(np.int8), s)
        tqs.append(a)
        tss.append(b)
    tbuf, tframe = frames(tqs, tss, TN, 8 * (TN // 32))
    g["ttile_x"], g["ttile_frame"] = tbuf, np.array([tframe], np.int32)
    g["ttile_t2r"] = np.stack([oracle.matmul_t2r(a, b, g["wt"], g["wst"], TN) for a, b in zip(tqs, tss)])
    # binary (the same stream on): signs a bit (1 for +1), the ternary scales and activations; binary_x of +-d groups
    signs = np.array([rt.next() & 1 for _ in range(ROWS * TN)], np.uint8)
    g["wb"] = pack_binary(signs, TN)
    g["b1r"] = oracle.matmul_b1r(tq, tarea, g["wb"], g["wst"], TN)
    g["btile_b1r"] = np.stack([oracle.matmul_b1r(a, b, g["wb"], g["wst"], TN) for a, b in zip(tqs, tss)])
    xb = np.array([(1 if rt.next() & 1 else -1) * 0.02 * (1 + (j >> 7)) for j in range(TN)], F)
    xb[3] = F(0.5 * xb[3])  # a value that is not its group's +-largest: binary_x refuses it
    g["xb"] = xb
    g["xb_bits"], g["xb_scales"], bad = oracle.binary_x(xb)
    g["xb_bad"] = np.array([bad], np.int32)
    # llama.cpp's blocks (seed 363): codebooks of stream bytes, and for each type SB_ROWS rows of SB_N weights of stream
    # bytes with float16 scales of 1e-5 .. 1e-2 where the type keeps them, one token (quantize_x at bias 0, sums_x)
    rb = LCG(363)
    books = np.array([rb.next() & 255 for _ in range(oracle.SB_CODEBOOKS)], np.uint8)
    g["sb_books"], g["sb_tables"] = books, oracle.sb_tables(books)
    xs_ = np.array([((rb.next() % 20001) - 10000) * 3e-4 for _ in range(SB_N)], F)
    q, s = oracle.quantize_x(xs_, 0)
    g["sb_x"], g["sb_xq"], g["sb_area"] = xs_, q, oracle.sums_x(q.view(np.int8), s)
    for name, t in oracle.SB_TYPES.items():
        size = oracle.sb_bytes(t)
        b = np.array([rb.next() & 255 for _ in range(SB_ROWS * (SB_N // 256) * size)], np.uint8).reshape(-1, size)
        for blk in b:
            for at in SB_SCALES.get(t, ()):
                blk[at:at + 2] = np.array([(1 + rb.next() % 1000) * 1e-5], np.float16).view(np.uint8)
        g[f"sb_w_{name}"] = b.reshape(-1)
        g[f"sb_out_{name}"] = oracle.matmul_sbr(q.view(np.int8), g["sb_area"], b.reshape(-1), g["sb_tables"], SB_N, t)
        g[f"sb_row_{name}"] = oracle.sb_row(b.reshape(-1)[:(SB_N // 256) * size], g["sb_tables"], SB_N, t)
    return g


if __name__ == "__main__":
    g = make()
    np.savez(os.path.join(HERE, "golden.npz"), **g)
    print(f"wrote {len(g)} arrays, {sum(a.nbytes for a in g.values())} bytes")
