"""The committed fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py from the reference tests'
LCG streams): the oracle must still produce them, and the HIP kernels must produce them bit for bit."""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
F = np.float32
ROWS, N, TN = 24, 288, 384
SB_ROWS, SB_N = 3, 512
SB_NAMES = ("Q2_K", "Q4_K", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ1_S", "IQ3_S", "IQ2_S", "IQ4_XS", "IQ1_M")
SB_NUMBERS = (10, 12, 16, 17, 18, 19, 21, 22, 23, 29)


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False) as g:
        return {k: g[k] for k in g.files}


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def test_oracle_reproduces_golden(oracle, golden):
    g = golden
    for bias in (0, 64):
        q, s = oracle.quantize_x(g["x"], bias)
        assert same(q.view(np.uint8), g[f"xq{bias}"]) and same(s, g[f"xs{bias}"])
    assert same(oracle.int8_sums(g["w"]), g["wc"])
    assert same(oracle.six_sums(g["w6"]), g["wc6"])
    assert same(oracle.matmul_q8r(g["xq64"], g["xs64"], g["w"], g["ws"], g["wc"], N), g["q8r"])
    assert same(oracle.matmul_q8(g["xq0"].view(np.int8), g["xs0"], g["w"], g["ws"], N), g["q8"])
    assert same(oracle.matmul_q6r(g["xq64"], g["xs64"], g["w6"], g["ws"], g["wc6"], N), g["q6r"])
    assert same(oracle.matmul_q6(g["xq0"].view(np.int8), g["xs0"], g["w6"], g["ws"], N), g["q6"])
    q, s = oracle.quantize_x(g["xt"], 0)
    tq, area = oracle.interleave(q.view(np.int8), s)
    assert same(tq.view(np.uint8), g["xtq"]) and same(area, g["xtarea"])
    assert same(oracle.matmul_t2r(g["xtq"].view(np.int8), g["xtarea"], g["wt"], g["wst"], TN), g["t2r"])
    assert same(oracle.matmul_b1r(g["xtq"].view(np.int8), g["xtarea"], g["wb"], g["wst"], TN), g["b1r"])
    bits, scales, bad = oracle.binary_x(g["xb"])
    assert same(bits, g["xb_bits"]) and same(scales, g["xb_scales"]) and bad == g["xb_bad"][0] == 1
    assert same(oracle.sb_tables(g["sb_books"]), g["sb_tables"])
    q, s = oracle.quantize_x(g["sb_x"], 0)
    assert same(q, g["sb_xq"]) and same(oracle.sums_x(q.view(np.int8), s), g["sb_area"])
    for name, t in oracle.SB_TYPES.items():
        w = g[f"sb_w_{name}"]
        assert same(oracle.matmul_sbr(g["sb_xq"].view(np.int8), g["sb_area"], w, g["sb_tables"], SB_N, t),
                    g[f"sb_out_{name}"]), name
        assert same(oracle.sb_row(w[:w.size // SB_ROWS], g["sb_tables"], SB_N, t), g[f"sb_row_{name}"]), name
        assert np.all(np.isfinite(g[f"sb_out_{name}"])), name
    frame = int(g["tile_frame"][0])
    for t in range(g["tile_x"].shape[0]):
        row = g["tile_x"][t]
        got = oracle.matmul_q8r(row[:N], row[N:N + 4 * (N // 32)].view(F), g["w"], g["ws"], g["wc"], N)
        assert same(got, g["tile_q8r"][t])
    assert frame % 16 == 0


def test_generator_is_deterministic(golden):
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_golden
    fresh = make_golden.make()
    assert sorted(fresh) == sorted(golden)
    for k in golden:
        assert same(fresh[k], golden[k]), k


@pytest.mark.gpu
def test_kernels_reproduce_golden(pkg, golden):
    from gpu_util import Arena
    g = golden
    k = pkg.load_kernels()
    arena = Arena(1 << 22)

    def out(count):
        return arena.alloc(4 * count, fill=np.full(count, -7, F))

    ax = arena.put(g["x"])
    for bias in (0, 64):
        xq, xs = arena.alloc(N), arena.alloc(4 * (N // 32))
        k.quantize_x(xq, xs, ax, N, bias)
        assert same(arena.get(xq, np.uint8, N), g[f"xq{bias}"]), bias
        assert same(arena.get(xs, F, N // 32), g[f"xs{bias}"]), bias
    aw, aws, aw6 = arena.put(g["w"]), arena.put(g["ws"]), arena.put(g["w6"])
    sums = arena.alloc(4 * g["wc"].size)
    k.int8_sums(sums, aw, g["wc"].size)
    assert same(arena.get(sums, np.int32, g["wc"].size), g["wc"])
    k.six_sums(sums, aw6, g["wc6"].size)
    assert same(arena.get(sums, np.int32, g["wc6"].size), g["wc6"])
    awc, awc6 = arena.put(g["wc"]), arena.put(g["wc6"])
    x64, s64 = arena.put(g["xq64"]), arena.put(g["xs64"])
    x0, s0 = arena.put(g["xq0"]), arena.put(g["xs0"])
    for name, args, want in (
            ("matmul_q8r", (x64, s64, aw, aws, awc, N, 0, ROWS), g["q8r"]),
            ("matmul_q8", (x0, s0, aw, aws, N, 0, ROWS), g["q8"]),
            ("matmul_q6r", (x64, s64, aw6, aws, awc6, N, 0, ROWS), g["q6r"]),
            ("matmul_q6", (x0, s0, aw6, aws, N, 0, ROWS), g["q6"])):
        o = out(ROWS)
        getattr(k, name)(o, *args)
        assert same(arena.get(o, F, ROWS), want), name
    # ternary: quantize_x (bias 0) and interleave in place, then the product
    txq, txs = arena.alloc(TN), arena.alloc(8 * (TN // 32))
    k.quantize_x(txq, txs, arena.put(g["xt"]), TN, 0)
    k.interleave(txq, txs, TN)
    assert same(arena.get(txq, np.uint8, TN), g["xtq"])
    assert same(arena.get(txs, F, 2 * (TN // 32)), g["xtarea"])
    awt, awst = arena.put(g["wt"]), arena.put(g["wst"])
    o = out(ROWS)
    k.matmul_t2r(o, txq, txs, awt, awst, TN, 0, ROWS, 3)
    assert same(arena.get(o, F, ROWS), g["t2r"])
    # the tiles: the fixture's 6 tokens, and 18 (each three times: the matrix-core path), every token its own number
    for count in (6, 18):
        reps = count // 6
        buf = arena.put(np.tile(g["tile_x"], (reps, 1)))
        frame = int(g["tile_frame"][0])
        o = out(ROWS * count)
        k.matmul_q8r_tile(o, buf, buf + N, aw, aws, awc, N, 0, ROWS, count, 4 * ROWS, frame)
        assert same(arena.get(o, F, ROWS * count).reshape(count, ROWS), np.tile(g["tile_q8r"], (reps, 1))), count
        tbuf = arena.put(np.tile(g["ttile_x"], (reps, 1)))
        tframe = int(g["ttile_frame"][0])
        o = out(ROWS * count)
        k.matmul_t2r_tile(o, tbuf, tbuf + TN, awt, awst, TN, 0, ROWS, count, 4 * ROWS, tframe, 3)
        assert same(arena.get(o, F, ROWS * count).reshape(count, ROWS), np.tile(g["ttile_t2r"], (reps, 1))), count
        awb = arena.put(g["wb"])
        o = out(ROWS * count)
        k.matmul_b1r_tile(o, tbuf, tbuf + TN, awb, awst, TN, 0, ROWS, count, 4 * ROWS, tframe, 2)
        assert same(arena.get(o, F, ROWS * count).reshape(count, ROWS), np.tile(g["btile_b1r"], (reps, 1))), count
    # binary: the token kernel, and binary_x
    o = out(ROWS)
    k.matmul_b1r(o, txq, txs, arena.put(g["wb"]), awst, TN, 0, ROWS, 2)
    assert same(arena.get(o, F, ROWS), g["b1r"])
    bits, scales = arena.alloc(TN // 8), arena.alloc(4 * (TN // 128))
    assert k.binary_x(bits, scales, arena.put(g["xb"]), TN) == g["xb_bad"][0]
    assert same(arena.get(bits, np.uint8, TN // 8), g["xb_bits"])
    assert same(arena.get(scales, F, TN // 128), g["xb_scales"])
    # llama.cpp's blocks: the tables, the sums of 16 and 8, the token product and the rows
    tab = arena.alloc(g["sb_tables"].size)
    assert k.sb_tables(tab, arena.put(g["sb_books"])) == g["sb_tables"].size
    assert same(arena.get(tab, np.uint8, g["sb_tables"].size), g["sb_tables"])
    xq, area = arena.put(g["sb_xq"]), arena.alloc(g["sb_area"].size)
    arena.write(area, g["sb_area"][:4 * (SB_N // 32)])
    k.sums_x(area, xq, SB_N)
    assert same(arena.get(area, np.uint8, g["sb_area"].size), g["sb_area"])
    for name, t in {n: int(n2) for n, n2 in zip(SB_NAMES, SB_NUMBERS)}.items():
        w = g[f"sb_w_{name}"]
        aw = arena.put(w)
        o = out(SB_ROWS)
        k.matmul_sbr(o, xq, area, aw, tab, SB_N, 0, SB_ROWS, t)
        assert same(arena.get(o, F, SB_ROWS), g[f"sb_out_{name}"]), name
        r = arena.alloc(4 * SB_N)
        k.sb_row(r, aw, tab, SB_N, t)
        assert same(arena.get(r, F, SB_N), g[f"sb_row_{name}"]), name
