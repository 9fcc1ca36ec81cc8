"""hq_matmul_q8r_tile_tol_ex: matmul_q8r_tile's products to the north star's float32 tolerance (every group's integer
exact, the groups added in this library's order), through the C-ABI on cuda:0.

The bar (written in each test): |got - want| <= 1e-5 max|want| over a matrix's outputs, want the reference's number
(the oracle's matmul_q8r with int8_sums' corrections; the reference's LINE, tests/tile-bench.ts:34-41), and the
reference's number to the bit where every term and partial sum is exact (power-of-two scales, small sums), so that a
wrong integer cannot hide inside the tolerance.  At the configs' full sizes every output is compared with the
bit-exact tile (itself the oracle's number, tests/test_gpu_shapes.py) and a sample of tokens with the oracle."""
import numpy as np
import pytest

from gpu_util import Arena
from models import F

pytestmark = pytest.mark.gpu
TOL = 1e-5  # |err| <= TOL * max|y| a matrix
SENTINEL = -7.25


@pytest.fixture(scope="module")
def L(pkg):
    import torch
    assert torch.cuda.is_available(), "the GPU tests need a GPU"
    return pkg.library()


@pytest.fixture(scope="module")
def arena():
    return Arena(3 << 29)


@pytest.fixture(autouse=True)
def fresh(arena, L):
    """every test here runs the tolerance tile itself, whatever its launch's size (hq_tol_min_tiles 0), unless it
    says otherwise"""
    arena.reset()
    before = L.hq_tol_min_tiles(0)
    yield
    L.hq_tol_min_tiles(before)


def frames(q, s, n):
    """tokens' bytes and scales one frame apart (the reference's S: the scales after the bytes)"""
    count = len(q)
    frame = ((n + 4 * (n // 32) + 15) // 16) * 16
    buf = np.zeros((count, frame), np.uint8)
    for t in range(count):
        buf[t, :n] = q[t].view(np.uint8)
        buf[t, n:n + 4 * (n // 32)] = np.asarray(s[t], F).view(np.uint8)
    return buf, frame


def quantized(oracle, rng, count, n):
    q, s = zip(*(oracle.quantize_x(rng.standard_normal(n).astype(F), 64) for _ in range(count)))
    return np.array(q), np.array(s)


def run_tol(L, arena, w, ws, buf, frame, n, r0, r1, count, rows_total):
    """the tolerance tile over rows r0..r1 of a [rows_total, n] matrix; returns the [count, rows_total] outputs (rows
    outside r0..r1 hold the sentinel)"""
    wq, wsa, xq = arena.put(w), arena.put(ws), arena.put(buf)
    os_ = 4 * rows_total
    out = arena.alloc(os_ * count, fill=np.full(rows_total * count, SENTINEL, F))
    need = L.hq_tol_work_bytes(n, count)
    assert need > 0
    work = arena.alloc(need)
    st = L.hq_matmul_q8r_tile_tol_ex(out, xq, xq + n, wq, wsa, n, r0, r1, count, os_, frame, work, need, None)
    assert st == 0, L.hq_last_error_message()
    return arena.get(out, F, rows_total * count).reshape(count, rows_total)


def reference(oracle, w, ws, q, s, n, rows=None):
    wc = oracle.int8_sums(w)
    full = [oracle.matmul_q8r(q[t], s[t], w, ws, wc, n) for t in range(len(q))]
    return np.array(full)


def within(got, want):
    bound = TOL * float(np.max(np.abs(want)))
    err = float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64))))
    return err <= bound, f"max |err| {err:.3e} against the bound {bound:.3e}"


@pytest.mark.parametrize("rows,n,count,r0,r1", [
    (300, 288, 37, 0, 300),      # 9 groups (a stage of one group at the end), 3 row tiles, one token tile
    (129, 800, 130, 0, 129),     # 25 groups, a row and two tokens past the tiles
    (64, 1024, 16, 0, 64),       # the fewest tokens the prompt path takes
    (1000, 4096, 200, 100, 900),  # a row range inside the matrix: nothing written outside it
    (257, 2048, 129, 1, 256),
])
def test_tolerance_against_the_oracle(L, arena, oracle, rows, n, count, r0, r1):
    rng = np.random.default_rng(rows * 31 + n + count)
    w = rng.integers(-128, 128, rows * n, dtype=np.int8)  # -128 included, as the reference's tests draw them
    ws = (np.abs(rng.standard_normal(rows * n // 32)) * (0.02 / 127)).astype(F)
    q, s = quantized(oracle, rng, count, n)
    buf, frame = frames(q, s, n)
    got = run_tol(L, arena, w, ws, buf, frame, n, r0, r1, count, rows)
    want = reference(oracle, w, ws, q, s, n)
    ok, msg = within(got[:, r0:r1], want[:, r0:r1])
    assert ok, f"{rows}x{n}, {count} tokens: {msg}"
    assert np.all(got[:, :r0] == SENTINEL) and np.all(got[:, r1:] == SENTINEL), "rows outside r0..r1 written"


def test_exact_where_every_order_is_exact(L, arena, oracle):
    """scales powers of two (2^-8 .. 2^-10 for the rows, 2^-5 .. 2^-6 for the tokens) and weights in [-8, 7]: every
    term f(ws xs) d is exact and every partial sum of a row's 64 groups stays below 2^24 units of the smallest
    scale, so every float32 order gives the same number; the tolerance tile must give the reference's to the bit
    (a wrong integer, scale or token cannot hide here)"""
    rng = np.random.default_rng(9)
    rows, n, count = 200, 2048, 150
    ng = n // 32
    w = rng.integers(-8, 8, rows * n, dtype=np.int8)
    ws = np.ldexp(np.ones(rows * ng, F), -(8 + rng.integers(0, 3, rows * ng))).astype(F)
    q = rng.integers(0, 128, (count, n)).astype(np.uint8)
    s = np.ldexp(np.ones((count, ng), F), -(5 + rng.integers(0, 2, (count, ng)))).astype(F)
    buf, frame = frames(q, s, n)
    got = run_tol(L, arena, w, ws, buf, frame, n, 0, rows, count, rows)
    want = reference(oracle, w, ws, q, s, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{int(np.sum(got != want))} outputs differ; first {got[got != want][:3]} vs {want[got != want][:3]}"


def test_relaxed_bytes_outside_0_127_are_signed(pkg, L, arena):
    """activation bytes 128..255 (outside the reference's relaxed domain, where its relaxed dot is machine-dependent)
    are taken as signed int8, as the bit-exact tile takes them: with exact scales the two tiles agree to the bit"""
    rng = np.random.default_rng(10)
    rows, n, count = 64, 512, 40
    ng = n // 32
    w = rng.integers(-8, 8, rows * n, dtype=np.int8)
    ws = np.full(rows * ng, 2.0 ** -9, F)
    q = rng.integers(0, 256, (count, n)).astype(np.uint8)
    s = np.full((count, ng), 2.0 ** -6, F)
    buf, frame = frames(q, s, n)
    got = run_tol(L, arena, w, ws, buf, frame, n, 0, rows, count, rows)
    wq, wsa, xq = arena.put(w), arena.put(ws), arena.put(buf)
    exact = arena.alloc(4 * rows * count)
    pkg.load_kernels().matmul_q8r_tile(exact, xq, xq + n, wq, wsa, 0, n, 0, rows, count, 4 * rows, frame)
    want = arena.get(exact, F, rows * count).reshape(count, rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name,rows,n,count", [("1B qkv", 3072, 2048, 512), ("1B down", 2048, 8192, 512),
                                               ("8B gate", 14336, 4096, 2048), ("8B down", 4096, 14336, 2048)])
def test_full_prompt_shapes(pkg, L, arena, oracle, name, rows, n, count):
    """configs 2 and 3 at full size: every output against the bit-exact tile (the reference's number), and a sample
    of tokens against the oracle"""
    k = pkg.load_kernels()
    rng = np.random.default_rng(rows + n)
    w = rng.integers(-127, 128, rows * n, dtype=np.int8)
    ws = (np.abs(rng.standard_normal(rows * n // 32)) * (0.02 / 127)).astype(F)
    q, s = quantized(oracle, rng, count, n)
    buf, frame = frames(q, s, n)
    got = run_tol(L, arena, w, ws, buf, frame, n, 0, rows, count, rows)
    wq, wsa, xq = arena.put(w), arena.put(ws), arena.put(buf)
    exact = arena.alloc(4 * rows * count)
    k.matmul_q8r_tile(exact, xq, xq + n, wq, wsa, 0, n, 0, rows, count, 4 * rows, frame)
    want = arena.get(exact, F, rows * count).reshape(count, rows)
    ok, msg = within(got, want)
    assert ok, f"{name}: {msg}"
    wc = oracle.int8_sums(w)
    for t in (0, 1, count // 2, count - 1):
        assert np.array_equal(want[t].view(np.uint32), oracle.matmul_q8r(q[t], s[t], w, ws, wc, n).view(np.uint32))


def test_small_launches_take_the_bit_exact_tile(L, arena, oracle):
    """under the default setting a launch of fewer tolerance tiles than two blocks a compute unit runs the bit-exact
    kernels: its outputs are hq_matmul_q8r_tile_ex's (corrections derived) to the bit, and the reference's; with
    every launch given the tile, the same call is within the tolerance"""
    import torch
    rng = np.random.default_rng(5150)
    rows, n, count = 300, 1024, 40  # 3 tiles
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    ws = (np.abs(rng.standard_normal(rows * (n // 32))) * 0.02 / 127).astype(F)
    q, s = quantized(oracle, rng, count, n)
    buf, frame = frames(q, s, n)
    want = reference(oracle, w, ws, q, s, n)
    assert L.hq_tol_min_tiles(-1) == 0
    got = run_tol(L, arena, w, ws, buf, frame, n, 0, rows, count, rows)
    assert np.array_equal(got.view(np.uint32), want.astype(F).view(np.uint32))
    # the bit-exact tile's own call on the same inputs
    wq, wsa, xq = arena.put(w), arena.put(ws), arena.put(buf)
    out = arena.alloc(4 * rows * count, fill=np.full(rows * count, SENTINEL, F))
    assert L.hq_matmul_q8r_tile_ex(out, xq, xq + n, wq, wsa, None, n, 0, rows, count, 4 * rows, frame, None) == 0
    exact = arena.get(out, F, rows * count).reshape(count, rows)
    assert np.array_equal(got.view(np.uint32), exact.view(np.uint32))
    L.hq_tol_min_tiles(0)
    forced = run_tol(L, arena, w, ws, buf, frame, n, 0, rows, count, rows)
    ok, msg = within(forced, want)
    assert ok, msg
